// Paged GQA decode attention for gfx950.
//
// Work unit: one workgroup per (split, kv_head, sequence).  The workgroup
// serves the whole query group of its KV head, so every K/V page byte is read
// from HBM once per call (the reference launches one program per *query*
// head and re-reads each page group-size times,
// tensorforge/kernels/triton_attention.py:99-102,481).  Tokens are visited up
// to the sequence's own device-side length, not up to the host bucket
// (reference loops to the pow2 bucket, :121), and sequences of length <= 0
// produce zero rows without touching the cache.
//
// Two kernel families share one output/partial format:
//
//  * MFMA (bf16/fp16, head_dim in {32,64,128}, group <= 16).  Each wavefront
//    walks 32-token chunks of its split.  Scores S^T[token, head] come from
//    v_mfma_f32_16x16x32 with the K tile loaded straight from HBM as the A
//    operand (lane = token row, 8 contiguous head_dim elements = one 16-byte
//    load) and the query group as the B operand (heads padded to 16 columns
//    with zeros).  The online softmax runs on the accumulator layout, where
//    a lane owns one head, so the running max/sum and the rescale of the
//    output accumulator are lane-local.  P.V uses the same instruction with
//    V^T as the A operand: V is staged in a per-wavefront LDS tile
//    transposed to [head_dim][token] so each lane reads its 4+4 tokens of one
//    dimension with two 8-byte LDS reads; P (converted to the storage type)
//    is already in the B-operand layout.  K/V for the next chunk are loaded
//    before the current chunk is computed (two chunks in flight per wave).
//    Wavefronts of a workgroup merge their (max, sum, acc) states in LDS.
//
//  * Generic (any dtype, head_dim <= 256, group <= 64, any page size).  A
//    straightforward LDS-tiled implementation kept for fp32 and unusual
//    shapes; it is the accuracy reference path on the GPU (fp32 math
//    throughout).
//
// Softmax runs in base 2: scores are multiplied by scale*log2(e) and
// exponentiated with exp2, which is the native v_exp_f32.  Partial maxima are
// therefore base-2 values; only tf_paged_gqa_decode_merge reads them.
//
// Reference semantics:
//   one-pass kernel   triton_attention.py:67-171 (online softmax :116-161)
//   split kernel      triton_attention.py:173-266 (partials :260-266)
//   reduce kernel     triton_attention.py:268-316 (LSE merge :288-316)
//   oracle            kernels/reference.py:46-93
#include "tf_common.hpp"

namespace tf {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

struct AttnParams {
  const void *query;
  const void *key_cache;
  const void *value_cache;
  const int32_t *block_tables;
  const int32_t *context_lengths;
  void *output;
  float *partial_max;
  float *partial_sum;
  float *partial_acc;
  int32_t batch;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t group;
  int32_t head_dim;
  int32_t num_blocks;
  int32_t block_size;
  int32_t page_shift;  // log2(block_size) when a power of two, else -1
  int32_t table_width;
  int32_t split_size;
  int32_t num_splits;
  int32_t partial_stride;
  int32_t max_tokens;  // min(num_splits * split_size, table_width * block_size)
  float scale_log2;
};

__device__ __forceinline__ int32_t clamp_context(const AttnParams &p, int32_t b) {
  int32_t ctx = p.context_lengths[b];
  if (ctx < 0) ctx = 0;
  if (ctx > p.max_tokens) ctx = p.max_tokens;
  return ctx;
}

// Element offset of token `t` of sequence row `table` for kv head 0, or -1
// when the token's page entry is outside the cache.
__device__ __forceinline__ int64_t token_offset(const AttnParams &p, const int32_t *table,
                                                int32_t t) {
  int32_t logical, offset;
  if (p.page_shift >= 0) {
    logical = t >> p.page_shift;
    offset = t & (p.block_size - 1);
  } else {
    logical = t / p.block_size;
    offset = t - logical * p.block_size;
  }
  const int32_t page = table[logical];
  if (page < 0 || page >= p.num_blocks) return -1;
  return (static_cast<int64_t>(page) * p.block_size + offset) *
         static_cast<int64_t>(p.kv_heads) * p.head_dim;
}

// Write the finished (max, sum, numerator) of one (row, query head) either
// as the final output (one split) or as a partial.
template <typename T>
__device__ __forceinline__ void store_result(const AttnParams &p, int32_t b, int32_t qh,
                                             int32_t split, int32_t d, float m, float l,
                                             float num) {
  if (p.num_splits == 1) {
    const float o = l > 0.f ? num / l : 0.f;
    static_cast<T *>(p.output)[(static_cast<int64_t>(b) * p.query_heads + qh) * p.head_dim + d] =
        from_float<T>(o);
  } else {
    const int64_t row = (static_cast<int64_t>(b) * p.query_heads + qh) * p.num_splits + split;
    p.partial_acc[row * p.partial_stride + d] = num;
    if (d == 0) {
      p.partial_max[row] = m;
      p.partial_sum[row] = l;
    }
  }
}

// Rows of length zero get zeros in one-pass mode (the merge kernel handles
// them in split mode).
template <typename T>
__device__ void zero_rows(const AttnParams &p, int32_t b, int32_t kvh) {
  if (p.num_splits != 1) return;
  T *out = static_cast<T *>(p.output) +
           (static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(kvh) * p.group) *
               p.head_dim;
  for (int i = threadIdx.x; i < p.group * p.head_dim; i += blockDim.x) out[i] = from_float<T>(0.f);
}

// ===========================================================================
// MFMA kernel
// ===========================================================================
template <typename T>
struct Mfma;

template <>
struct Mfma<__bf16> {
  typedef __bf16 vec8 __attribute__((ext_vector_type(8)));
  typedef __bf16 vec4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<_Float16> {
  typedef _Float16 vec8 __attribute__((ext_vector_type(8)));
  typedef _Float16 vec4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kChunk = 32;             // tokens per wavefront step (two 16-row tiles)
constexpr int kVtStride = kChunk + 4;  // LDS row of the transposed V tile (elements)

template <int D, int NW>
constexpr int mfma_lds_bytes() {
  // max(transposed V tiles, cross-wave merge buffers for 16 heads)
  return (NW * D * kVtStride * 2) > (NW * (16 * D + 32) * 4) ? (NW * D * kVtStride * 2)
                                                             : (NW * (16 * D + 32) * 4);
}

template <typename T, int D, int NW, bool UNIFORM_PAGE>
__global__ void __launch_bounds__(NW * 64)
paged_decode_mfma_kernel(AttnParams p) {
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  using vec4 = typename M::vec4;
  constexpr int KS = D / 32;  // k-steps of the score product
  constexpr int NB = D / 16;  // 16-dim blocks of the output
  __shared__ __attribute__((aligned(16))) unsigned char lds[mfma_lds_bytes<D, NW>()];

  const int32_t split = blockIdx.x;
  const int32_t kvh = blockIdx.y;
  const int32_t b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15;
  const int q4 = lane >> 4;

  const int32_t ctx = clamp_context(p, b);
  const int32_t s0 = split * p.split_size;
  if (s0 >= ctx) {
    if (split == 0) zero_rows<T>(p, b, kvh);
    return;
  }
  const int32_t s1 = min(s0 + p.split_size, ctx);
  const int32_t nchunks = (s1 - s0 + kChunk - 1) / kChunk;

  // Query group as the B operand: lane holds q[head l16][32ks + 8q4 .. +8].
  vec8 qf[KS];
  {
    const T *qrow = static_cast<const T *>(p.query) +
                    (static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(kvh) * p.group +
                     l16) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (l16 < p.group)
        qf[ks] = *reinterpret_cast<const vec8 *>(qrow + 32 * ks + 8 * q4);
      else
        qf[ks] = vec8{};
    }
  }

  const int32_t *table = p.block_tables + static_cast<int64_t>(b) * p.table_width;
  const int64_t token_stride = static_cast<int64_t>(p.kv_heads) * D;
  const T *kbase = static_cast<const T *>(p.key_cache) + static_cast<int64_t>(kvh) * D + 8 * q4;
  const T *vbase = static_cast<const T *>(p.value_cache) + static_cast<int64_t>(kvh) * D + 8 * q4;

  // Physical page of tile j of chunk c.  With UNIFORM_PAGE (block_size a
  // multiple of 16, so a 16-token tile never straddles pages) the page is
  // wave-uniform and the table read is a scalar load; otherwise each lane
  // reads the entry of its own token.
  auto fetch_pages = [&](int32_t c, int32_t(&pg)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int32_t t = s0 + c * kChunk + 16 * j + (UNIFORM_PAGE ? 0 : l16);
      pg[j] = -1;
      if (t < s1) {
        const int32_t logical = p.page_shift >= 0 ? (t >> p.page_shift) : (t / p.block_size);
        pg[j] = table[logical];
      }
    }
  };

  // Issue the K/V loads of chunk c: lane covers token row l16 of tiles 0/1
  // and head_dim elements [32ks + 8q4, +8).  Absent tokens load from the
  // always-valid element 0 of the cache and are masked later, so every load
  // is unconditional.  `valid` bit t of tile j marks token 16j + t present.
  auto load_kv = [&](int32_t c, const int32_t(&pg)[2], vec8(&kf)[2][KS], vec8(&vf)[2][KS],
                     uint32_t(&valid)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int32_t t = s0 + c * kChunk + 16 * j + l16;
      const int32_t page = pg[j];
      const bool ok = t < s1 && page >= 0 && page < p.num_blocks;
      int32_t offset;
      if (p.page_shift >= 0)
        offset = t & (p.block_size - 1);
      else
        offset = t - (t / p.block_size) * p.block_size;
      int64_t off = (static_cast<int64_t>(page) * p.block_size + offset) * token_stride;
      if (!ok) off = -static_cast<int64_t>(kvh) * D - 8 * q4;
      valid[j] = static_cast<uint32_t>(__ballot(ok) & 0xffffull);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[j][ks] = *reinterpret_cast<const vec8 *>(kbase + off + 32 * ks);
        vf[j][ks] = *reinterpret_cast<const vec8 *>(vbase + off + 32 * ks);
      }
    }
  };

  f32x4 acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;  // running max of head l16 (base 2)
  float l_run = 0.f;      // lane-partial running sum of head l16

  T *vt = reinterpret_cast<T *>(lds) + wave * D * kVtStride;

  auto compute = [&](vec8(&kf)[2][KS], vec8(&vf)[2][KS], const uint32_t(&valid)[2]) {
    // Scores: lane holds S[token 16j + 4q4 + r][head l16].
    float sc[8];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s = M::mma(kf[j][ks], qf[ks], s);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = (valid[j] >> (4 * q4 + r)) & 1u;
        sc[4 * j + r] = ok ? s[r] * p.scale_log2 : kNegInf;
      }
    }
    float mx = sc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sc[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (mx == kNegInf) return;  // uniform: no token of the chunk is present
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    vec8 pf;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pr = exp2f(sc[i] - m_new);
      psum += pr;
      pf[i] = static_cast<T>(pr);
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int n = 0; n < NB; ++n) acc[n] *= alpha;

    // Absent tokens carry p = 0 but their V rows were loaded from a stand-in
    // address; clear them so 0 * (non-finite) cannot leak in.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (valid[j] != 0xffffu && !((valid[j] >> l16) & 1u)) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) vf[j][ks] = vec8{};
      }
    }
    // Stage V^T[dim][token] for this chunk in the wave's LDS tile.  LDS
    // requests of one wavefront are served in order, so the compiler
    // barriers below are the only ordering needed.
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          vt[(32 * ks + 8 * q4 + e) * kVtStride + 16 * j + l16] = vf[j][ks][e];
    __asm__ volatile("" ::: "memory");
    // P.V: A = V^T (row = dim 16n + l16, k = 8q4 + i -> token 4q4+i of tile
    // 0 for i < 4, of tile 1 for i >= 4); B = P in the same k order.
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const T *row = vt + (16 * n + l16) * kVtStride + 4 * q4;
      const vec4 lo = *reinterpret_cast<const vec4 *>(row);
      const vec4 hi = *reinterpret_cast<const vec4 *>(row + 16);
      const vec8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[n] = M::mma(a, pf, acc[n]);
    }
    __asm__ volatile("" ::: "memory");
  };

  // Two register sets alternate so a chunk's K/V stay in flight while the
  // previous one is computed; page ids run one chunk further ahead.
  vec8 ka[2][KS], va[2][KS], kb[2][KS], vb[2][KS];
  uint32_t vala[2] = {0u, 0u}, valb[2] = {0u, 0u};
  int32_t pa[2] = {-1, -1}, pb[2] = {-1, -1};
  int32_t c = wave;
  if (c < nchunks) {
    fetch_pages(c, pa);
    if (c + NW < nchunks) fetch_pages(c + NW, pb);
    load_kv(c, pa, ka, va, vala);
  }
  while (c < nchunks) {
    if (c + 2 * NW < nchunks) fetch_pages(c + 2 * NW, pa);
    if (c + NW < nchunks) load_kv(c + NW, pb, kb, vb, valb);
    compute(ka, va, vala);
    c += NW;
    if (c >= nchunks) break;
    if (c + 2 * NW < nchunks) fetch_pages(c + 2 * NW, pb);
    if (c + NW < nchunks) load_kv(c + NW, pa, ka, va, vala);
    compute(kb, vb, valb);
    c += NW;
  }

  // Lane-partial sums -> per-head sums within the wave.
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  // Cross-wave merge through LDS (the V tiles are dead after the barrier).
  __syncthreads();
  float *red_ml = reinterpret_cast<float *>(lds);  // [NW][2][16]
  float *red_acc = red_ml + NW * 32;               // [NW][16][D]
  if (q4 == 0) {
    red_ml[wave * 32 + l16] = m_run;
    red_ml[wave * 32 + 16 + l16] = l_run;
  }
#pragma unroll
  for (int n = 0; n < NB; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) red_acc[(wave * 16 + l16) * D + 16 * n + 4 * q4 + r] = acc[n][r];
  __syncthreads();

  for (int idx = threadIdx.x; idx < p.group * D; idx += NW * 64) {
    const int g = idx / D;
    const int d = idx - g * D;
    float mmax = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) mmax = fmaxf(mmax, red_ml[w * 32 + g]);
    float num = 0.f, den = 0.f;
    if (mmax != kNegInf) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float e = exp2f(red_ml[w * 32 + g] - mmax);
        den += red_ml[w * 32 + 16 + g] * e;
        num += red_acc[(w * 16 + g) * D + d] * e;
      }
    }
    store_result<T>(p, b, kvh * p.group + g, split, d, mmax, den, num);
  }
}

// ===========================================================================
// Generic kernel (fp32 math, LDS tiles)
// ===========================================================================
constexpr int kGenericThreads = 256;
constexpr int kGenericTile = 16;
constexpr int kGenericMaxAcc = 32;  // group * head_dim <= 256 * 32

template <typename T>
__global__ void __launch_bounds__(kGenericThreads)
paged_decode_generic_kernel(AttnParams p) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int D = p.head_dim;
  const int G = p.group;
  float *ks = smem;                            // [tile][D + 1]
  float *vs = ks + kGenericTile * (D + 1);     // [tile][D]
  float *sc = vs + kGenericTile * D;           // [G][tile]
  float *m_run = sc + G * kGenericTile;        // [G]
  float *l_run = m_run + G;                    // [G]
  float *alpha = l_run + G;                    // [G]
  int *tok_ok = reinterpret_cast<int *>(alpha + G);  // [tile]

  const int32_t split = blockIdx.x;
  const int32_t kvh = blockIdx.y;
  const int32_t b = blockIdx.z;
  const int32_t ctx = clamp_context(p, b);
  const int32_t s0 = split * p.split_size;
  if (s0 >= ctx) {
    if (split == 0) zero_rows<T>(p, b, kvh);
    return;
  }
  const int32_t s1 = min(s0 + p.split_size, ctx);
  const int32_t *table = p.block_tables + static_cast<int64_t>(b) * p.table_width;
  const T *q = static_cast<const T *>(p.query) +
               (static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(kvh) * G) * D;
  const T *kbase = static_cast<const T *>(p.key_cache) + static_cast<int64_t>(kvh) * D;
  const T *vbase = static_cast<const T *>(p.value_cache) + static_cast<int64_t>(kvh) * D;

  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    m_run[g] = kNegInf;
    l_run[g] = 0.f;
  }
  float acc[kGenericMaxAcc];
#pragma unroll
  for (int i = 0; i < kGenericMaxAcc; ++i) acc[i] = 0.f;

  for (int32_t t0 = s0; t0 < s1; t0 += kGenericTile) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < kGenericTile * D; idx += blockDim.x) {
      const int tt = idx / D;
      const int d = idx - tt * D;
      const int32_t t = t0 + tt;
      int64_t off = -1;
      if (t < s1) off = token_offset(p, table, t);
      float kv = 0.f, vv = 0.f;
      if (off >= 0) {
        kv = to_float(kbase[off + d]);
        vv = to_float(vbase[off + d]);
      }
      ks[tt * (D + 1) + d] = kv;
      vs[tt * D + d] = vv;
      if (d == 0) tok_ok[tt] = off >= 0;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * kGenericTile; idx += blockDim.x) {
      const int g = idx / kGenericTile;
      const int tt = idx - g * kGenericTile;
      float s = kNegInf;
      if (tok_ok[tt]) {
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot += to_float(q[g * D + d]) * ks[tt * (D + 1) + d];
        s = dot * p.scale_log2;
      }
      sc[idx] = s;
    }
    __syncthreads();
    for (int g = threadIdx.x; g < G; g += blockDim.x) {
      float mx = kNegInf;
      for (int tt = 0; tt < kGenericTile; ++tt) mx = fmaxf(mx, sc[g * kGenericTile + tt]);
      const float m_new = fmaxf(m_run[g], mx);
      float a = 1.f, sum = 0.f;
      if (m_new != kNegInf) {
        a = exp2f(m_run[g] - m_new);
        for (int tt = 0; tt < kGenericTile; ++tt) {
          const float pr = exp2f(sc[g * kGenericTile + tt] - m_new);
          sc[g * kGenericTile + tt] = pr;
          sum += pr;
        }
      } else {
        for (int tt = 0; tt < kGenericTile; ++tt) sc[g * kGenericTile + tt] = 0.f;
      }
      l_run[g] = l_run[g] * a + sum;
      m_run[g] = m_new;
      alpha[g] = a;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kGenericMaxAcc; ++i) {
      const int idx = threadIdx.x + i * kGenericThreads;
      if (idx < G * D) {
        const int g = idx / D;
        const int d = idx - g * D;
        float a = acc[i] * alpha[g];
        for (int tt = 0; tt < kGenericTile; ++tt) a += sc[g * kGenericTile + tt] * vs[tt * D + d];
        acc[i] = a;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kGenericMaxAcc; ++i) {
    const int idx = threadIdx.x + i * kGenericThreads;
    if (idx < G * D) {
      const int g = idx / D;
      const int d = idx - g * D;
      store_result<T>(p, b, kvh * G + g, split, d, m_run[g], l_run[g], acc[i]);
    }
  }
}

size_t generic_lds_bytes(int D, int G) {
  return sizeof(float) * (static_cast<size_t>(kGenericTile) * (D + 1) +
                          static_cast<size_t>(kGenericTile) * D + static_cast<size_t>(G) * kGenericTile +
                          3 * static_cast<size_t>(G) + kGenericTile);
}

// ===========================================================================
// Log-sum-exp merge of split partials
// ===========================================================================
template <typename T>
__global__ void __launch_bounds__(64)
merge_partials_kernel(const float *__restrict__ partial_max, const float *__restrict__ partial_sum,
                      const float *__restrict__ partial_acc,
                      const int32_t *__restrict__ context_lengths, T *__restrict__ output,
                      int32_t query_heads, int32_t head_dim, int32_t split_size,
                      int32_t num_splits, int32_t partial_stride, int32_t max_tokens) {
  const int32_t qh = blockIdx.x;
  const int32_t b = blockIdx.y;
  int32_t ctx = context_lengths[b];
  if (ctx < 0) ctx = 0;
  if (ctx > max_tokens) ctx = max_tokens;
  const int32_t nvalid = (ctx + split_size - 1) / split_size;
  const int64_t base = (static_cast<int64_t>(b) * query_heads + qh) * num_splits;
  T *out = output + (static_cast<int64_t>(b) * query_heads + qh) * head_dim;
  float gmax = kNegInf;
  for (int32_t s = 0; s < nvalid; ++s) gmax = fmaxf(gmax, partial_max[base + s]);
  float den = 0.f;
  if (gmax != kNegInf)
    for (int32_t s = 0; s < nvalid; ++s) den += partial_sum[base + s] * exp2f(partial_max[base + s] - gmax);
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    float num = 0.f;
    if (gmax != kNegInf)
      for (int32_t s = 0; s < nvalid; ++s)
        num += partial_acc[(base + s) * partial_stride + d] * exp2f(partial_max[base + s] - gmax);
    out[d] = from_float<T>(den > 0.f ? num / den : 0.f);
  }
}

// ===========================================================================
// Host side
// ===========================================================================
int32_t choose_variant(int32_t dtype, int32_t head_dim, int32_t group, int32_t flags) {
  if (flags & TF_ATTENTION_FLAG_FORCE_GENERIC) return TF_ATTENTION_GENERIC;
  if (dtype == TF_DTYPE_FLOAT32) return TF_ATTENTION_GENERIC;
  if (group > 16) return TF_ATTENTION_GENERIC;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return TF_ATTENTION_GENERIC;
  return TF_ATTENTION_MFMA;
}

constexpr int kMfmaWaves = 4;

template <typename T, int D>
void launch_mfma(const AttnParams &p, dim3 grid, hipStream_t stream) {
  // Whole-tile pages need 16-aligned tile starts: one pass starts at token 0,
  // split mode at multiples of split_size.
  const bool uniform = p.block_size % 16 == 0 && (p.num_splits == 1 || p.split_size % 16 == 0);
  if (uniform)
    hipLaunchKernelGGL((paged_decode_mfma_kernel<T, D, kMfmaWaves, true>), grid,
                       dim3(kMfmaWaves * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((paged_decode_mfma_kernel<T, D, kMfmaWaves, false>), grid,
                       dim3(kMfmaWaves * 64), 0, stream, p);
}

template <typename T>
void launch_mfma_dim(const AttnParams &p, dim3 grid, hipStream_t stream) {
  switch (p.head_dim) {
    case 32: launch_mfma<T, 32>(p, grid, stream); break;
    case 64: launch_mfma<T, 64>(p, grid, stream); break;
    default: launch_mfma<T, 128>(p, grid, stream); break;
  }
}

int32_t validate(const void *query, const void *key_cache, const void *value_cache,
                 const int32_t *block_tables, const int32_t *context_lengths, int32_t batch,
                 int32_t query_heads, int32_t kv_heads, int32_t head_dim, int32_t num_blocks,
                 int32_t block_size, int32_t table_width, int32_t split_size, int32_t num_splits,
                 int32_t dtype) {
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (batch < 0 || query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0 ||
      block_size <= 0 || table_width <= 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "attention dimensions must be positive");
  if (query_heads % kv_heads != 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "query heads must be a multiple of kv heads");
  if (head_dim > 256) return fail(TF_ERROR_INVALID_ARGUMENT, "head_dim must be <= 256");
  if (split_size <= 0 || num_splits <= 0 || num_splits > 65535)
    return fail(TF_ERROR_INVALID_ARGUMENT, "split_size and num_splits must be positive");
  if (batch > 65535 || kv_heads > 65535) return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  if (batch > 0 && (!query || !key_cache || !value_cache || !block_tables || !context_lengths))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  return TF_SUCCESS;
}

int32_t make_params(AttnParams &p, const void *query, const void *key_cache,
                    const void *value_cache, const int32_t *block_tables,
                    const int32_t *context_lengths, void *output, float *partial_max,
                    float *partial_sum, float *partial_acc, int64_t partial_capacity,
                    int32_t partial_row_stride, int32_t batch, int32_t query_heads,
                    int32_t kv_heads, int32_t head_dim, int32_t num_blocks, int32_t block_size,
                    int32_t table_width, int32_t split_size, int32_t num_splits, float scale,
                    int32_t dtype) {
  if (int32_t s = validate(query, key_cache, value_cache, block_tables, context_lengths, batch,
                           query_heads, kv_heads, head_dim, num_blocks, block_size, table_width,
                           split_size, num_splits, dtype))
    return s;
  if (num_splits > 1) {
    if (!partial_max || !partial_sum || !partial_acc)
      return fail(TF_ERROR_INVALID_ARGUMENT, "split attention needs partial buffers");
    if (partial_row_stride < head_dim)
      return fail(TF_ERROR_INVALID_ARGUMENT, "partial row stride is smaller than head_dim");
    if (partial_capacity < static_cast<int64_t>(batch) * query_heads * num_splits)
      return fail(TF_ERROR_INVALID_ARGUMENT, "partial buffers are too small");
  }
  p.query = query;
  p.key_cache = key_cache;
  p.value_cache = value_cache;
  p.block_tables = block_tables;
  p.context_lengths = context_lengths;
  p.output = output;
  p.partial_max = partial_max;
  p.partial_sum = partial_sum;
  p.partial_acc = partial_acc;
  p.batch = batch;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.group = query_heads / kv_heads;
  p.head_dim = head_dim;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.page_shift = -1;
  if ((block_size & (block_size - 1)) == 0) p.page_shift = __builtin_ctz(block_size);
  p.table_width = table_width;
  p.split_size = split_size;
  p.num_splits = num_splits;
  p.partial_stride = partial_row_stride;
  const int64_t split_tokens = static_cast<int64_t>(num_splits) * split_size;
  const int64_t table_tokens = static_cast<int64_t>(table_width) * block_size;
  int64_t max_tokens = split_tokens < table_tokens ? split_tokens : table_tokens;
  if (max_tokens > 0x7fffffff) max_tokens = 0x7fffffff;
  p.max_tokens = static_cast<int32_t>(max_tokens);
  p.scale_log2 = scale * kLog2e;
  return TF_SUCCESS;
}

int32_t launch_split_stage(const AttnParams &p, int32_t dtype, int32_t flags, hipStream_t stream) {
  if (p.batch == 0) return TF_SUCCESS;
  const dim3 grid(static_cast<unsigned>(p.num_splits), static_cast<unsigned>(p.kv_heads),
                  static_cast<unsigned>(p.batch));
  const int32_t variant = choose_variant(dtype, p.head_dim, p.group, flags);
  if (variant == TF_ATTENTION_MFMA) {
    if (dtype == TF_DTYPE_BFLOAT16)
      launch_mfma_dim<__bf16>(p, grid, stream);
    else
      launch_mfma_dim<_Float16>(p, grid, stream);
    return check_launch("paged_gqa_decode (mfma)");
  }
  if (p.group > 64 || p.group * p.head_dim > kGenericThreads * kGenericMaxAcc)
    return fail(TF_ERROR_UNSUPPORTED,
                "generic attention supports group <= 64 and group * head_dim <= 8192");
  const size_t lds = generic_lds_bytes(p.head_dim, p.group);
  switch (dtype) {
    case TF_DTYPE_FLOAT32:
      hipLaunchKernelGGL(paged_decode_generic_kernel<float>, grid, dim3(kGenericThreads), lds,
                         stream, p);
      break;
    case TF_DTYPE_FLOAT16:
      hipLaunchKernelGGL(paged_decode_generic_kernel<_Float16>, grid, dim3(kGenericThreads), lds,
                         stream, p);
      break;
    default:
      hipLaunchKernelGGL(paged_decode_generic_kernel<__bf16>, grid, dim3(kGenericThreads), lds,
                         stream, p);
      break;
  }
  return check_launch("paged_gqa_decode (generic)");
}

int32_t launch_merge(const float *partial_max, const float *partial_sum, const float *partial_acc,
                     const int32_t *context_lengths, void *output, int32_t batch,
                     int32_t query_heads, int32_t head_dim, int32_t split_size, int32_t num_splits,
                     int32_t partial_stride, int32_t max_tokens, int32_t dtype,
                     hipStream_t stream) {
  if (batch == 0) return TF_SUCCESS;
  const dim3 grid(static_cast<unsigned>(query_heads), static_cast<unsigned>(batch));
  switch (dtype) {
    case TF_DTYPE_FLOAT32:
      hipLaunchKernelGGL(merge_partials_kernel<float>, grid, dim3(64), 0, stream, partial_max,
                         partial_sum, partial_acc, context_lengths, static_cast<float *>(output),
                         query_heads, head_dim, split_size, num_splits, partial_stride, max_tokens);
      break;
    case TF_DTYPE_FLOAT16:
      hipLaunchKernelGGL(merge_partials_kernel<_Float16>, grid, dim3(64), 0, stream, partial_max,
                         partial_sum, partial_acc, context_lengths,
                         static_cast<_Float16 *>(output), query_heads, head_dim, split_size,
                         num_splits, partial_stride, max_tokens);
      break;
    default:
      hipLaunchKernelGGL(merge_partials_kernel<__bf16>, grid, dim3(64), 0, stream, partial_max,
                         partial_sum, partial_acc, context_lengths, static_cast<__bf16 *>(output),
                         query_heads, head_dim, split_size, num_splits, partial_stride, max_tokens);
      break;
  }
  return check_launch("paged_gqa_decode merge");
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_paged_gqa_decode_variant(int32_t dtype, int32_t head_dim, int32_t group_size,
                                               int32_t flags) {
  return tf::choose_variant(dtype, head_dim, group_size, flags);
}

extern "C" int32_t tf_paged_gqa_decode(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths, void *output,
    float *partial_max, float *partial_sum, float *partial_accumulator, int64_t partial_capacity,
    int32_t partial_row_stride, int32_t batch, int32_t query_heads, int32_t kv_heads,
    int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t table_width,
    int32_t split_size, int32_t num_splits, float scale, int32_t dtype, int32_t flags,
    void *stream) {
  using namespace tf;
  clear_error();
  if (batch > 0 && !output) return fail(TF_ERROR_INVALID_ARGUMENT, "null output pointer");
  AttnParams p;
  if (int32_t s = make_params(p, query, key_cache, value_cache, block_tables, context_lengths,
                              output, partial_max, partial_sum, partial_accumulator,
                              partial_capacity, partial_row_stride, batch, query_heads, kv_heads,
                              head_dim, num_blocks, block_size, table_width, split_size,
                              num_splits, scale, dtype))
    return s;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int32_t st = launch_split_stage(p, dtype, flags, s)) return st;
  if (num_splits == 1) return TF_SUCCESS;
  return launch_merge(partial_max, partial_sum, partial_accumulator, context_lengths, output,
                      batch, query_heads, head_dim, split_size, num_splits, partial_row_stride,
                      p.max_tokens, dtype, s);
}

extern "C" int32_t tf_paged_gqa_decode_partials(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths, float *partial_max,
    float *partial_sum, float *partial_accumulator, int64_t partial_capacity,
    int32_t partial_row_stride, int32_t batch, int32_t query_heads, int32_t kv_heads,
    int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t table_width,
    int32_t split_size, int32_t num_splits, float scale, int32_t dtype, int32_t flags,
    void *stream) {
  using namespace tf;
  clear_error();
  if (!partial_max || !partial_sum || !partial_accumulator)
    return fail(TF_ERROR_INVALID_ARGUMENT, "partials stage needs partial buffers");
  if (num_splits < 2) return fail(TF_ERROR_INVALID_ARGUMENT, "partials stage needs num_splits >= 2");
  AttnParams p;
  if (int32_t s = make_params(p, query, key_cache, value_cache, block_tables, context_lengths,
                              nullptr, partial_max, partial_sum, partial_accumulator,
                              partial_capacity, partial_row_stride, batch, query_heads, kv_heads,
                              head_dim, num_blocks, block_size, table_width, split_size,
                              num_splits, scale, dtype))
    return s;
  return launch_split_stage(p, dtype, flags, static_cast<hipStream_t>(stream));
}

extern "C" int32_t tf_paged_gqa_decode_merge(
    const float *partial_max, const float *partial_sum, const float *partial_accumulator,
    const int32_t *context_lengths, void *output, int64_t partial_capacity,
    int32_t partial_row_stride, int32_t batch, int32_t query_heads, int32_t head_dim,
    int32_t split_size, int32_t num_splits, int32_t max_tokens, int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (batch < 0 || query_heads <= 0 || head_dim <= 0 || head_dim > 256 || split_size <= 0 ||
      num_splits <= 0 || max_tokens < 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "merge dimensions out of range");
  if (batch > 65535 || query_heads > 65535) return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  if (partial_row_stride < head_dim)
    return fail(TF_ERROR_INVALID_ARGUMENT, "partial row stride is smaller than head_dim");
  if (partial_capacity < static_cast<int64_t>(batch) * query_heads * num_splits)
    return fail(TF_ERROR_INVALID_ARGUMENT, "partial buffers are too small");
  if (batch > 0 && (!partial_max || !partial_sum || !partial_accumulator || !context_lengths ||
                    !output))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const int64_t split_tokens = static_cast<int64_t>(num_splits) * split_size;
  const int32_t clamp =
      static_cast<int32_t>(split_tokens < max_tokens ? split_tokens : max_tokens);
  return launch_merge(partial_max, partial_sum, partial_accumulator, context_lengths, output,
                      batch, query_heads, head_dim, split_size, num_splits, partial_row_stride,
                      clamp, dtype, static_cast<hipStream_t>(stream));
}
