// Causal GQA attention of packed prompts (prefill) on MFMA.
//
// The prompts of a prefill batch are packed into one token stream with no
// padding: token rows q [T, Hq * D], k [T, Hkv * D], v [T, Hkv * D] (row
// strides in elements, so v can be a column slice of the fused QKV rows).
// A work item is a 64-token query block of one prompt: its tokens
// [b0, b0 + 64) attend causally to the prompt's tokens [s, min(b0 + 64, e)),
// where [s, e) is the prompt's token range.  The host lists the blocks
// (block start, prompt start, prompt end), heaviest first.
//
// One workgroup of four wavefronts per (block, kv head, group of QH query
// heads of that kv head); wavefront w serves the block's 16-token tile
// [b0 + 16 w, +16) for the QH heads.  Each 32-token K/V chunk is loaded once
// for the workgroup (whole rows, 16 bytes per thread) into one of two LDS
// buffers while the previous chunk is computed, so a chunk's bytes serve 64
// query tokens x QH heads instead of the 16 x QH of a wavefront alone.
//   scores  v_mfma_f32_16x16x32 with the K chunk (16 tokens x 32 dims per
//           tile, read from LDS in the A-operand layout) and the head's
//           query tile as the B operand: lane (l16, q4), register r holds
//           S[key token t0 + 16 j + 4 q4 + r][query token i0 + l16], so the
//           online softmax of a query token is lane-local across q4 lanes;
//   P.V     P converted to the storage type is already the B operand; V^T
//           (A operand) is read from the chunk staged token-major with
//           ds_read_b64_tr_b16, once per chunk for all QH heads.
// Softmax in base 2 with a lazily raised running maximum (raised only when a
// score exceeds it by more than 2^8), fp32 accumulation, one rounding of the
// output.

// Reference semantics: the causal scaled-dot-product attention of prefill,
// tensorforge/runtime/prefill.py:84-88 (causal mask over the padded
// prompts) and :109-118 (torch SDPA with enable_gqa), here without padding.
#include <type_traits>

#include "tf_common.hpp"

namespace tf {
namespace {

constexpr float kPrefillLog2e = 1.4426950408889634f;
constexpr float kPrefillNegInf = -__builtin_huge_valf();
constexpr float kPrefillRescale = 8.f;
constexpr int kPrefillTile = 16;   // query tokens per wavefront
constexpr int kPrefillWaves = 4;   // wavefronts per workgroup
constexpr int kPrefillBlock = kPrefillTile * kPrefillWaves;  // query tokens per work item
constexpr int kPrefillChunk = 32;  // key tokens per step

template <typename T>
struct PrefillMfma;

template <>
struct PrefillMfma<__bf16> {
  typedef __bf16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct PrefillMfma<_Float16> {
  typedef _Float16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

typedef short pf_i16x4 __attribute__((ext_vector_type(4)));
typedef short pf_i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) pf_i16x4 pf_lds_i16x4;

struct PrefillParams {
  const void *q;
  const void *k;
  const void *v;
  void *out;
  const int32_t *tiles;  // [ntiles][3]: query start, prompt start, prompt end
  int64_t q_stride;
  int64_t k_stride;
  int64_t v_stride;
  int64_t out_stride;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t group;
  float scale_log2;
};

template <int D>
constexpr int prefill_row_bytes() { return D * 2 + 16; }

template <typename T, int D, int QH>
__global__ void __launch_bounds__(64 * kPrefillWaves)
prefill_attention_kernel(PrefillParams p) {
  using M = PrefillMfma<T>;
  using vec8 = typename M::vec8;
  constexpr int KS = D / 32;
  constexpr int NB = D / 16;
  constexpr int kRow = prefill_row_bytes<D>();  // V rows (padded for the transpose reads)
  // K rows are 2 D bytes with their 16-byte pieces permuted: piece p of row r
  // sits at p ^ ((r / R) % P), P = D / 8 pieces per row, R = 128 / D rows
  // per 256 bytes (1 at D 128), so the 16 lanes of an A-operand read (rows
  // 16 j .. +15, one piece each) and the 16 threads of a staging store
  // cover the 64 banks once.
  constexpr int kPieces = D / 8;
  constexpr int kRowsPer256 = D >= 128 ? 1 : 128 / D;
  constexpr int kRowK = 2 * D;
  __shared__ __attribute__((aligned(16))) unsigned char k_lds[2][kPrefillChunk * kRowK];
  __shared__ __attribute__((aligned(16))) unsigned char v_lds[2][kPrefillChunk * kRow];
  auto k_offset = [](int row, int piece) {
    return row * kRowK + 16 * (piece ^ ((row / kRowsPer256) & (kPieces - 1)));
  };

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int32_t *tile = p.tiles + 3 * static_cast<int64_t>(blockIdx.x);
  const int32_t b0 = tile[0];
  const int32_t s = tile[1];
  const int32_t e = tile[2];
  const int32_t groups = p.group / QH;
  const int32_t kvh = blockIdx.y / groups;
  const int32_t h0 = kvh * p.group + (blockIdx.y - kvh * groups) * QH;
  // Keys of the block [s, kend_blk); this wavefront's tile [i0, i0 + 16)
  // needs [s, kend) (none when the tile starts past the prompt).
  const int32_t kend_blk = min(b0 + kPrefillBlock, e);
  const int32_t i0 = b0 + kPrefillTile * wave;
  const int32_t kend = min(i0 + kPrefillTile, e);
  const int32_t qt = i0 + l16;  // this lane's query token (column)
  const bool q_ok = qt < e;

  const T *qbase = static_cast<const T *>(p.q);
  const T *kbase = static_cast<const T *>(p.k) + static_cast<int64_t>(kvh) * D;
  const T *vbase = static_cast<const T *>(p.v) + static_cast<int64_t>(kvh) * D;

  vec8 qf[QH][KS];  // B operand: q[token i0 + l16][head h0 + hq][32 ks + 8 q4 .. +8]
  {
    const T *qrow = qbase + static_cast<int64_t>(q_ok ? qt : s) * p.q_stride;
#pragma unroll
    for (int hq = 0; hq < QH; ++hq)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[hq][ks] = q_ok ? *reinterpret_cast<const vec8 *>(qrow + static_cast<int64_t>(h0 + hq) * D +
                                                            32 * ks + 8 * q4)
                          : vec8{};
  }

  f32x4 acc[QH][NB];
  float m_run[QH], l_run[QH];
#pragma unroll
  for (int hq = 0; hq < QH; ++hq) {
    m_run[hq] = kPrefillNegInf;
    l_run[hq] = 0.f;
#pragma unroll
    for (int n = 0; n < NB; ++n) acc[hq][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int32_t nch = (kend_blk - s + kPrefillChunk - 1) / kPrefillChunk;
  const int32_t my_nch = i0 < e ? (kend - s + kPrefillChunk - 1) / kPrefillChunk : 0;

  // Staging: the workgroup loads a chunk's K and V rows whole (D / 8
  // threads of 16 bytes per row) into one of two register sets, two chunks
  // ahead of the one being computed, and stores them token-major into the
  // chunk's buffer.  Rows past the block's keys read the prompt's first
  // row: their V rows are stored as zeros (0 * p), their scores are masked.
  constexpr int kLanesPerRow = D / 8;
  constexpr int kRowsPerPass = 64 * kPrefillWaves / kLanesPerRow;
  constexpr int kPasses = (kPrefillChunk + kRowsPerPass - 1) / kRowsPerPass;
  const int srow = tid / kLanesPerRow;
  const int spiece = tid - srow * kLanesPerRow;
  vec8 kreg[2][kPasses], vreg[2][kPasses];  // register set c % 2 holds chunk c
  // (the set is a compile-time index: the chunk loop is unrolled by two, so
  // the sets stay in registers)
  auto gload = [&](int32_t c, auto set_tag) {
    constexpr int set = decltype(set_tag)::value;
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int row = srow + kRowsPerPass * ps;
      const int32_t t = s + kPrefillChunk * c + row;
      const int32_t src = (row < kPrefillChunk && t < kend_blk) ? t : s;
      kreg[set][ps] = *reinterpret_cast<const vec8 *>(kbase + static_cast<int64_t>(src) * p.k_stride + 8 * spiece);
      vreg[set][ps] = *reinterpret_cast<const vec8 *>(vbase + static_cast<int64_t>(src) * p.v_stride + 8 * spiece);
    }
  };
  auto lstore = [&](int32_t c, auto set_tag) {
    constexpr int set = decltype(set_tag)::value;
    unsigned char *kdst = k_lds[set];
    unsigned char *vdst = v_lds[set];
    const bool tail = s + kPrefillChunk * (c + 1) > kend_blk;  // uniform
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int row = srow + kRowsPerPass * ps;
      if (row < kPrefillChunk) {
        *reinterpret_cast<vec8 *>(kdst + k_offset(row, spiece)) = kreg[set][ps];
        vec8 v = vreg[set][ps];
        if (tail && s + kPrefillChunk * c + row >= kend_blk) v = vec8{};
        *reinterpret_cast<vec8 *>(vdst + row * kRow + 16 * spiece) = v;
      }
    }
  };

  auto compute = [&](int32_t c, int buf) {
    const int32_t t0 = s + kPrefillChunk * c;
    const unsigned char *kb = k_lds[buf];
    const unsigned char *vb = v_lds[buf];
    // K in the A-operand layout: lane (l16, q4) of tile j holds token
    // t0 + 16 j + l16, dims [32 ks + 8 q4, +8).
    vec8 kf[2][KS];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kf[j][ks] = *reinterpret_cast<const vec8 *>(kb + k_offset(16 * j + l16, 4 * ks + q4));
    // V^T once for all heads.
    vec8 vtf[NB];
    {
      const unsigned char *rd = vb + (4 * q4 + (l16 >> 2)) * kRow + (l16 & 3) * 8;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const pf_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4 *)(rd + 32 * n));
        const pf_i16x4 hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4 *)(rd + 16 * kRow + 32 * n));
        vtf[n] = __builtin_bit_cast(vec8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
    // Causal mask: needed when some key token of the chunk lies past the
    // tile's first query token or past the tile's keys.
    const bool masked = t0 + kPrefillChunk > kend || t0 + kPrefillChunk - 1 > i0;
#pragma unroll
    for (int hq = 0; hq < QH; ++hq) {
      float sc[8];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f32x4 acc_s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc_s = M::mma(kf[j][ks], qf[hq][ks], acc_s);
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[4 * j + r] = acc_s[r];
      }
      if (masked) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int32_t kt = t0 + 16 * j + 4 * q4 + r;
            if (kt >= kend || kt > qt) sc[4 * j + r] = kPrefillNegInf;
          }
      }
      float mx = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                       fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
      mx *= p.scale_log2;
      if (__ballot(mx > m_run[hq] + kPrefillRescale) != 0) {
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run[hq], mx);
        // A column whose keys are all masked so far keeps m = -inf.
        const float alpha = m_new == kPrefillNegInf ? 1.f : __builtin_amdgcn_exp2f(m_run[hq] - m_new);
        m_run[hq] = m_new;
        l_run[hq] *= alpha;
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[hq][n] *= alpha;
      }
      // m_run is finite here: every query column sees its prompt's first
      // key (token s <= the query) in chunk 0, whose scores raise it from
      // -inf; masked scores give weights exp2(-inf) = 0.
      vec8 pf;
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], p.scale_log2, -m_run[hq]));
        psum += pr;
        pf[i] = static_cast<T>(pr);
      }
      l_run[hq] += psum;
#pragma unroll
      for (int n = 0; n < NB; ++n) acc[hq][n] = M::mma(vtf[n], pf, acc[hq][n]);
    }
  };

  // Chunk c is computed from buffer c % 2 while the loads of chunks c + 1
  // and c + 2 are in flight; after it, chunk c + 1 is stored into the other
  // buffer (last read for chunk c - 1, before the previous barrier) and the
  // loads of c + 3 are issued into the register set c + 1 freed.  One
  // barrier per chunk publishes the stored buffer and retires the one just
  // read.
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  gload(0, Set0{});
  if (nch > 1) gload(1, Set1{});
  lstore(0, Set0{});
  if (nch > 2) gload(2, Set0{});
  __syncthreads();
  for (int32_t c = 0; c < nch; c += 2) {
    // even chunk c: buffer and register set 0; then chunk c + 1 (set 1)
    if (c < my_nch) compute(c, 0);  // wavefront-uniform
    if (c + 1 < nch) {
      lstore(c + 1, Set1{});
      if (c + 3 < nch) gload(c + 3, Set1{});
    }
    __syncthreads();
    if (c + 1 >= nch) break;
    if (c + 1 < my_nch) compute(c + 1, 1);
    if (c + 2 < nch) {
      lstore(c + 2, Set0{});
      if (c + 4 < nch) gload(c + 4, Set0{});
    }
    __syncthreads();
  }

  // Lane-partial sums -> per-column sums; write the query tokens of the prompt.
  if (!q_ok) return;
  T *orow = static_cast<T *>(p.out) + static_cast<int64_t>(qt) * p.out_stride;
  typedef T t4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int hq = 0; hq < QH; ++hq) {
    float l = l_run[hq];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    T *dst = orow + static_cast<int64_t>(h0 + hq) * D;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const t4 o = {from_float<T>(acc[hq][n][0] * inv), from_float<T>(acc[hq][n][1] * inv),
                    from_float<T>(acc[hq][n][2] * inv), from_float<T>(acc[hq][n][3] * inv)};
      *reinterpret_cast<t4 *>(dst + 16 * n + 4 * q4) = o;
    }
  }
}

template <typename T, int D, int QH>
void launch_prefill(const PrefillParams &p, int32_t ntiles, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ntiles),
                  static_cast<unsigned>(p.kv_heads * (p.group / QH)));
  hipLaunchKernelGGL((prefill_attention_kernel<T, D, QH>), grid, dim3(64 * kPrefillWaves), 0,
                     stream, p);
}

template <typename T, int D>
void launch_prefill_qh(const PrefillParams &p, int32_t ntiles, int32_t heads_per_wave,
                       hipStream_t stream) {
  // Query heads per wavefront (a power of two dividing the group): as asked,
  // else 2 at head_dim >= 64 and 1 at 32 (measured best on MI355X over a
  // cfg5 batch of 19 prompts, 8,058 tokens: 97.5 / 102.1 / 111.8 us for 2 /
  // 1 / 4 at D 64, 165 / 165 / 199 at D 128, 39.8 / 47.0 for 1 / 2 at D 32);
  // at most 4 at head_dim 128, for registers.
  constexpr int kMax = D >= 128 ? 4 : 8;
  int32_t qh = heads_per_wave > 0 ? heads_per_wave : (D >= 64 ? 2 : 1);
  if (qh > kMax) qh = kMax;
  if (qh > p.group) qh = p.group;
  switch (qh) {
    case 1: launch_prefill<T, D, 1>(p, ntiles, stream); break;
    case 2: launch_prefill<T, D, 2>(p, ntiles, stream); break;
    case 4: launch_prefill<T, D, 4>(p, ntiles, stream); break;
    default:
      if constexpr (kMax >= 8) launch_prefill<T, D, 8>(p, ntiles, stream);
      break;
  }
}

template <typename T>
void launch_prefill_dim(const PrefillParams &p, int32_t head_dim, int32_t ntiles,
                        int32_t heads_per_wave, hipStream_t stream) {
  switch (head_dim) {
    case 32: launch_prefill_qh<T, 32>(p, ntiles, heads_per_wave, stream); break;
    case 64: launch_prefill_qh<T, 64>(p, ntiles, heads_per_wave, stream); break;
    default: launch_prefill_qh<T, 128>(p, ntiles, heads_per_wave, stream); break;
  }
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_prefill_attention(const void *q, int64_t q_row_stride, const void *k,
                                        int64_t k_row_stride, const void *v,
                                        int64_t v_row_stride, void *output,
                                        int64_t output_row_stride, const int32_t *tiles,
                                        int32_t num_tiles, int32_t query_heads, int32_t kv_heads,
                                        int32_t head_dim, float scale,
                                        int32_t heads_per_wave, int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (dtype != TF_DTYPE_FLOAT16 && dtype != TF_DTYPE_BFLOAT16)
    return fail(TF_ERROR_UNSUPPORTED, "prefill attention supports fp16 and bf16");
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(TF_ERROR_UNSUPPORTED, "prefill attention supports head_dim 32, 64 and 128");
  if (query_heads <= 0 || kv_heads <= 0 || query_heads % kv_heads != 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "query heads must be a positive multiple of kv heads");
  const int32_t group = query_heads / kv_heads;
  if (group > 16 || (group & (group - 1)) != 0)
    return fail(TF_ERROR_UNSUPPORTED, "prefill attention supports groups of 1, 2, 4, 8 or 16");
  if (heads_per_wave < 0 || heads_per_wave > 8 || (heads_per_wave & (heads_per_wave - 1)) != 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "heads_per_wave must be 0 or a power of two <= 8");
  if (num_tiles < 0 || num_tiles > 0x7fffffff / 3)
    return fail(TF_ERROR_INVALID_ARGUMENT, "invalid tile count");
  if (q_row_stride < static_cast<int64_t>(query_heads) * head_dim ||
      output_row_stride < static_cast<int64_t>(query_heads) * head_dim ||
      k_row_stride < static_cast<int64_t>(kv_heads) * head_dim ||
      v_row_stride < static_cast<int64_t>(kv_heads) * head_dim)
    return fail(TF_ERROR_INVALID_ARGUMENT, "row strides are shorter than the rows");
  if (num_tiles == 0) return TF_SUCCESS;
  if (!q || !k || !v || !output || !tiles)
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                          reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(output) |
                          static_cast<uintptr_t>(q_row_stride * 2) |
                          static_cast<uintptr_t>(k_row_stride * 2) |
                          static_cast<uintptr_t>(v_row_stride * 2) |
                          static_cast<uintptr_t>(output_row_stride * 2);
  if (align % 16 != 0)
    return fail(TF_ERROR_UNSUPPORTED, "prefill attention needs 16-byte aligned rows");
  if (static_cast<int64_t>(kv_heads) * group > 65535) return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  PrefillParams p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = output;
  p.tiles = tiles;
  p.q_stride = q_row_stride;
  p.k_stride = k_row_stride;
  p.v_stride = v_row_stride;
  p.out_stride = output_row_stride;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.group = group;
  p.scale_log2 = scale * kPrefillLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TF_DTYPE_BFLOAT16)
    launch_prefill_dim<__bf16>(p, head_dim, num_tiles, heads_per_wave, s);
  else
    launch_prefill_dim<_Float16>(p, head_dim, num_tiles, heads_per_wave, s);
  return check_launch("prefill_attention");
}
