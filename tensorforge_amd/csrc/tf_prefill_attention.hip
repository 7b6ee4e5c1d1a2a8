// Causal GQA attention of packed prompts (prefill) on MFMA.
//
// The prompts of a prefill batch are packed into one token stream with no
// padding: token rows q [T, Hq * D], k [T, Hkv * D], v [T, Hkv * D] (row
// strides in elements, so v can be a column slice of the fused QKV rows).
// A work item is a 16-token query tile of one prompt: its tokens
// [i0, i0 + 16) attend causally to the prompt's tokens [s, min(i0 + 16, e)),
// where [s, e) is the prompt's token range.  The host lists the tiles
// (query start, prompt start, prompt end), heaviest first.
//
// One wavefront per (tile, kv head, group of QH query heads of that kv
// head): each 32-token K/V chunk is read once for its QH heads.
//   scores  v_mfma_f32_16x16x32 with the K chunk (16 tokens x 32 dims per
//           tile) as the A operand straight from memory and the head's
//           query tile as the B operand: lane (l16, q4), register r holds
//           S[key token t0 + 16 j + 4 q4 + r][query token i0 + l16], so the
//           online softmax of a query token is lane-local across q4 lanes;
//   P.V     P converted to the storage type is already the B operand; V^T
//           (A operand) is read from the chunk staged token-major in the
//           wavefront's LDS with ds_read_b64_tr_b16, once per chunk for all
//           QH heads.
// Softmax in base 2 with a lazily raised running maximum (raised only when a
// score exceeds it by more than 2^8), fp32 accumulation, one rounding of the
// output.  Two chunks of loads are in flight.
//
// Reference semantics: the causal scaled-dot-product attention of prefill,
// tensorforge/runtime/prefill.py:84-88 (causal mask over the padded
// prompts) and :109-118 (torch SDPA with enable_gqa), here without padding.
#include "tf_common.hpp"

namespace tf {
namespace {

constexpr float kPrefillLog2e = 1.4426950408889634f;
constexpr float kPrefillNegInf = -__builtin_huge_valf();
constexpr float kPrefillRescale = 8.f;
constexpr int kPrefillTile = 16;   // query tokens per work item
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
__global__ void __launch_bounds__(64)
prefill_attention_kernel(PrefillParams p) {
  using M = PrefillMfma<T>;
  using vec8 = typename M::vec8;
  constexpr int KS = D / 32;
  constexpr int NB = D / 16;
  constexpr int kRow = prefill_row_bytes<D>();
  __shared__ __attribute__((aligned(16))) unsigned char vt[kPrefillChunk * kRow];

  const int lane = threadIdx.x;
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int32_t *tile = p.tiles + 3 * static_cast<int64_t>(blockIdx.x);
  const int32_t i0 = tile[0];
  const int32_t s = tile[1];
  const int32_t e = tile[2];
  const int32_t groups = p.group / QH;
  const int32_t kvh = blockIdx.y / groups;
  const int32_t h0 = kvh * p.group + (blockIdx.y - kvh * groups) * QH;
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
  const int32_t nch = (kend - s + kPrefillChunk - 1) / kPrefillChunk;

  // K/V of chunk c (c >= nch: a masked stand-in chunk, so every load is
  // unconditional).  Lane (l16, q4) of tile j holds token t0 + 16 j + l16.
  auto load = [&](int32_t c, vec8(&kf)[2][KS], vec8(&vf)[2][KS]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int32_t t = s + kPrefillChunk * c + 16 * j + l16;
      const int32_t row = (c < nch && t < kend) ? t : s;
      const T *kr = kbase + static_cast<int64_t>(row) * p.k_stride + 8 * q4;
      const T *vr = vbase + static_cast<int64_t>(row) * p.v_stride + 8 * q4;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[j][ks] = *reinterpret_cast<const vec8 *>(kr + 32 * ks);
        vf[j][ks] = *reinterpret_cast<const vec8 *>(vr + 32 * ks);
      }
    }
  };

  auto compute = [&](int32_t c, vec8(&kf)[2][KS], vec8(&vf)[2][KS]) {
    const int32_t t0 = s + kPrefillChunk * c;
    // Tokens past kend read a stand-in row: zero their V rows.
    const bool partial = t0 + kPrefillChunk > kend;
    if (partial) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          vf[j][ks] = (t0 + 16 * j + l16 < kend) ? vf[j][ks] : vec8{};
    }
    // Stage V token-major and read V^T once for all heads.
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        *reinterpret_cast<vec8 *>(vt + (16 * j + l16) * kRow + (32 * ks + 8 * q4) * 2) = vf[j][ks];
    __asm__ volatile("" ::: "memory");
    vec8 vtf[NB];
    {
      const unsigned char *rd = vt + (4 * q4 + (l16 >> 2)) * kRow + (l16 & 3) * 8;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const pf_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4 *)(rd + 32 * n));
        const pf_i16x4 hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((pf_lds_i16x4 *)(rd + 16 * kRow + 32 * n));
        vtf[n] = __builtin_bit_cast(vec8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
    __asm__ volatile("" ::: "memory");
    // Causal mask: needed when some key token of the chunk lies past the
    // tile's first query token or past kend.
    const bool masked = partial || t0 + kPrefillChunk - 1 > i0;
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
      vec8 pf;
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float pr = m_run[hq] == kPrefillNegInf
                             ? 0.f
                             : __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i], p.scale_log2, -m_run[hq]));
        psum += pr;
        pf[i] = static_cast<T>(pr);
      }
      l_run[hq] += psum;
#pragma unroll
      for (int n = 0; n < NB; ++n) acc[hq][n] = M::mma(vtf[n], pf, acc[hq][n]);
    }
  };

  vec8 ka[2][KS], va[2][KS], kb[2][KS], vb[2][KS];
  load(0, ka, va);
  for (int32_t c = 0; c < nch; c += 2) {
    load(c + 1, kb, vb);
    compute(c, ka, va);
    if (c + 1 >= nch) break;
    load(c + 2, ka, va);
    compute(c + 1, kb, vb);
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
  hipLaunchKernelGGL((prefill_attention_kernel<T, D, QH>), grid, dim3(64), 0, stream, p);
}

template <typename T, int D>
void launch_prefill_qh(const PrefillParams &p, int32_t ntiles, int32_t heads_per_wave,
                       hipStream_t stream) {
  // Query heads per wavefront (a power of two dividing the group): as asked,
  // else 4 (at most 4 at head_dim 128, for registers).
  constexpr int kMax = D >= 128 ? 4 : 8;
  int32_t qh = heads_per_wave > 0 ? heads_per_wave : 4;
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
