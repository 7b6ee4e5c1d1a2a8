// Decode-shaped linear layer on MFMA: y[M, N] = x[M, K] . w[N, K]^T for
// M <= 64 rows (one token per decode lane), bf16 / fp16 storage, fp32
// accumulation, one rounding.
//
// At decode batch sizes the layer is a stream over the weight matrix (N*K
// elements, each used M times): it is HBM-bound, and what limits a library
// GEMM tiled for large M is parallelism -- a 16 x 64 output tiling of a
// 2048 x 2048 weight gives 128 workgroups that each walk all of K.  Here a
// workgroup owns 16 output columns and splits K across up to 16 wavefronts,
// so a launch has N/16 x (K / k_per_wave) wavefronts each streaming a short
// 16-row slab of w, with several k-steps of loads in flight; the partial
// sums meet once in LDS.
//
// MFMA v_mfma_f32_16x16x32 (bf16 / f16) with
//   A = x rows:  lane (l16, q4) holds x[16 mt + l16][k + 8 q4 .. +8]
//   B = w rows:  lane (l16, q4) holds w[n0 + l16][k + 8 q4 .. +8]
//   C:           lane (l16, q4), register r holds y[16 mt + 4 q4 + r][n0 + l16]
// so both operands are one 16-byte load per lane from a K-contiguous row.
//
// Reference semantics: torch.nn.functional.linear(x, w) without bias, the
// nn.Linear projections of the reference's model (q/k/v/o at
// tensorforge/model/layers.py:88-95, gate/up/down at :144-146) as its decode
// step calls them (tensorforge/runtime/decode_bucket.py:441-447, 470,
// 500-505).
#include "tf_common.hpp"

namespace tf {
namespace {

template <typename T>
struct Mma16;

template <>
struct Mma16<__bf16> {
  typedef __bf16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mma16<_Float16> {
  typedef _Float16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// k-steps (of 32) whose loads are issued together: 16 operand loads per
// batch (kUnroll * (MT + 1) <= 20), so they all stay in registers.
template <int MT>
constexpr int unroll_for() { return MT <= 1 ? 8 : (MT == 2 ? 4 : (MT == 3 ? 4 : 4)); }

// blockIdx.x = 16-column tile; wavefront w sums k in [w * kpw, (w + 1) * kpw).
template <typename T, int MT>
__global__ void __launch_bounds__(1024)
linear_rows_kernel(const T *__restrict__ x, int64_t x_stride, const T *__restrict__ w,
                   int64_t w_stride, T *__restrict__ y, int64_t y_stride, int32_t m, int32_t n,
                   int32_t k, int32_t k_per_wave) {
  using M = Mma16<T>;
  using vec8 = typename M::vec8;
  constexpr int kUnroll = unroll_for<MT>();
  extern __shared__ __attribute__((aligned(16))) float partial[];  // [waves][MT * 4][64]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int32_t n0 = blockIdx.x * 16;
  const int32_t col = min(n0 + l16, n - 1);  // tail columns read a valid row
  const int32_t k0 = wave * k_per_wave;
  const int32_t k1 = min(k0 + k_per_wave, k);

  const T *wrow = w + static_cast<int64_t>(col) * w_stride + 8 * q4;
  const T *xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = x + static_cast<int64_t>(min(16 * mt + l16, m - 1)) * x_stride + 8 * q4;

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  int32_t kk = k0;
  for (; kk + 32 * kUnroll <= k1; kk += 32 * kUnroll) {
    vec8 wb[kUnroll];
    vec8 xa[kUnroll][MT];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      wb[u] = *reinterpret_cast<const vec8 *>(wrow + kk + 32 * u);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        xa[u][mt] = *reinterpret_cast<const vec8 *>(xrow[mt] + kk + 32 * u);
    }
    // Keep the scheduler from interleaving the batch's loads with its
    // MFMAs: it would otherwise trade loads in flight for registers.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = M::mma(xa[u][mt], wb[u], acc[mt]);
  }
  for (; kk < k1; kk += 32) {
    const vec8 wb = *reinterpret_cast<const vec8 *>(wrow + kk);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      acc[mt] = M::mma(*reinterpret_cast<const vec8 *>(xrow[mt] + kk), wb, acc[mt]);
  }

  // Cross-wavefront sum: item (mt, r, lane) is y[16 mt + 4 q4 + r][n0 + l16].
  constexpr int kItems = MT * 4 * 64;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) partial[wave * kItems + (mt * 4 + r) * 64 + lane] = acc[mt][r];
  __syncthreads();
  for (int item = threadIdx.x; item < kItems; item += blockDim.x) {
    float sum = 0.f;
    for (int wv = 0; wv < waves; ++wv) sum += partial[wv * kItems + item];
    const int mt = item / 256;
    const int r = (item >> 6) & 3;
    const int il = item & 63;
    const int32_t row = 16 * mt + 4 * (il >> 4) + r;
    const int32_t c = n0 + (il & 15);
    if (row < m && c < n) y[static_cast<int64_t>(row) * y_stride + c] = from_float<T>(sum);
  }
}

template <typename T, int MT>
void launch_rows(const void *x, int64_t x_stride, const void *w, int64_t w_stride, void *y,
                 int64_t y_stride, int32_t m, int32_t n, int32_t k, int32_t waves,
                 int32_t k_per_wave, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(waves) * MT * 4 * 64 * sizeof(float);
  hipLaunchKernelGGL((linear_rows_kernel<T, MT>), dim3((n + 15) / 16), dim3(waves * 64), lds,
                     stream, static_cast<const T *>(x), x_stride, static_cast<const T *>(w),
                     w_stride, static_cast<T *>(y), y_stride, m, n, k, k_per_wave);
}

template <typename T>
void launch_rows_mt(const void *x, int64_t x_stride, const void *w, int64_t w_stride, void *y,
                    int64_t y_stride, int32_t m, int32_t n, int32_t k, int32_t waves,
                    int32_t k_per_wave, hipStream_t stream) {
#define TF_ROWS_CASE(MT)                                                                \
  launch_rows<T, MT>(x, x_stride, w, w_stride, y, y_stride, m, n, k, waves, k_per_wave, \
                     stream)
  switch ((m + 15) / 16) {
    case 1: TF_ROWS_CASE(1); break;
    case 2: TF_ROWS_CASE(2); break;
    case 3: TF_ROWS_CASE(3); break;
    default: TF_ROWS_CASE(4); break;
  }
#undef TF_ROWS_CASE
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_linear_rows(const void *x, int64_t x_row_stride, const void *weight,
                                  int64_t weight_row_stride, void *y, int64_t y_row_stride,
                                  int32_t m, int32_t n, int32_t k, int32_t waves_per_tile,
                                  int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (dtype != TF_DTYPE_FLOAT16 && dtype != TF_DTYPE_BFLOAT16)
    return fail(TF_ERROR_UNSUPPORTED, "linear_rows supports fp16 and bf16");
  if (m < 0 || n < 0 || k < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "sizes must be non-negative");
  if (m > 64) return fail(TF_ERROR_UNSUPPORTED, "linear_rows supports at most 64 rows");
  if (k % 32 != 0) return fail(TF_ERROR_UNSUPPORTED, "linear_rows needs K to be a multiple of 32");
  if (x_row_stride < k || weight_row_stride < k || y_row_stride < n)
    return fail(TF_ERROR_INVALID_ARGUMENT, "row strides are shorter than the rows");
  if (m == 0 || n == 0) return TF_SUCCESS;
  if (!x || !weight || !y) return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                          static_cast<uintptr_t>(x_row_stride * 2) |
                          static_cast<uintptr_t>(weight_row_stride * 2);
  if (align % 16 != 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_rows needs 16-byte aligned x and weight rows");
  if (k == 0) return fail(TF_ERROR_UNSUPPORTED, "linear_rows needs K > 0");
  // Wavefronts per 16-column tile: enough for ~2048 wavefronts in the launch
  // (8 per CU), at most 16, each with at least one k-step.
  const int32_t tiles = (n + 15) / 16;
  int32_t waves = waves_per_tile > 0 ? waves_per_tile : (2048 + tiles - 1) / tiles;
  waves = waves < 1 ? 1 : (waves > 16 ? 16 : waves);
  if (waves > k / 32) waves = k / 32;
  const int32_t steps = k / 32;
  const int32_t k_per_wave = ((steps + waves - 1) / waves) * 32;
  waves = (k + k_per_wave - 1) / k_per_wave;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TF_DTYPE_BFLOAT16)
    launch_rows_mt<__bf16>(x, x_row_stride, weight, weight_row_stride, y, y_row_stride, m, n, k,
                           waves, k_per_wave, s);
  else
    launch_rows_mt<_Float16>(x, x_row_stride, weight, weight_row_stride, y, y_row_stride, m, n,
                             k, waves, k_per_wave, s);
  return check_launch("linear_rows");
}
