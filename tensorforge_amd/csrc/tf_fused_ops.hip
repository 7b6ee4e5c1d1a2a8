// Row-wise RMSNorm, fused residual-add + RMSNorm and elementwise SwiGLU.
//
// All three are HBM-bound streaming kernels.  A row of the norms is held in
// registers (up to kMaxVecs 16-byte vectors per lane) so each input byte is
// read once; the sum of squares is reduced across the wavefront with lane
// shuffles and across wavefronts through LDS.  Arithmetic is fp32 and every
// output is rounded once to the storage type.
//
// Reference semantics:
//   rms_norm           tensorforge/kernels/triton_ops.py:36-66 (kernel),
//                      :179-205 (host); oracle kernels/reference.py:10-15
//   residual_rms_norm  triton_ops.py:68-97, :208-243 -- the residual sum is
//                      stored rounded, the norm uses the fp32 sum
//   swiglu             triton_ops.py:106-122, :246-260 -- g*sigmoid(g)*u in
//                      fp32, one rounding
//   swiglu_rows        the same activation read from one fused gate|up
//                      projection row (no reference counterpart: the
//                      reference runs gate and up as two GEMMs)
#include "tf_common.hpp"

namespace tf {
namespace {

// Register-cache capacity (vectors per lane) of the norm kernels: 8 x 16-byte
// vectors for the vector path, 32 scalars for odd widths; with the largest
// workgroup (kMaxNormThreads lanes) both cover the 16384-column limit of the
// reference contract.
template <int VEC>
constexpr int max_vecs() { return VEC == 1 ? 32 : 8; }

// Norm workgroups are 1, 2, 4 or 8 wavefronts: the reference's autotune
// set for these kernels (tensorforge/kernels/triton_ops.py:28-33), which
// its observability hook reports as `num_warps`.
constexpr int kMaxNormThreads = 512;

template <typename T, int VEC>
struct alignas(sizeof(T) * VEC) Vec {
  T v[VEC];
};

// Sum across the whole workgroup (blockDim.x multiple of 64, <= 1024).
__device__ __forceinline__ float block_sum(float v, float *scratch) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float total = 0.f;
  for (int w = 0; w < waves; ++w) total += scratch[w];
  return total;
}

// Token ids of a decode step's rows: row b reads state[source[b]] when
// source[b] >= 0 (the token its lane sampled last step) and host[b]
// otherwise; ids are clamped to the table.
struct GatherRows {
  const int64_t *state = nullptr;
  int64_t state_len = 0;
  const int64_t *source = nullptr;
  const int64_t *host = nullptr;
  int64_t vocab = 0;
};

// One workgroup per row.  RESIDUAL selects the fused residual variant.
// PARTIALS (with RESIDUAL) reads no `inputs`:
// element j of the row is round(sum_s partials[s][row][j]) over `splits`
// dense fp32 [rows, columns] planes, the rounded result of a split-K
// projection (tf_linear_partials) whose sum is fused here.  GATHER (plain
// norm) reads row id(b) of `inputs` -- an embedding table -- and also stores
// that row to `residual_output`.
template <typename T, int VEC, bool RESIDUAL, bool PARTIALS, bool GATHER = false>
__global__ void __launch_bounds__(kMaxNormThreads)
rms_norm_kernel(const T *__restrict__ inputs, const T *__restrict__ residual,
                const T *__restrict__ weight, T *__restrict__ residual_output,
                T *__restrict__ output, int32_t columns, float eps,
                const float *__restrict__ partials, int32_t splits, int64_t plane,
                GatherRows gather) {
  __shared__ float scratch[16];
  using V = Vec<T, VEC>;
  const int64_t row = blockIdx.x;
  const int32_t nvec = columns / VEC;
  int64_t in_row = row;
  if constexpr (GATHER) {
    const int64_t src = gather.source[row];
    int64_t id = src >= 0 ? gather.state[src < gather.state_len ? src : gather.state_len - 1]
                          : gather.host[row];
    in_row = id < 0 ? 0 : (id >= gather.vocab ? gather.vocab - 1 : id);
  }
  const V *x = reinterpret_cast<const V *>(inputs + (PARTIALS ? 0 : in_row * columns));
  const float *prow = PARTIALS ? partials + row * columns : nullptr;
  const V *r = reinterpret_cast<const V *>(residual + (RESIDUAL ? row * columns : 0));
  V *ro = reinterpret_cast<V *>(residual_output + (RESIDUAL || GATHER ? row * columns : 0));
  V *y = reinterpret_cast<V *>(output + row * columns);
  const V *w = reinterpret_cast<const V *>(weight);

  constexpr int kMaxVecs = max_vecs<VEC>();
  float cache[kMaxVecs][VEC];
  float sq = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxVecs; ++k) {
    const int32_t idx = threadIdx.x + k * blockDim.x;
    if (idx < nvec) {
      V xv;
      if constexpr (PARTIALS) {
        float sum[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) sum[e] = 0.f;
        // Slices in groups of kGroup whose loads are all issued before any
        // is added (a slice past the last re-reads slice 0 and is dropped),
        // so a row costs one memory round trip per kGroup slices; the sum
        // still runs in slice order.
        constexpr int kGroup = 8;
        const float *base = prow + static_cast<int64_t>(idx) * VEC;
        for (int32_t s0 = 0; s0 < splits; s0 += kGroup) {
          float v[kGroup][VEC];
#pragma unroll
          for (int g = 0; g < kGroup; ++g) {
            const float *src = base + (s0 + g < splits ? s0 + g : 0) * plane;
            if constexpr (VEC % 4 == 0) {
#pragma unroll
              for (int q = 0; q < VEC / 4; ++q) {
                const f32x4 x4 = *reinterpret_cast<const f32x4 *>(src + 4 * q);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[g][4 * q + e] = x4[e];
              }
            } else {
#pragma unroll
              for (int e = 0; e < VEC; ++e) v[g][e] = src[e];
            }
          }
#pragma unroll
          for (int g = 0; g < kGroup; ++g)
            if (s0 + g < splits)
#pragma unroll
              for (int e = 0; e < VEC; ++e) sum[e] += v[g][e];
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) xv.v[e] = from_float<T>(sum[e]);
      } else {
        xv = x[idx];
        if constexpr (GATHER) ro[idx] = xv;
      }
      V rv;
      if constexpr (RESIDUAL) rv = r[idx];
      V sv;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float s = to_float(xv.v[e]);
        if constexpr (RESIDUAL) {
          s += to_float(rv.v[e]);
          sv.v[e] = from_float<T>(s);
        }
        cache[k][e] = s;
        sq += s * s;
      }
      if constexpr (RESIDUAL) ro[idx] = sv;
    }
  }
  const float inv_rms = rsqrtf(block_sum(sq, scratch) / static_cast<float>(columns) + eps);
#pragma unroll
  for (int k = 0; k < kMaxVecs; ++k) {
    const int32_t idx = threadIdx.x + k * blockDim.x;
    if (idx < nvec) {
      V wv = w[idx];
      V out;
#pragma unroll
      for (int e = 0; e < VEC; ++e) out.v[e] = from_float<T>(cache[k][e] * inv_rms * to_float(wv.v[e]));
      y[idx] = out;
    }
  }
}

template <typename T, int VEC>
__device__ __forceinline__ Vec<T, VEC> swiglu_vec(const Vec<T, VEC> &gv, const Vec<T, VEC> &uv) {
  Vec<T, VEC> out;
#pragma unroll
  for (int e = 0; e < VEC; ++e) out.v[e] = from_float<T>(swiglu_act(to_float(gv.v[e]), to_float(uv.v[e])));
  return out;
}

template <typename T, int VEC>
__global__ void __launch_bounds__(256)
swiglu_kernel(const T *__restrict__ gate, const T *__restrict__ up, T *__restrict__ output,
              int64_t nvec) {
  using V = Vec<T, VEC>;
  const V *g = reinterpret_cast<const V *>(gate);
  const V *u = reinterpret_cast<const V *>(up);
  V *o = reinterpret_cast<V *>(output);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nvec; i += stride)
    o[i] = swiglu_vec<T, VEC>(g[i], u[i]);
}

// Row r of `gate_up` holds gate[0..columns) then up[0..columns); strides in
// elements.  cvec = columns / VEC vectors per row.
template <typename T, int VEC>
__global__ void __launch_bounds__(256)
swiglu_rows_kernel(const T *__restrict__ gate_up, int64_t in_stride, T *__restrict__ output,
                   int64_t out_stride, int64_t rows, int32_t cvec) {
  using V = Vec<T, VEC>;
  const int64_t total = rows * cvec;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += stride) {
    const int64_t r = i / cvec;
    const int64_t c = i - r * cvec;
    const V *g = reinterpret_cast<const V *>(gate_up + r * in_stride);
    reinterpret_cast<V *>(output + r * out_stride)[c] = swiglu_vec<T, VEC>(g[c], g[cvec + c]);
  }
}

template <typename T, int VEC, bool RESIDUAL>
void launch_norm(const void *inputs, const void *residual, const void *weight,
                 void *residual_output, void *output, int64_t rows, int32_t columns,
                 float eps, const float *partials, int32_t splits, hipStream_t stream,
                 const GatherRows *gather) {
  const int32_t nvec = columns / VEC;
  // The fewest wavefronts (1, 2, 4 or 8) that leave each lane at most two
  // vectors (one when the inputs are summed from split-K partials, which
  // costs more loads per vector); wider rows give each of 8 wavefronts'
  // lanes more vectors, up to the register cache's max_vecs<VEC>().
  const int per_lane = partials ? 1 : 2;
  int threads = 64;
  while (threads < kMaxNormThreads && threads * per_lane < nvec) threads *= 2;
  const int64_t plane = rows * static_cast<int64_t>(columns);
  if (!RESIDUAL && gather)
    hipLaunchKernelGGL((rms_norm_kernel<T, VEC, false, false, true>), dim3(static_cast<unsigned>(rows)),
                       dim3(threads), 0, stream, static_cast<const T *>(inputs),
                       static_cast<const T *>(residual), static_cast<const T *>(weight),
                       static_cast<T *>(residual_output), static_cast<T *>(output), columns, eps,
                       nullptr, 0, plane, *gather);
  else if (RESIDUAL && partials)
    hipLaunchKernelGGL((rms_norm_kernel<T, VEC, RESIDUAL, RESIDUAL>), dim3(static_cast<unsigned>(rows)),
                       dim3(threads), 0, stream, static_cast<const T *>(inputs),
                       static_cast<const T *>(residual), static_cast<const T *>(weight),
                       static_cast<T *>(residual_output), static_cast<T *>(output), columns, eps,
                       partials, splits, plane, GatherRows{});
  else
    hipLaunchKernelGGL((rms_norm_kernel<T, VEC, RESIDUAL, false>), dim3(static_cast<unsigned>(rows)),
                       dim3(threads), 0, stream, static_cast<const T *>(inputs),
                       static_cast<const T *>(residual), static_cast<const T *>(weight),
                       static_cast<T *>(residual_output), static_cast<T *>(output), columns, eps,
                       nullptr, 0, plane, GatherRows{});
}

template <typename T, bool RESIDUAL>
int32_t dispatch_norm(const void *inputs, const void *residual, const void *weight,
                      void *residual_output, void *output, int64_t rows, int32_t columns,
                      float eps, const float *partials, int32_t splits, hipStream_t stream,
                      const GatherRows *gather) {
  constexpr int kVec = 16 / sizeof(T);
  uintptr_t align = reinterpret_cast<uintptr_t>(partials ? partials : inputs) |
                    reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(output);
  if (RESIDUAL)
    align |= reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(residual_output);
  if (gather) align |= reinterpret_cast<uintptr_t>(residual_output);
  const bool vectorised = columns % kVec == 0 && align % 16 == 0 &&
                          columns / kVec <= kMaxNormThreads * max_vecs<kVec>();
  if (vectorised) {
    launch_norm<T, kVec, RESIDUAL>(inputs, residual, weight, residual_output, output, rows,
                                   columns, eps, partials, splits, stream, gather);
  } else if (columns <= kMaxNormThreads * max_vecs<1>()) {
    launch_norm<T, 1, RESIDUAL>(inputs, residual, weight, residual_output, output, rows,
                                columns, eps, partials, splits, stream, gather);
  } else {
    return fail(TF_ERROR_UNSUPPORTED, "RMSNorm row does not fit the register cache");
  }
  return check_launch(RESIDUAL ? "residual_rms_norm" : "rms_norm");
}

template <bool RESIDUAL>
int32_t norm_entry(const void *inputs, const void *residual, const void *weight,
                   void *residual_output, void *output, int64_t rows, int32_t columns,
                   float eps, int32_t dtype, void *stream, const float *partials = nullptr,
                   int32_t splits = 0, const GatherRows *gather = nullptr) {
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (rows < 0 || columns <= 0 || columns > 16384)
    return fail(TF_ERROR_INVALID_ARGUMENT, "RMSNorm needs 0 <= rows and 0 < columns <= 16384");
  if (rows > 0x7fffffff) return fail(TF_ERROR_UNSUPPORTED, "too many rows for one launch");
  if (!(eps > 0.f)) return fail(TF_ERROR_INVALID_ARGUMENT, "eps must be positive");
  if (!(partials ? static_cast<const void *>(partials) : inputs) || !weight || !output ||
      (RESIDUAL && (!residual || !residual_output)) || (gather && !residual_output))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (rows == 0) return TF_SUCCESS;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TF_DTYPE_FLOAT32:
      return dispatch_norm<float, RESIDUAL>(inputs, residual, weight, residual_output, output,
                                            rows, columns, eps, partials, splits, s, gather);
    case TF_DTYPE_FLOAT16:
      return dispatch_norm<_Float16, RESIDUAL>(inputs, residual, weight, residual_output,
                                               output, rows, columns, eps, partials, splits, s, gather);
    default:
      return dispatch_norm<__bf16, RESIDUAL>(inputs, residual, weight, residual_output, output,
                                             rows, columns, eps, partials, splits, s, gather);
  }
}

template <typename T>
int32_t swiglu_dispatch(const void *gate, const void *up, void *output, int64_t numel,
                        hipStream_t stream) {
  constexpr int kVec = 16 / sizeof(T);
  const uintptr_t align = reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) |
                          reinterpret_cast<uintptr_t>(output);
  const int threads = 256;
  if (numel % kVec == 0 && align % 16 == 0) {
    const int64_t nvec = numel / kVec;
    int64_t blocks = (nvec + threads - 1) / threads;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL((swiglu_kernel<T, kVec>), dim3(static_cast<unsigned>(blocks)),
                       dim3(threads), 0, stream, static_cast<const T *>(gate),
                       static_cast<const T *>(up), static_cast<T *>(output), nvec);
  } else {
    int64_t blocks = (numel + threads - 1) / threads;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL((swiglu_kernel<T, 1>), dim3(static_cast<unsigned>(blocks)), dim3(threads),
                       0, stream, static_cast<const T *>(gate), static_cast<const T *>(up),
                       static_cast<T *>(output), numel);
  }
  return check_launch("swiglu");
}

template <typename T>
int32_t swiglu_rows_dispatch(const void *gate_up, int64_t in_stride, void *output,
                             int64_t out_stride, int64_t rows, int32_t columns,
                             hipStream_t stream) {
  constexpr int kVec = 16 / sizeof(T);
  const uintptr_t align = reinterpret_cast<uintptr_t>(gate_up) |
                          reinterpret_cast<uintptr_t>(output) |
                          static_cast<uintptr_t>(in_stride * sizeof(T)) |
                          static_cast<uintptr_t>(out_stride * sizeof(T)) |
                          static_cast<uintptr_t>(columns * sizeof(T));
  const int threads = 256;
  const bool vec = align % 16 == 0;
  const int32_t cvec = vec ? columns / kVec : columns;
  int64_t blocks = (rows * cvec + threads - 1) / threads;
  if (blocks > 8192) blocks = 8192;
  if (vec)
    hipLaunchKernelGGL((swiglu_rows_kernel<T, kVec>), dim3(static_cast<unsigned>(blocks)),
                       dim3(threads), 0, stream, static_cast<const T *>(gate_up), in_stride,
                       static_cast<T *>(output), out_stride, rows, cvec);
  else
    hipLaunchKernelGGL((swiglu_rows_kernel<T, 1>), dim3(static_cast<unsigned>(blocks)),
                       dim3(threads), 0, stream, static_cast<const T *>(gate_up), in_stride,
                       static_cast<T *>(output), out_stride, rows, cvec);
  return check_launch("swiglu_rows");
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_rms_norm(const void *inputs, const void *weight, void *output,
                               int64_t rows, int32_t columns, float eps, int32_t dtype,
                               void *stream) {
  return tf::norm_entry<false>(inputs, nullptr, weight, nullptr, output, rows, columns, eps,
                               dtype, stream);
}

extern "C" int32_t tf_embedding_rms_norm(const int64_t *token_state, int64_t token_state_len,
                                         const int64_t *source_lanes, const int64_t *host_tokens,
                                         const void *embedding, int64_t vocab, const void *weight,
                                         void *x_output, void *norm_output, int64_t rows,
                                         int32_t columns, float eps, int32_t dtype,
                                         void *stream) {
  using namespace tf;
  clear_error();
  if (rows > 0 && (!token_state || !source_lanes || !host_tokens))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null token pointer");
  if (rows > 0 && (token_state_len < 1 || vocab < 1))
    return fail(TF_ERROR_INVALID_ARGUMENT, "token state and vocabulary must be non-empty");
  GatherRows gather;
  gather.state = token_state;
  gather.state_len = token_state_len;
  gather.source = source_lanes;
  gather.host = host_tokens;
  gather.vocab = vocab;
  return norm_entry<false>(embedding, nullptr, weight, x_output, norm_output, rows, columns, eps,
                           dtype, stream, nullptr, 0, &gather);
}

extern "C" int32_t tf_residual_rms_norm(const void *inputs, const void *residual,
                                        const void *weight, void *residual_output,
                                        void *norm_output, int64_t rows, int32_t columns,
                                        float eps, int32_t dtype, void *stream) {
  return tf::norm_entry<true>(inputs, residual, weight, residual_output, norm_output, rows,
                              columns, eps, dtype, stream);
}

extern "C" int32_t tf_residual_rms_norm_partials(const float *partials, int32_t splits,
                                                 const void *residual, const void *weight,
                                                 void *residual_output, void *norm_output,
                                                 int64_t rows, int32_t columns, float eps,
                                                 int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (splits < 1) return fail(TF_ERROR_INVALID_ARGUMENT, "splits must be positive");
  if (!partials) return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  return norm_entry<true>(nullptr, residual, weight, residual_output, norm_output, rows, columns,
                          eps, dtype, stream, partials, splits);
}

extern "C" int32_t tf_swiglu(const void *gate, const void *up, void *output, int64_t numel,
                             int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (numel < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "numel must be non-negative");
  if (numel == 0) return TF_SUCCESS;
  if (!gate || !up || !output) return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TF_DTYPE_FLOAT32:
      return swiglu_dispatch<float>(gate, up, output, numel, s);
    case TF_DTYPE_FLOAT16:
      return swiglu_dispatch<_Float16>(gate, up, output, numel, s);
    default:
      return swiglu_dispatch<__bf16>(gate, up, output, numel, s);
  }
}

extern "C" int32_t tf_swiglu_rows(const void *gate_up, int64_t gate_up_row_stride, void *output,
                                  int64_t output_row_stride, int64_t rows, int32_t columns,
                                  int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (rows < 0 || columns < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "sizes must be non-negative");
  if (gate_up_row_stride < 2 * static_cast<int64_t>(columns) || output_row_stride < columns)
    return fail(TF_ERROR_INVALID_ARGUMENT, "row strides are shorter than the rows");
  if (rows == 0 || columns == 0) return TF_SUCCESS;
  if (!gate_up || !output) return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TF_DTYPE_FLOAT32:
      return swiglu_rows_dispatch<float>(gate_up, gate_up_row_stride, output, output_row_stride,
                                         rows, columns, s);
    case TF_DTYPE_FLOAT16:
      return swiglu_rows_dispatch<_Float16>(gate_up, gate_up_row_stride, output,
                                            output_row_stride, rows, columns, s);
    default:
      return swiglu_rows_dispatch<__bf16>(gate_up, gate_up_row_stride, output,
                                          output_row_stride, rows, columns, s);
  }
}
