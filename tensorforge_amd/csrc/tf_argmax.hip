// Greedy sampling: the argmax of every row of a logits matrix.
//
// Reference semantics: torch.argmax(logits, dim=-1) as the continuous
// scheduler applies it to each step's logits (scheduler/continuous.py:
// 265-275; runtime/generation.py:43): the index of the largest value, the
// first such index on ties, and a NaN counts as larger than every number
// (the first NaN wins).
//
// One workgroup of 1024 threads per row.  A pass issues all of a thread's
// 16-byte loads (up to kLoads vectors: 32768 bf16/fp16 or 16384 fp32
// elements per pass) before it compares any, so a TinyLlama row (32000
// bf16, 64 KB) is one memory round trip, held in registers for the second
// scan; the per-thread results meet through lane shuffles within each
// wavefront and LDS across the 16.
#include "tf_common.hpp"

namespace tf {
namespace {

constexpr int kArgmaxThreads = 1024;
constexpr int kLoads = 4;  // 16-byte vectors per thread per pass
constexpr int32_t kNone = 0x7fffffff;  // index of "no element yet"

// Two branch-free passes over the row: the largest value (and whether any
// element is a NaN), then the first index holding it (the first NaN when
// there is one).  A NaN never wins fmaxf, so the NaN case is carried by the
// flag.  fmaxf may return either zero for (-0, +0) and x == target holds
// for both, so a row whose largest value is zero picks its first zero of
// either sign, as torch's strict comparison does.
template <typename T, int VEC>
__global__ void __launch_bounds__(kArgmaxThreads)
argmax_rows_kernel(const T *__restrict__ logits, int64_t row_stride, int32_t columns,
                   int64_t *__restrict__ out) {
  struct alignas(sizeof(T) * VEC) Vec {
    T v[VEC];
  };
  constexpr int kWaves = kArgmaxThreads / 64;
  constexpr int32_t kPass = kArgmaxThreads * kLoads;  // vectors per pass
  __shared__ float wave_max[kWaves];
  __shared__ int32_t wave_int[kWaves];
  const T *row = logits + static_cast<int64_t>(blockIdx.x) * row_stride;
  const Vec *vrow = reinterpret_cast<const Vec *>(row);
  const int32_t nvec = columns / VEC;
  const int32_t tid = static_cast<int32_t>(threadIdx.x);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;

  auto load_pass = [&](int32_t base, Vec(&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int32_t i = base + u * kArgmaxThreads + tid;
      if (i < nvec) v[u] = vrow[i];
    }
  };
  float vmax = -__builtin_inff();
  int32_t nan = 0;
  auto scan_max = [&](int32_t base, const Vec(&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      if (base + u * kArgmaxThreads + tid >= nvec) continue;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float x = to_float(v[u].v[e]);
        vmax = fmaxf(vmax, x);
        nan |= x != x;
      }
    }
  };
  Vec first_pass[kLoads];
  load_pass(0, first_pass);
  scan_max(0, first_pass);
  for (int32_t base = kPass; base < nvec; base += kPass) {
    Vec v[kLoads];
    load_pass(base, v);
    scan_max(base, v);
  }
  // Columns past the last whole vector (VEC == 1 covers every column above).
  for (int32_t c = nvec * VEC + tid; c < columns; c += kArgmaxThreads) {
    const float x = to_float(row[c]);
    vmax = fmaxf(vmax, x);
    nan |= x != x;
  }
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    vmax = fmaxf(vmax, __shfl_xor(vmax, offset, 64));
    nan |= __shfl_xor(nan, offset, 64);
  }
  if (lane == 0) {
    wave_max[wave] = vmax;
    wave_int[wave] = nan;
  }
  __syncthreads();
  float target = wave_max[0];
  int32_t any_nan = wave_int[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    target = fmaxf(target, wave_max[w]);
    any_nan |= wave_int[w];
  }
  __syncthreads();  // the slots are reused below

  int32_t first = kNone;
  auto scan_first = [&](int32_t base, const Vec(&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int32_t i = base + u * kArgmaxThreads + tid;
      if (i >= nvec) continue;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float x = to_float(v[u].v[e]);
        const bool hit = any_nan ? x != x : x == target;
        first = min(first, hit ? i * VEC + e : kNone);
      }
    }
  };
  scan_first(0, first_pass);
  for (int32_t base = kPass; base < nvec; base += kPass) {
    Vec v[kLoads];
    load_pass(base, v);
    scan_first(base, v);
  }
  for (int32_t c = nvec * VEC + tid; c < columns; c += kArgmaxThreads) {
    const float x = to_float(row[c]);
    const bool hit = any_nan ? x != x : x == target;
    first = min(first, hit ? c : kNone);
  }
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) first = min(first, __shfl_xor(first, offset, 64));
  if (lane == 0) wave_int[wave] = first;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kWaves; ++w) first = min(first, wave_int[w]);
    out[blockIdx.x] = first;
  }
}

template <typename T>
void launch_argmax(const void *logits, int64_t row_stride, int32_t rows, int32_t columns,
                   int64_t *out, hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(T);
  const bool vector = reinterpret_cast<uintptr_t>(logits) % 16 == 0 && row_stride % VEC == 0;
  if (vector)
    hipLaunchKernelGGL((argmax_rows_kernel<T, VEC>), dim3(static_cast<unsigned>(rows)),
                       dim3(kArgmaxThreads), 0, stream, static_cast<const T *>(logits), row_stride,
                       columns, out);
  else
    hipLaunchKernelGGL((argmax_rows_kernel<T, 1>), dim3(static_cast<unsigned>(rows)),
                       dim3(kArgmaxThreads), 0, stream, static_cast<const T *>(logits), row_stride,
                       columns, out);
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_argmax_rows(const void *logits, int64_t row_stride, int32_t rows,
                                  int32_t columns, int32_t dtype, int64_t *out, void *stream) {
  using namespace tf;
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (rows < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "rows must be non-negative");
  if (columns < 1) return fail(TF_ERROR_INVALID_ARGUMENT, "argmax needs at least one column");
  if (row_stride < columns) return fail(TF_ERROR_INVALID_ARGUMENT, "row stride is shorter than the rows");
  if (rows == 0) return TF_SUCCESS;
  if (!logits || !out) return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TF_DTYPE_FLOAT32:
      launch_argmax<float>(logits, row_stride, rows, columns, out, s);
      break;
    case TF_DTYPE_FLOAT16:
      launch_argmax<_Float16>(logits, row_stride, rows, columns, out, s);
      break;
    default:
      launch_argmax<__bf16>(logits, row_stride, rows, columns, out, s);
      break;
  }
  return check_launch("argmax_rows");
}
