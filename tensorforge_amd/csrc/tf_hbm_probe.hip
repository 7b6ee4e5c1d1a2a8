// Read-bandwidth probe: the rate at which this GPU streams bytes from HBM.
//
// The measurement side of the decode-attention roofline.  The attention
// kernels are HBM-bound, so their achieved rate is compared with what a
// plain streaming read reaches on the same device in the same process: each
// workgroup reads one contiguous slice of the buffer with 16-byte
// nontemporal loads, `loads` of them in flight per lane, and folds the words
// into a value that is stored only if it equals a constant (so the loads
// cannot be dropped).  The reference measures its ceiling with a device copy
// instead (tensorforge/benchmark/kernel_benchmark.py:176-192).
#include "tf_common.hpp"

namespace tf {
namespace {

template <int LOADS>
__global__ void __launch_bounds__(1024) hbm_read_kernel(const u32x4 *__restrict__ base,
                                                        int64_t elements, int64_t per_wg,
                                                        uint32_t *__restrict__ sink) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * per_wg;
  int64_t last = first + per_wg;
  if (last > elements) last = elements;
  const int64_t stride = blockDim.x;
  uint32_t acc = 0;
  for (int64_t i = first + threadIdx.x; i < last; i += stride * LOADS) {
    u32x4 v[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int64_t idx = i + u * stride;
      v[u] = idx < last ? __builtin_nontemporal_load(base + idx) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < LOADS; ++u) acc ^= v[u].x + v[u].y + v[u].z + v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_hbm_read_probe(const void *buffer, int64_t bytes, int32_t workgroups,
                                     int32_t waves, int32_t loads, uint32_t *sink, void *stream) {
  using namespace tf;
  clear_error();
  if (bytes <= 0 || bytes % 16 != 0 || workgroups <= 0 || waves <= 0 || waves > 16 || !buffer ||
      !sink || (reinterpret_cast<uintptr_t>(buffer) & 15) != 0)
    return fail(TF_ERROR_INVALID_ARGUMENT,
                "probe needs a 16-byte aligned buffer of a positive multiple of 16 bytes, "
                "workgroups > 0 and 1..16 waves");
  const int64_t elements = bytes / 16;
  const int64_t per_wg = (elements + workgroups - 1) / workgroups;
  const u32x4 *base = static_cast<const u32x4 *>(buffer);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(workgroups)), block(64u * static_cast<unsigned>(waves));
  switch (loads) {
    case 2:
      hipLaunchKernelGGL(hbm_read_kernel<2>, grid, block, 0, s, base, elements, per_wg, sink);
      break;
    case 4:
      hipLaunchKernelGGL(hbm_read_kernel<4>, grid, block, 0, s, base, elements, per_wg, sink);
      break;
    case 8:
      hipLaunchKernelGGL(hbm_read_kernel<8>, grid, block, 0, s, base, elements, per_wg, sink);
      break;
    default:
      return fail(TF_ERROR_INVALID_ARGUMENT, "loads in flight must be 2, 4 or 8");
  }
  return check_launch("hbm read probe");
}
