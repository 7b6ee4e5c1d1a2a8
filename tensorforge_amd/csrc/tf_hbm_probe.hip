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
//
// The page-gather probe reads the K and V pages of one attention call --
// the same scattered physical pages, every byte of each -- and nothing
// else: the attainable rate of the call's own access pattern, with no
// compute, no softmax state and no output.  Each wavefront takes an equal
// contiguous range of the page list and reads its pages whole (1 KB per
// load instruction), one page of K and V in flight per wavefront.
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

constexpr int kGatherLoads = 8;  // 1 KB pieces of a page per tensor per step

__global__ void __launch_bounds__(1024) page_gather_kernel(const u32x4 *__restrict__ kbase,
                                                           const u32x4 *__restrict__ vbase,
                                                           const int32_t *__restrict__ pages,
                                                           int32_t npages, int64_t page_vecs,
                                                           int32_t num_blocks,
                                                           uint32_t *__restrict__ sink) {
  const int32_t waves = blockDim.x >> 6;
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * waves + (threadIdx.x >> 6);
  const int64_t nw = static_cast<int64_t>(gridDim.x) * waves;
  const int lane = threadIdx.x & 63;
  const int64_t p0 = npages * gw / nw;
  const int64_t p1 = npages * (gw + 1) / nw;
  uint32_t acc = 0;
  for (int64_t p = p0; p < p1; ++p) {
    const int32_t page = pages[p];
    if (page < 0 || page >= num_blocks) continue;
    const int64_t base = static_cast<int64_t>(page) * page_vecs;
    for (int64_t c = 0; c < page_vecs; c += 64 * kGatherLoads) {
      u32x4 kv[kGatherLoads], vv[kGatherLoads];
#pragma unroll
      for (int u = 0; u < kGatherLoads; ++u) {
        const int64_t idx = c + 64 * u + lane;
        const bool in = idx < page_vecs;
        kv[u] = in ? __builtin_nontemporal_load(kbase + base + idx) : u32x4{0, 0, 0, 0};
        vv[u] = in ? __builtin_nontemporal_load(vbase + base + idx) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < kGatherLoads; ++u)
        acc ^= kv[u].x + kv[u].y + kv[u].z + kv[u].w + vv[u].x + vv[u].y + vv[u].z + vv[u].w;
    }
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

extern "C" int32_t tf_hbm_page_gather_probe(const void *key_cache, const void *value_cache,
                                            const int32_t *pages, int32_t npages,
                                            int64_t page_bytes, int32_t num_blocks,
                                            int32_t workgroups, int32_t waves, uint32_t *sink,
                                            void *stream) {
  using namespace tf;
  clear_error();
  if (npages < 0 || page_bytes <= 0 || page_bytes % 1024 != 0 || num_blocks <= 0 ||
      workgroups <= 0 || waves <= 0 || waves > 16 || !sink ||
      (npages > 0 && (!key_cache || !value_cache || !pages)) ||
      (reinterpret_cast<uintptr_t>(key_cache) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(value_cache) & 15) != 0)
    return fail(TF_ERROR_INVALID_ARGUMENT,
                "page gather probe needs 16-byte aligned caches, pages of a positive multiple "
                "of 1024 bytes, num_blocks > 0, workgroups > 0 and 1..16 waves");
  if (npages == 0) return TF_SUCCESS;
  hipLaunchKernelGGL(page_gather_kernel, dim3(static_cast<unsigned>(workgroups)),
                     dim3(64u * static_cast<unsigned>(waves)), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4 *>(key_cache), static_cast<const u32x4 *>(value_cache),
                     pages, npages, page_bytes / 16, num_blocks, sink);
  return check_launch("page gather probe");
}
