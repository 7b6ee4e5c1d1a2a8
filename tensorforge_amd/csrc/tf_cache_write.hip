// Paged KV append: bit-exact scatter of token rows into [blocks, block_size,
// kv_heads, head_dim] pages.
//
// A token row of one cache layer (kv_heads * head_dim elements) is contiguous
// both in the source and in the page, so the write is a row copy addressed by
// a slot index (physical_block * block_size + offset).  Rows are moved in
// 16-byte units when every pointer and the row size allow it; the payload is
// never converted, which makes the copy bit-exact for every dtype.
//
// Reference semantics:
//   single-token writer  tensorforge/kernels/triton_cache.py:23-63 (kernel),
//                        :68-133 (host contract: masked lanes store nothing)
//   multi-token append   tensorforge/cache/paged.py:212-235 (copy / index_put
//                        of T rows at positions start..start+T-1)
#include "tf_common.hpp"

namespace tf {
namespace {

// Source of the destination slot of row `r`.
struct TokenSlots {  // physical_blocks / block_offsets / active_mask (int32)
  const int32_t *physical_blocks;
  const int32_t *block_offsets;
  const int32_t *active_mask;
  int32_t block_size;
  __device__ __forceinline__ int64_t operator()(int64_t r) const {
    if (active_mask[r] == 0) return -1;
    const int32_t off = block_offsets[r];
    if (off < 0 || off >= block_size) return -1;
    return static_cast<int64_t>(physical_blocks[r]) * block_size + off;
  }
};

struct MappedSlots {  // int64 slot mapping, negative = padded lane
  const int64_t *slots;
  __device__ __forceinline__ int64_t operator()(int64_t r) const { return slots[r]; }
};

// Rows start..start+T-1 of one sequence through its block-table row:
// position p -> page table[p / block_size], offset p % block_size.  Entries
// outside the table or the cache are skipped.
struct RangeSlots {
  const int32_t *table;
  int32_t table_width;
  int32_t start;
  int32_t block_size;
  int32_t num_blocks;
  __device__ __forceinline__ int64_t operator()(int64_t r) const {
    const int64_t pos = start + r;
    const int64_t logical = pos / block_size;
    if (logical >= table_width) return -1;
    const int32_t page = table[logical];
    if (page < 0 || page >= num_blocks) return -1;
    return static_cast<int64_t>(page) * block_size + (pos - logical * block_size);
  }
};

// grid.x covers the 2 * row_units units of one row (K then V), grid.y rows.
template <typename Unit, typename SlotFn>
__global__ void __launch_bounds__(256)
kv_scatter_kernel(const Unit *__restrict__ keys, const Unit *__restrict__ values,
                  Unit *__restrict__ key_cache, Unit *__restrict__ value_cache,
                  SlotFn slot_of, int64_t row_units, int64_t num_slots) {
  const int64_t row = blockIdx.y;
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (unit >= 2 * row_units) return;
  const int64_t slot = slot_of(row);
  if (slot < 0 || slot >= num_slots) return;
  const bool is_value = unit >= row_units;
  const int64_t u = is_value ? unit - row_units : unit;
  const Unit *src = is_value ? values : keys;
  Unit *dst = is_value ? value_cache : key_cache;
  dst[slot * row_units + u] = src[row * row_units + u];
}

template <typename SlotFn>
int32_t launch_scatter(const void *keys, const void *values, void *key_cache,
                       void *value_cache, SlotFn slot_of, int64_t rows,
                       int64_t row_bytes, int64_t num_slots, hipStream_t stream,
                       const char *name) {
  if (rows == 0) return TF_SUCCESS;
  if (rows > 65535) return fail(TF_ERROR_UNSUPPORTED, "KV append supports at most 65535 rows per call");
  const uintptr_t align = reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(values) |
                          reinterpret_cast<uintptr_t>(key_cache) |
                          reinterpret_cast<uintptr_t>(value_cache) | static_cast<uintptr_t>(row_bytes);
  const int threads = 256;
  if (align % 16 == 0) {
    const int64_t units = row_bytes / 16;
    dim3 grid(static_cast<unsigned>((2 * units + threads - 1) / threads), static_cast<unsigned>(rows));
    hipLaunchKernelGGL((kv_scatter_kernel<uint4, SlotFn>), grid, dim3(threads), 0, stream,
                       static_cast<const uint4 *>(keys), static_cast<const uint4 *>(values),
                       static_cast<uint4 *>(key_cache), static_cast<uint4 *>(value_cache), slot_of,
                       units, num_slots);
  } else if (align % 4 == 0) {
    const int64_t units = row_bytes / 4;
    dim3 grid(static_cast<unsigned>((2 * units + threads - 1) / threads), static_cast<unsigned>(rows));
    hipLaunchKernelGGL((kv_scatter_kernel<uint32_t, SlotFn>), grid, dim3(threads), 0, stream,
                       static_cast<const uint32_t *>(keys), static_cast<const uint32_t *>(values),
                       static_cast<uint32_t *>(key_cache), static_cast<uint32_t *>(value_cache),
                       slot_of, units, num_slots);
  } else {
    const int64_t units = row_bytes / 2;
    dim3 grid(static_cast<unsigned>((2 * units + threads - 1) / threads), static_cast<unsigned>(rows));
    hipLaunchKernelGGL((kv_scatter_kernel<uint16_t, SlotFn>), grid, dim3(threads), 0, stream,
                       static_cast<const uint16_t *>(keys), static_cast<const uint16_t *>(values),
                       static_cast<uint16_t *>(key_cache), static_cast<uint16_t *>(value_cache),
                       slot_of, units, num_slots);
  }
  return check_launch(name);
}

int32_t check_geometry(const void *keys, const void *values, const void *key_cache,
                       const void *value_cache, int32_t kv_heads, int32_t head_dim,
                       int32_t num_blocks, int32_t block_size, int32_t dtype) {
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0 || block_size <= 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "cache dimensions must be positive");
  if (!keys || !values || !key_cache || !value_cache)
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  return TF_SUCCESS;
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_paged_kv_write_token(
    const void *keys, const void *values, void *key_cache, void *value_cache,
    const int32_t *physical_blocks, const int32_t *block_offsets,
    const int32_t *active_mask, int32_t batch, int32_t kv_heads, int32_t head_dim,
    int32_t num_blocks, int32_t block_size, int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (int32_t s = check_geometry(keys, values, key_cache, value_cache, kv_heads, head_dim,
                                 num_blocks, block_size, dtype))
    return s;
  if (batch < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "batch must be non-negative");
  if (batch > 0 && (!physical_blocks || !block_offsets || !active_mask))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null control vector");
  const int64_t row_bytes = static_cast<int64_t>(kv_heads) * head_dim * dtype_size(dtype);
  TokenSlots slots{physical_blocks, block_offsets, active_mask, block_size};
  return launch_scatter(keys, values, key_cache, value_cache, slots, batch, row_bytes,
                        static_cast<int64_t>(num_blocks) * block_size,
                        static_cast<hipStream_t>(stream), "paged_kv_write_token");
}

extern "C" int32_t tf_paged_kv_write_slots(
    const void *keys, const void *values, void *key_cache, void *value_cache,
    const int64_t *slot_mapping, int32_t tokens, int32_t kv_heads, int32_t head_dim,
    int32_t num_blocks, int32_t block_size, int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (int32_t s = check_geometry(keys, values, key_cache, value_cache, kv_heads, head_dim,
                                 num_blocks, block_size, dtype))
    return s;
  if (tokens < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "tokens must be non-negative");
  if (tokens > 0 && !slot_mapping) return fail(TF_ERROR_INVALID_ARGUMENT, "null slot mapping");
  const int64_t row_bytes = static_cast<int64_t>(kv_heads) * head_dim * dtype_size(dtype);
  MappedSlots slots{slot_mapping};
  return launch_scatter(keys, values, key_cache, value_cache, slots, tokens, row_bytes,
                        static_cast<int64_t>(num_blocks) * block_size,
                        static_cast<hipStream_t>(stream), "paged_kv_write_slots");
}

extern "C" int32_t tf_paged_kv_write_range(
    const void *keys, const void *values, void *key_cache, void *value_cache,
    const int32_t *block_table, int32_t table_width, int32_t start_position, int32_t tokens,
    int32_t kv_heads, int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t dtype,
    void *stream) {
  using namespace tf;
  clear_error();
  if (int32_t s = check_geometry(keys, values, key_cache, value_cache, kv_heads, head_dim,
                                 num_blocks, block_size, dtype))
    return s;
  if (tokens < 0 || start_position < 0 || table_width <= 0)
    return fail(TF_ERROR_INVALID_ARGUMENT,
                "tokens and start_position must be non-negative, table_width positive");
  if (tokens > 0 && !block_table) return fail(TF_ERROR_INVALID_ARGUMENT, "null block table");
  const int64_t row_bytes = static_cast<int64_t>(kv_heads) * head_dim * dtype_size(dtype);
  RangeSlots slots{block_table, table_width, start_position, block_size, num_blocks};
  return launch_scatter(keys, values, key_cache, value_cache, slots, tokens, row_bytes,
                        static_cast<int64_t>(num_blocks) * block_size,
                        static_cast<hipStream_t>(stream), "paged_kv_write_range");
}
