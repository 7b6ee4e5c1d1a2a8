// Fused RoPE + paged KV append: one launch per layer turns the fused QKV
// projection of a batch of tokens (one per decode lane, or a packed set of
// prompts) into the rotated query and writes the rotated key and the value
// of every active token into its cache page; optionally also the rotated key
// densely (prefill attention reads it).
//
// Input row b of `qkv` holds [q heads | k heads | v heads], head_dim each.
// RoPE uses the half-split rotation with per-dimension cos/sin tables
// indexed by the lane's position:
//   out[j]     = x[j] cos[j]     - x[j+D/2] sin[j]
//   out[j+D/2] = x[j+D/2] cos[j+D/2] + x[j] sin[j+D/2]        (j < D/2)
// computed in fp32 and rounded once to the storage type.
//
// Reference semantics this one launch replaces:
//   RoPE on q and k       tensorforge/model/layers.py:33-69
//                         (apply_batched_rotary_embedding, :57-69)
//   cache write           tensorforge/runtime/decode_bucket.py:448-458 ->
//                         tensorforge/kernels/triton_cache.py:23-63
//                         (masked lanes store nothing)
//   the .contiguous() copies of q, k and v at decode_bucket.py:449-450, 460
//   prefill RoPE + append runtime/prefill.py:99-115 (apply_rotary_embedding,
//                         then one write_layer per request)
#include "tf_common.hpp"

namespace tf {
namespace {

// One workgroup per lane.  Threads walk the (Hq + Hkv) * D/2 rotation pairs
// (consecutive threads take consecutive j, so loads and stores coalesce),
// then the Hkv * D value elements.
template <typename T>
__global__ void __launch_bounds__(256)
rope_kv_append_kernel(const T *__restrict__ qkv, int64_t row_stride,
                      const int64_t *__restrict__ positions, const T *__restrict__ cos_table,
                      const T *__restrict__ sin_table, int32_t table_rows,
                      T *__restrict__ query_out, T *__restrict__ key_out,
                      T *__restrict__ key_cache,
                      T *__restrict__ value_cache, const int32_t *__restrict__ physical_blocks,
                      const int32_t *__restrict__ block_offsets,
                      const int32_t *__restrict__ active_mask, int32_t query_heads,
                      int32_t kv_heads, int32_t head_dim, int32_t num_blocks,
                      int32_t block_size) {
  const int64_t b = blockIdx.x;
  const int32_t half = head_dim >> 1;
  int64_t pos = positions[b];
  // The host validates positions; clamping keeps a bad one inside the table.
  pos = pos < 0 ? 0 : (pos >= table_rows ? table_rows - 1 : pos);
  const T *row = qkv + b * row_stride;
  const T *cs = cos_table + pos * head_dim;
  const T *sn = sin_table + pos * head_dim;
  const int32_t page = physical_blocks[b];
  const int32_t offset = block_offsets[b];
  const bool store = active_mask[b] != 0 && page >= 0 && page < num_blocks && offset >= 0 &&
                     offset < block_size;
  const int64_t row_elems = static_cast<int64_t>(kv_heads) * head_dim;
  const int64_t slot = static_cast<int64_t>(page) * block_size + offset;
  T *q_row = query_out + b * static_cast<int64_t>(query_heads) * head_dim;

  const int32_t pairs = (query_heads + kv_heads) * half;
  for (int32_t i = threadIdx.x; i < pairs; i += blockDim.x) {
    const int32_t head = i / half;
    const int32_t j = i - head * half;
    const T *src = row + static_cast<int64_t>(head) * head_dim;
    const float x1 = to_float(src[j]);
    const float x2 = to_float(src[j + half]);
    const float o1 = rope_lo(x1, x2, to_float(cs[j]), to_float(sn[j]));
    const float o2 = rope_hi(x1, x2, to_float(cs[j + half]), to_float(sn[j + half]));
    const T r1 = from_float<T>(o1);
    const T r2 = from_float<T>(o2);
    if (head < query_heads) {
      T *dst = q_row + static_cast<int64_t>(head) * head_dim;
      dst[j] = r1;
      dst[j + half] = r2;
    } else {
      const int64_t kh = static_cast<int64_t>(head - query_heads) * head_dim;
      if (store) {
        T *dst = key_cache + slot * row_elems + kh;
        dst[j] = r1;
        dst[j + half] = r2;
      }
      if (key_out) {
        T *dst = key_out + b * row_elems + kh;
        dst[j] = r1;
        dst[j + half] = r2;
      }
    }
  }
  if (store) {
    const T *v = row + static_cast<int64_t>(query_heads + kv_heads) * head_dim;
    T *dst = value_cache + slot * row_elems;
    for (int32_t i = threadIdx.x; i < row_elems; i += blockDim.x) dst[i] = v[i];
  }
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_rope_kv_append(
    const void *qkv, int64_t qkv_row_stride, const int64_t *positions, const void *cos_table,
    const void *sin_table, int32_t table_rows, void *query_out, void *key_out, void *key_cache,
    void *value_cache, const int32_t *physical_blocks, const int32_t *block_offsets,
    const int32_t *active_mask, int32_t batch, int32_t query_heads, int32_t kv_heads,
    int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (batch < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "batch must be non-negative");
  if (query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || (head_dim & 1) || num_blocks <= 0 ||
      block_size <= 0 || table_rows <= 0)
    return fail(TF_ERROR_INVALID_ARGUMENT,
                "heads, blocks and table rows must be positive and head_dim even");
  if (query_heads % kv_heads)
    return fail(TF_ERROR_INVALID_ARGUMENT, "query_heads must be a multiple of kv_heads");
  if (qkv_row_stride < static_cast<int64_t>(query_heads + 2 * kv_heads) * head_dim)
    return fail(TF_ERROR_INVALID_ARGUMENT, "qkv row stride is shorter than the q, k, v heads");
  if (batch == 0) return TF_SUCCESS;
  if (!qkv || !positions || !cos_table || !sin_table || !query_out || !key_cache || !value_cache ||
      !physical_blocks || !block_offsets || !active_mask)
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const dim3 grid(static_cast<unsigned>(batch));
  const dim3 block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TF_ROPE_LAUNCH(T)                                                                     \
  hipLaunchKernelGGL((rope_kv_append_kernel<T>), grid, block, 0, s,                          \
                     static_cast<const T *>(qkv), qkv_row_stride, positions,                 \
                     static_cast<const T *>(cos_table), static_cast<const T *>(sin_table),   \
                     table_rows, static_cast<T *>(query_out), static_cast<T *>(key_out),     \
                     static_cast<T *>(key_cache),                                            \
                     static_cast<T *>(value_cache), physical_blocks, block_offsets,          \
                     active_mask, query_heads, kv_heads, head_dim, num_blocks, block_size)
  switch (dtype) {
    case TF_DTYPE_FLOAT32: TF_ROPE_LAUNCH(float); break;
    case TF_DTYPE_FLOAT16: TF_ROPE_LAUNCH(_Float16); break;
    default: TF_ROPE_LAUNCH(__bf16); break;
  }
#undef TF_ROPE_LAUNCH
  return check_launch("rope_kv_append");
}
