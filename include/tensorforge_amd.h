/*
 * tensorforge_amd.h -- C ABI of the MI355X (gfx950) batched-decode hot path.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream passed
 * as `void *` (a hipStream_t; NULL selects the default stream).  Kernels are
 * enqueued asynchronously on that stream; nothing here allocates, frees or
 * synchronises, so every call is safe inside HIP graph capture.  Tensors are
 * dense row-major (C-contiguous) in the layouts documented per function.
 *
 * Return value: TF_SUCCESS (0) or a nonzero tf_status; tf_last_error() then
 * holds a message for the calling thread.
 *
 * Reference interfaces replaced (Kakarottoooo/TensorForge, paths relative to
 * the repository root):
 *   tf_paged_gqa_decode*     tensorforge/kernels/triton_attention.py:326-518
 *                            (kernels :67-171 one-pass, :173-266 split,
 *                            :268-316 log-sum-exp reduce)
 *   tf_paged_kv_write_token  tensorforge/kernels/triton_cache.py:68-133
 *                            (kernel :23-63)
 *   tf_paged_kv_write_slots  tensorforge/cache/paged.py:221-235
 *                            (slot-mapping form of the multi-token scatter)
 *   tf_paged_kv_write_range  tensorforge/cache/paged.py:191-236
 *                            (PagedKVCache.write_layer through a table row)
 *   tf_rope_kv_append        tensorforge/model/layers.py:46-69 (RoPE)
 *                            + tensorforge/runtime/decode_bucket.py:448-458
 *                            (the decode step's cache write) and
 *                            runtime/prefill.py:99-115 (prefill's)
 *   tf_rms_norm              tensorforge/kernels/triton_ops.py:179-205
 *   tf_embedding_rms_norm    token feedback + embedding + first input norm
 *                            (runtime/decode_bucket.py:427-440)
 *   tf_residual_rms_norm     tensorforge/kernels/triton_ops.py:208-243
 *   tf_swiglu                tensorforge/kernels/triton_ops.py:246-260
 *   tf_linear_rows           the nn.Linear projections of the decode step
 *                            (tensorforge/model/layers.py:88-95, 144-146;
 *                            runtime/decode_bucket.py:441-447, 470, 500-505)
 *   tf_linear_partials,      the same projections at 17..64 rows, split over
 *   tf_linear_partials_sum   K into fp32 partials and their row sum
 *   tf_linear_stream         the same projections staged through LDS with
 *                            whole-row loads (direct or split-K partials)
 *   tf_linear_kstream        the same projections, K split over a 16-column
 *                            workgroup's wavefronts (narrow weights)
 *   tf_linear_kswiglu        its K-split form
 *   tf_linear_kstream_norm,  the same K-split projections fused with the
 *   tf_linear_kswiglu_norm   RMSNorm before them (triton_ops.py:179-205)
 *   tf_linear_kstream_residual  and with the residual add after them
 *                            (triton_ops.py:208-243)
 *   tf_linear_swiglu         the MLP's gate|up projection with its SwiGLU
 *                            (model/layers.py:144-158)
 *   tf_prefill_attention     prefill's causal attention (runtime/prefill.py:84-88, 109-118)
 *   tf_argmax_rows           greedy sampling, torch.argmax(logits, dim=-1)
 *                            (scheduler/continuous.py:265-275)
 *   tf_hbm_read_probe        measurement only: the read-rate ceiling the attention
 *                            roofline is compared with (the reference measures
 *                            its ceiling with a device copy,
 *                            tensorforge/benchmark/kernel_benchmark.py:176-192)
 *   tf_hbm_page_gather_probe measurement only: the rate of reading one attention
 *                            call's K/V pages and nothing else (no counterpart
 *                            in the reference)
 */
#ifndef TENSORFORGE_AMD_H_
#define TENSORFORGE_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Floating-point element types of the payload tensors. */
enum tf_dtype {
  TF_DTYPE_FLOAT32 = 0,
  TF_DTYPE_FLOAT16 = 1,
  TF_DTYPE_BFLOAT16 = 2
};

enum tf_status {
  TF_SUCCESS = 0,
  TF_ERROR_INVALID_ARGUMENT = 1, /* a size, pointer or dtype is out of range */
  TF_ERROR_UNSUPPORTED = 2,      /* valid request this build cannot serve   */
  TF_ERROR_LAUNCH = 3            /* the HIP runtime rejected a launch        */
};

/* Attention kernel families (tf_paged_gqa_decode_variant). */
enum tf_attention_variant {
  TF_ATTENTION_GENERIC = 0, /* any dtype, head_dim <= 256, group <= 64,
                               any block size                              */
  TF_ATTENTION_MFMA = 1     /* bf16/fp16, head_dim in {32,64,128},
                               group <= 16, block_size % 16 == 0, and
                               split_size % 32 == 0 when num_splits > 1    */
};

/* tf_paged_gqa_decode* flags.  FORCE_GENERIC selects the generic family.
 * Tuning fields of the MFMA grid kernel (0 selects the defaults):
 *   bits 8-15   wavefronts per kv head (heads x this <= 8, else 1)
 *   bits 20-23  kv heads per workgroup, which read the same token rows
 *               together (must divide kv_heads and be <= 8, else 1)
 *   bits 24-30  tokens per wavefront / 64; a row then uses ceil(its tokens
 *               / that) of the head's wavefronts (0: all)
 * Other bits (2, 4, 8, 64, 128 and bits 16-19) are rejected with
 * TF_ERROR_UNSUPPORTED.
 * VALU (the MFMA grid kernel's calls, head_dim 64, no RoPE) computes the
 * score and P.V products on the VALU -- packed two-element dot products
 * (v_dot2_f32_bf16 / _f16) and fp32 FMAs -- with the same grid, loads and
 * LDS staging: the comparison form for the MFMA products.
 * BALANCED (MFMA grid kernel, split-KV with the merge launch: num_splits >
 * batch, batch <= 64, split_counters null) sizes the partitions from the
 * rows' lengths on the device instead of using split_size for every row:
 * with total = the sum of the (clamped) lengths, every row is cut into
 * partitions of max(split_size, ceil32(ceil(total / (num_splits - batch))))
 * tokens, at most num_splits per group of kv heads (heads per workgroup)
 * over all rows together, and the launch is one compact grid of
 * (kv_heads / heads per workgroup) x num_splits workgroups that take those
 * partitions in row order.  Ragged
 * long rows then spread over the grid evenly where fixed partitions leave
 * most of it without work.  Partials land in slot j < ceil(len / partition)
 * of their row, as with fixed partitions; the merge recomputes the size. */
#define TF_ATTENTION_FLAG_FORCE_GENERIC 1
#define TF_ATTENTION_FLAG_VALU 16
#define TF_ATTENTION_FLAG_BALANCED 32
#define TF_ATTENTION_WAVES_PER_CU_SHIFT 8
#define TF_ATTENTION_HEADS_PER_WG_SHIFT 20
#define TF_ATTENTION_TOKENS_PER_WAVE_SHIFT 24

/* Message describing the last failure on the calling thread ("" if none). */
const char *tf_last_error(void);

/* Version of this ABI; bumped on any signature change or added entry point. */
int32_t tf_abi_version(void);

/* Which kernel family tf_paged_gqa_decode uses for these parameters
 * (a split_size that is not a multiple of 32 also selects the generic one). */
int32_t tf_paged_gqa_decode_variant(int32_t dtype, int32_t head_dim,
                                    int32_t group_size, int32_t block_size,
                                    int32_t flags);

/*
 * Paged GQA decode attention: one query token per sequence.
 *   query           [batch, query_heads, head_dim]            dtype
 *   key/value_cache [num_blocks, block_size, kv_heads, head_dim] dtype
 *   block_tables    [batch, table_width] int32 (physical page of each
 *                   logical page; entries outside [0, num_blocks) are skipped)
 *   context_lengths [batch] int32 (<= 0: the output row is written as zeros)
 *   output          [batch, query_heads, head_dim]            dtype
 * Query head h reads KV head h / (query_heads / kv_heads).  The context of a
 * row is split into num_splits partitions of split_size tokens; tokens past
 * num_splits * split_size or past table_width * block_size are ignored.
 * num_splits == 1 computes each row in one pass and the partial buffers may be
 * NULL.  Otherwise fp32 partials are written at index
 * (b * query_heads + h) * num_splits + s (partial_accumulator rows are
 * partial_row_stride floats apart) and merged by log-sum-exp; partial_capacity
 * is the number of partial rows the buffers hold.  scale multiplies q.k.
 * split_counters: NULL, or batch * kv_heads int32 counters that are zero
 * before the first call.  With counters the last workgroup of each
 * (row, kv head) merges the partials inside the split kernel (one launch)
 * and returns its counter to zero; without them a merge kernel follows.
 * Calls sharing partial buffers or counters must not overlap in time.
 * Replaces triton_attention.py:326-518.
 */
int32_t tf_paged_gqa_decode(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths, void *output,
    float *partial_max, float *partial_sum, float *partial_accumulator,
    int32_t *split_counters, int64_t partial_capacity, int32_t partial_row_stride,
    int32_t batch,
    int32_t query_heads, int32_t kv_heads, int32_t head_dim,
    int32_t num_blocks, int32_t block_size, int32_t table_width,
    int32_t split_size, int32_t num_splits, float scale, int32_t dtype,
    int32_t flags, void *stream);

/*
 * tf_paged_gqa_decode fused with the decode step's RoPE and KV append
 * (MFMA grid kernel only: bf16/fp16, head_dim 32/64/128, group <= 16,
 * block_size % 16 == 0).  Row b of `qkv` (qkv_row_stride
 * elements apart) holds [query heads | kv heads of k | kv heads of v],
 * head_dim each, unrotated.  Each workgroup rotates its query group at
 * positions[b] (half-split RoPE with the cos/sin tables [table_rows,
 * head_dim], positions clamped into the table, fp32 math rounded once, as
 * tf_rope_kv_append) and, when active_mask[b] != 0 and the slot
 * (append_pages[b], append_offsets[b]) lies in the cache, writes the row's
 * rotated k and its v into that slot before reading the row's tokens.
 * context_lengths count the new token; everything else is as in
 * tf_paged_gqa_decode.  Replaces the RoPE, cache write and attention of the
 * decode step (model/layers.py:57-69; runtime/decode_bucket.py:448-469).
 */
int32_t tf_paged_gqa_decode_rope_append(
    const void *qkv, int64_t qkv_row_stride, const int64_t *positions,
    const void *cos_table, const void *sin_table, int32_t table_rows,
    void *key_cache, void *value_cache, const int32_t *append_pages,
    const int32_t *append_offsets, const int32_t *active_mask,
    const int32_t *block_tables, const int32_t *context_lengths, void *output,
    float *partial_max, float *partial_sum, float *partial_accumulator,
    int32_t *split_counters, int64_t partial_capacity, int32_t partial_row_stride,
    int32_t batch, int32_t query_heads, int32_t kv_heads, int32_t head_dim,
    int32_t num_blocks, int32_t block_size, int32_t table_width,
    int32_t split_size, int32_t num_splits, float scale, int32_t dtype,
    int32_t flags, void *stream);

/*
 * tf_paged_gqa_decode without a caller workspace: no partial buffers and no
 * counters are passed, and nothing is allocated.  No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Split partials (num_splits > 1: batch * query_heads *
 * num_splits rows of next_pow2(head_dim) + 2 floats) live in a fixed
 * device array of TF_NOALLOC_SCRATCH_BYTES that each GPU holds until the
 * process ends; larger requests fail with TF_ERROR_INVALID_ARGUMENT.  The
 * split stage writes every partial the merge reads, so the array needs no
 * clearing.  All calls on one GPU share that array: calls that overlap in
 * time on one GPU race.  There are no arrival counters (the merge is a
 * launch); other arguments are as in tf_paged_gqa_decode, whose kernels it
 * runs, with the same results.
 */
#define TF_NOALLOC_SCRATCH_BYTES (8LL << 20)
int32_t tf_paged_gqa_decode_noalloc(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths, void *output,
    int32_t batch, int32_t query_heads, int32_t kv_heads, int32_t head_dim,
    int32_t num_blocks, int32_t block_size, int32_t table_width,
    int32_t split_size, int32_t num_splits, float scale, int32_t dtype,
    int32_t flags, void *stream);

/*
 * First stage of tf_paged_gqa_decode alone (num_splits >= 1): writes the
 * partials of every non-empty split.  Partial max values are base-2
 * logarithms of the unnormalised scores (score * scale * log2(e)).
 * Replaces the split kernel launch, triton_attention.py:433-460.
 */
int32_t tf_paged_gqa_decode_partials(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths,
    float *partial_max, float *partial_sum, float *partial_accumulator,
    int64_t partial_capacity, int32_t partial_row_stride, int32_t batch,
    int32_t query_heads, int32_t kv_heads, int32_t head_dim,
    int32_t num_blocks, int32_t block_size, int32_t table_width,
    int32_t split_size, int32_t num_splits, float scale, int32_t dtype,
    int32_t flags, void *stream);

/*
 * Second stage: log-sum-exp merge of the partials of each (row, query head)
 * into output.  Reads only the ceil(context / split_size) splits a row owns.
 * Replaces the reduce kernel launch, triton_attention.py:461-474.
 */
int32_t tf_paged_gqa_decode_merge(
    const float *partial_max, const float *partial_sum,
    const float *partial_accumulator, const int32_t *context_lengths,
    void *output, int64_t partial_capacity, int32_t partial_row_stride,
    int32_t batch, int32_t query_heads, int32_t head_dim, int32_t split_size,
    int32_t num_splits, int32_t max_tokens, int32_t dtype, void *stream);

/*
 * One KV token per batch lane:
 *   if active_mask[b] != 0:
 *     key_cache[physical_blocks[b], block_offsets[b], :, :] = keys[b]
 *     value_cache[...] = values[b]
 * keys/values [batch, kv_heads, head_dim]; caches as in tf_paged_gqa_decode.
 * A bit-exact copy; lanes whose destination lies outside the cache are
 * skipped.  Replaces triton_cache.py:68-133.
 */
int32_t tf_paged_kv_write_token(
    const void *keys, const void *values, void *key_cache, void *value_cache,
    const int32_t *physical_blocks, const int32_t *block_offsets,
    const int32_t *active_mask, int32_t batch, int32_t kv_heads,
    int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t dtype,
    void *stream);

/*
 * Multi-token append through a slot mapping:
 *   slot = slot_mapping[t] (= physical_block * block_size + offset)
 *   if 0 <= slot < num_blocks * block_size: cache token row `slot` = row t
 * keys/values [tokens, kv_heads, head_dim]; slot -1 marks padded lanes.
 * A bit-exact copy.  Replaces the index_put of cache/paged.py:221-235.
 */
int32_t tf_paged_kv_write_slots(
    const void *keys, const void *values, void *key_cache, void *value_cache,
    const int64_t *slot_mapping, int32_t tokens, int32_t kv_heads,
    int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t dtype,
    void *stream);

/*
 * Append of `tokens` rows for one sequence at logical positions
 * start_position .. start_position + tokens - 1 through the sequence's
 * block-table row (table_width int32 entries):
 *   cache token row (block_table[p / block_size], p % block_size) = row p - start
 * keys/values [tokens, kv_heads, head_dim]; positions whose table entry is
 * missing or outside the cache are skipped.  A bit-exact copy, one launch
 * with no host-side index construction.  Replaces
 * PagedKVCache.write_layer, cache/paged.py:212-235 (single-token copy_ and
 * multi-token index_put).
 */
int32_t tf_paged_kv_write_range(
    const void *keys, const void *values, void *key_cache, void *value_cache,
    const int32_t *block_table, int32_t table_width, int32_t start_position,
    int32_t tokens, int32_t kv_heads, int32_t head_dim, int32_t num_blocks,
    int32_t block_size, int32_t dtype, void *stream);

/*
 * RoPE fused with the paged KV append (a decode step's lanes, or the packed
 * tokens of several prompts).  qkv [batch, row] with
 * row stride qkv_row_stride elements holds [q heads | k heads | v heads]
 * (head_dim each); cos_table/sin_table [table_rows, head_dim] in the same
 * dtype; positions int64 [batch] (clamped into the table).  Writes the
 * rotated query to query_out [batch, query_heads, head_dim] for every lane,
 * the rotated key to key_out [batch, kv_heads, head_dim] when key_out is not
 * NULL, and for lanes with active_mask != 0 the rotated key and the value
 * into cache token row (physical_blocks[b], block_offsets[b]).  Rotation
 * (half-split): out[j] = x[j] cos[j] - x[j+D/2] sin[j],
 * out[j+D/2] = x[j+D/2] cos[j+D/2] + x[j] sin[j+D/2], fp32 arithmetic,
 * one rounding.  Replaces apply_batched_rotary_embedding
 * (model/layers.py:57-69) and the write at runtime/decode_bucket.py:448-458
 * (kernels/triton_cache.py:23-63), with their .contiguous() copies; for
 * prefill, apply_rotary_embedding and the per-request write_layer loop of
 * runtime/prefill.py:99-115.
 */
int32_t tf_rope_kv_append(
    const void *qkv, int64_t qkv_row_stride, const int64_t *positions,
    const void *cos_table, const void *sin_table, int32_t table_rows,
    void *query_out, void *key_out, void *key_cache, void *value_cache,
    const int32_t *physical_blocks, const int32_t *block_offsets,
    const int32_t *active_mask, int32_t batch, int32_t query_heads,
    int32_t kv_heads, int32_t head_dim, int32_t num_blocks, int32_t block_size,
    int32_t dtype, void *stream);

/*
 * The decode step's input rows and the first layer's RMSNorm in one launch:
 * row b takes token id = token_state[source_lanes[b]] when source_lanes[b]
 * >= 0 (the token its lane sampled last step) and host_tokens[b] otherwise
 * (int64 arrays; lane and token indices are clamped to token_state_len and
 * vocab), copies embedding[id] (a [vocab, columns] table) to x_output[b] and
 * writes RMSNorm(x) with `weight` to norm_output[b] -- bit for bit the
 * gather followed by tf_rms_norm.  Replaces the token feedback, embedding
 * lookup and first input norm of the decode step
 * (tensorforge/runtime/decode_bucket.py:427-440; the norm
 * tensorforge/kernels/triton_ops.py:179-205).
 */
int32_t tf_embedding_rms_norm(const int64_t *token_state, int64_t token_state_len,
                              const int64_t *source_lanes, const int64_t *host_tokens,
                              const void *embedding, int64_t vocab, const void *weight,
                              void *x_output, void *norm_output, int64_t rows, int32_t columns,
                              float eps, int32_t dtype, void *stream);

/*
 * Row-wise RMSNorm over [rows, columns]: y = x * rsqrt(mean(x^2) + eps) * w,
 * fp32 arithmetic, one rounding.  columns <= 16384.
 * Replaces triton_ops.py:179-205.
 */
int32_t tf_rms_norm(const void *inputs, const void *weight, void *output,
                    int64_t rows, int32_t columns, float eps, int32_t dtype,
                    void *stream);

/*
 * s = x + r in fp32; residual_output = round(s);
 * norm_output = round(s * rsqrt(mean(s^2) + eps) * w) (normalises the fp32
 * sum).  Replaces triton_ops.py:208-243.
 */
int32_t tf_residual_rms_norm(const void *inputs, const void *residual,
                             const void *weight, void *residual_output,
                             void *norm_output, int64_t rows, int32_t columns,
                             float eps, int32_t dtype, void *stream);

/*
 * tf_residual_rms_norm with the inputs given as fp32 split-K partials
 * (dense [splits, rows, columns], as tf_linear_partials writes them):
 *   inputs[r][j] = round(sum_s partials[s][r][j])
 * then exactly tf_residual_rms_norm.  Fuses the K-slice sum of the o and
 * down projections into the norm that consumes them (the reference runs
 * the torch GEMM, then residual_rms_norm: runtime/decode_bucket.py:470-483,
 * 505-515; triton_ops.py:208-243).
 */
int32_t tf_residual_rms_norm_partials(const float *partials, int32_t splits,
                                      const void *residual, const void *weight,
                                      void *residual_output, void *norm_output,
                                      int64_t rows, int32_t columns, float eps,
                                      int32_t dtype, void *stream);

/*
 * Elementwise SwiGLU: output = g * sigmoid(g) * u in fp32, one rounding.
 * Replaces triton_ops.py:246-260.
 */
int32_t tf_swiglu(const void *gate, const void *up, void *output,
                  int64_t numel, int32_t dtype, void *stream);

/*
 * SwiGLU over a fused gate|up projection: row r of gate_up (row stride
 * gate_up_row_stride elements) holds gate[0..columns) then up[0..columns);
 * output[r, c] = g * sigmoid(g) * u with the arithmetic of tf_swiglu.  No
 * reference counterpart: it lets the decode step run the gate and up
 * projections (tensorforge/model/layers.py:146-158, two GEMMs there) as one
 * GEMM over stacked weights.
 */
int32_t tf_swiglu_rows(const void *gate_up, int64_t gate_up_row_stride,
                       void *output, int64_t output_row_stride, int64_t rows,
                       int32_t columns, int32_t dtype, void *stream);

/*
 * Greedy sampling: out[r] = argmax over c < columns of logits[r * row_stride
 * + c] for r < rows (fp32, fp16 or bf16; out int64) -- torch.argmax(logits,
 * dim=-1) as the continuous scheduler applies it to a step's logits
 * (tensorforge/scheduler/continuous.py:265-275): the first index of the
 * largest value, a NaN counting as larger than every number.  columns >= 1,
 * row_stride >= columns (elements).
 */
int32_t tf_argmax_rows(const void *logits, int64_t row_stride, int32_t rows, int32_t columns,
                       int32_t dtype, int64_t *out, void *stream);

/*
 * Decode-shaped linear layer y[m, n] = x[m, k] . weight[n, k]^T (no bias),
 * fp16 or bf16, fp32 accumulation, one rounding; m <= 64, k a multiple of
 * 32, x and weight rows 16-byte aligned (strides in elements).  K is split
 * over waves_per_tile wavefronts per 16-column tile (0 = chosen from the
 * shape).  Replaces the torch GEMM of the reference's nn.Linear projections
 * at decode batch sizes (model/layers.py:88-95, 144-146).
 */
int32_t tf_linear_rows(const void *x, int64_t x_row_stride, const void *weight,
                       int64_t weight_row_stride, void *y, int64_t y_row_stride,
                       int32_t m, int32_t n, int32_t k, int32_t waves_per_tile,
                       int32_t dtype, void *stream);

/*
 * Split-K form of the same product for up to 64 rows:
 *   partials[s][i][j] = sum over k in slice s of x[i][k] * weight[j][k]  (fp32)
 * The K / 32 k-steps are dealt into `splits` contiguous non-empty slices
 * (splits must be in [1, K / 32] and leave no slice empty); partials is
 * dense [splits, m, n] fp32.  K % 32 == 0, 16-byte aligned rows, fp16/bf16.
 * Replaces the torch GEMM of the decode projections
 * (tensorforge/model/layers.py:88-95, 144-146) at 17..64 rows.
 */
int32_t tf_linear_partials(const void *x, int64_t x_row_stride, const void *weight,
                           int64_t weight_row_stride, float *partials, int32_t m,
                           int32_t n, int32_t k, int32_t splits, int32_t dtype,
                           void *stream);

/*
 * Weight-streaming form of the same product for up to 64 rows: with
 * partials == NULL and splits == 1, y[i][j] = round(sum_k x[i][k] *
 * weight[j][k]) into fp16/bf16 rows of y; with a partials buffer, the
 * fp32 slice sums of tf_linear_partials (same slices, same [splits, m, n]
 * layout).  Operands are staged through LDS with whole-row loads.  K % 32
 * == 0, 16-byte aligned x and weight rows.  Replaces the torch GEMM of the
 * decode projections (tensorforge/model/layers.py:88-95, 144-146) as the
 * decode step calls them (tensorforge/runtime/decode_bucket.py:441-447,
 * 470, 500-505).
 */
int32_t tf_linear_stream(const void *x, int64_t x_row_stride, const void *weight,
                         int64_t weight_row_stride, void *y, int64_t y_row_stride,
                         float *partials, int32_t m, int32_t n, int32_t k, int32_t splits,
                         int32_t dtype, void *stream);

/*
 * y = round(x @ weight^T) for up to 64 rows with K split over the four
 * wavefronts of a 16-column workgroup, each staging its k chunks of x and
 * weight through LDS with whole-row loads: the form for weights with few
 * 64-column tiles (a 2560-row qkv projection).  K % 32 == 0, 16-byte aligned
 * x and weight rows, fp16/bf16.  Replaces the torch GEMM of the decode
 * projections (tensorforge/model/layers.py:88-95) as the decode step calls
 * them (tensorforge/runtime/decode_bucket.py:441-447).
 */
int32_t tf_linear_kstream(const void *x, int64_t x_row_stride, const void *weight,
                          int64_t weight_row_stride, void *y, int64_t y_row_stride, int32_t m,
                          int32_t n, int32_t k, int32_t dtype, void *stream);

/*
 * tf_linear_swiglu's result (the stacked gate|up projection and its SwiGLU,
 * bit for bit tf_linear_kstream of the stacked weight followed by
 * tf_swiglu_rows) with K split over the four wavefronts of a workgroup of
 * 16 activation columns: the form for 33..64 rows, where x is large.
 */
int32_t tf_linear_kswiglu(const void *x, int64_t x_row_stride, const void *gate_up_weight,
                          int64_t weight_row_stride, void *y, int64_t y_row_stride, int32_t m,
                          int32_t intermediate, int32_t k, int32_t dtype, void *stream);

/*
 * tf_linear_kstream with the RMSNorm of x's rows applied to the product:
 *   y[i][j] = round(rsqrt(mean_k(x[i][k]^2) + eps) * (x[i] . w'[j]))
 * for a weight w' whose columns carry the norm's gain (w'[j][k] =
 * round(w[j][k] * gain[k]), the caller folds it once).  Replaces the
 * reference's RMSNorm (tensorforge/kernels/triton_ops.py:179-205) followed
 * by the projection (model/layers.py:88-95) -- the same product with the
 * gain rounded into the weight instead of into the normalised row; no
 * normalised x is written.  eps > 0.
 */
int32_t tf_linear_kstream_norm(const void *x, int64_t x_row_stride, const void *weight,
                               int64_t weight_row_stride, void *y, int64_t y_row_stride, int32_t m,
                               int32_t n, int32_t k, float eps, int32_t dtype, void *stream);

/*
 * tf_linear_kswiglu under the same row norm: both products of row i are
 * scaled by rsqrt(mean_k(x[i][k]^2) + eps) before the activation, the
 * stacked weight carrying the norm's gain.  Replaces the reference's
 * post-attention RMSNorm followed by the MLP's gate and up projections and
 * SwiGLU (triton_ops.py:179-205; model/layers.py:144-158).  At 49-64 rows
 * with k = 2048 (and 2048-8192 intermediate columns) the launch keeps each
 * workgroup's 32 rows of x in LDS and streams only the weight; the results
 * are the same bits either way.
 */
int32_t tf_linear_kswiglu_norm(const void *x, int64_t x_row_stride, const void *gate_up_weight,
                               int64_t weight_row_stride, void *y, int64_t y_row_stride, int32_t m,
                               int32_t intermediate, int32_t k, float eps, int32_t dtype,
                               void *stream);

/*
 * tf_linear_kstream added to the residual stream:
 *   y[i][j] = round(round(x[i] . w[j]) + residual[i][j])
 * -- the residual output of the reference's residual_rms_norm
 * (triton_ops.py:208-243) over the projection (the o / down projections of
 * runtime/decode_bucket.py:470-474, 505), bit for bit; the norm itself is
 * left to the consumer (tf_linear_kstream_norm).  y may not alias residual.
 */
int32_t tf_linear_kstream_residual(const void *x, int64_t x_row_stride, const void *weight,
                                   int64_t weight_row_stride, const void *residual,
                                   int64_t residual_row_stride, void *y, int64_t y_row_stride,
                                   int32_t m, int32_t n, int32_t k, int32_t dtype, void *stream);

/*
 * The MLP's stacked gate|up projection and its SwiGLU in one launch:
 *   y[i][j] = round(swiglu(round(x[i] . w[j]), round(x[i] . w[intermediate + j])))
 * for j < intermediate, with gate_up_weight stacking the gate rows
 * [0, intermediate) over the up rows [intermediate, 2 * intermediate) and
 * swiglu(g, u) = g * sigmoid(g) * u in fp32 -- bit for bit
 * tf_linear_stream of the stacked weight followed by tf_swiglu_rows.  Up to
 * 64 rows, K % 32 == 0, 16-byte aligned x and weight rows.  Replaces
 * silu(gate(x)) * up(x) of the MLP (tensorforge/model/layers.py:144-158;
 * the activation tensorforge/kernels/triton_ops.py:246-260) as the decode
 * step calls it (tensorforge/runtime/decode_bucket.py:500-505).
 */
int32_t tf_linear_swiglu(const void *x, int64_t x_row_stride, const void *gate_up_weight,
                         int64_t weight_row_stride, void *y, int64_t y_row_stride, int32_t m,
                         int32_t intermediate, int32_t k, int32_t dtype, void *stream);

/*
 * y[i][j] = round(sum_s partials[s][i][j]) into fp16/bf16 rows of y
 * (n and y_row_stride multiples of 4, 16-byte aligned buffers).  With
 * tf_linear_partials it is the projection x @ weight^T with fp32
 * accumulation and one rounding, as torch's GEMM computes it.
 */
int32_t tf_linear_partials_sum(const float *partials, int32_t splits, int32_t m,
                               int32_t n, void *y, int64_t y_row_stride,
                               int32_t dtype, void *stream);

/*
 * Causal GQA attention over packed prompts (prefill).  Token rows:
 *   q [T, query_heads * head_dim], k and v [T, kv_heads * head_dim] (row
 *   strides in elements), output [T, query_heads * head_dim].
 * tiles [num_tiles][3] int32: (first query token i0, prompt start s, prompt
 * end e) of each 64-token query block, s <= i0 < e, i0 - s a multiple of 64;
 * the block's tokens [i0, min(i0 + 64, e)) attend to [s, token] of their
 * prompt.  Heaviest blocks first runs best.  fp16/bf16, head_dim 32/64/128,
 * groups of 1..16 query heads per kv head; heads_per_wave (0: default)
 * picks how many of a group's heads one wavefront serves.  Replaces the
 * masked SDPA of prefill (runtime/prefill.py:84-88, 109-118).
 */
int32_t tf_prefill_attention(const void *q, int64_t q_row_stride, const void *k,
                             int64_t k_row_stride, const void *v, int64_t v_row_stride,
                             void *output, int64_t output_row_stride,
                             const int32_t *tiles, int32_t num_tiles,
                             int32_t query_heads, int32_t kv_heads, int32_t head_dim,
                             float scale, int32_t heads_per_wave, int32_t dtype,
                             void *stream);

/*
 * Measurement only: stream `bytes` (a positive multiple of 16) of the
 * 16-byte aligned `buffer` from HBM with 16-byte nontemporal loads.
 * `workgroups` workgroups of `waves` (1..16) wavefronts each read one
 * contiguous slice, `loads` (2, 4 or 8) loads in flight per lane.  `sink` is
 * one uint32 the kernel may write (so the loads are kept).  Timing it gives
 * the attainable read rate the attention kernels are compared with.
 */
int32_t tf_hbm_read_probe(const void *buffer, int64_t bytes, int32_t workgroups,
                          int32_t waves, int32_t loads, uint32_t *sink, void *stream);

/*
 * Measurement only: read every byte of the K and V pages listed in `pages`
 * (npages physical page ids; ids outside [0, num_blocks) are skipped), each
 * page `page_bytes` (a positive multiple of 1024) in both caches, with
 * 16-byte nontemporal loads: `workgroups` workgroups of `waves` (1..16)
 * wavefronts, each wavefront an equal contiguous range of the list.  No
 * compute and no output besides the `sink` word.  Timing it over the page
 * list of an attention call gives the attainable rate of that call's own
 * scattered-page access pattern.  No counterpart in the reference.
 */
int32_t tf_hbm_page_gather_probe(const void *key_cache, const void *value_cache,
                                 const int32_t *pages, int32_t npages, int64_t page_bytes,
                                 int32_t num_blocks, int32_t workgroups, int32_t waves,
                                 uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TENSORFORGE_AMD_H_ */
