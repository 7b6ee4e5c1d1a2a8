// Paged GQA decode attention for gfx950.
//
// Work unit: one workgroup per (split, kv_head, sequence).  The workgroup
// serves the whole query group of its KV head, so every K/V page byte is read
// from HBM once per call (the reference launches one program per *query*
// head and re-reads each page group-size times,
// tensorforge/kernels/triton_attention.py:99-102,481).  Tokens are visited up
// to the sequence's own device-side length, not up to the host bucket
// (reference loops to the pow2 bucket, :121), and sequences of length <= 0
// produce zero rows without touching the cache.
//
// Two kernel families share one output/partial format:
//
//  * MFMA (bf16/fp16, head_dim in {32,64,128}, group <= 16).  Each wavefront
//    walks 32-token chunks of its split.  Scores S^T[token, head] come from
//    v_mfma_f32_16x16x32 with the K tile loaded straight from HBM as the A
//    operand (lane = token row, 8 contiguous head_dim elements = one 16-byte
//    load) and the query group as the B operand (heads padded to 16 columns
//    with zeros).  The online softmax runs on the accumulator layout, where
//    a lane owns one head, so the running max/sum and the rescale of the
//    output accumulator are lane-local.  P.V uses the same instruction with
//    V^T as the A operand: the V rows are stored token-major into a
//    per-wavefront LDS tile exactly as loaded, and ds_read_b64_tr_b16 reads
//    them back transposed (lane = output dimension, 4 consecutive tokens),
//    two reads per 16-dimension block; P (converted to the storage type) is
//    already in the B-operand layout.  K/V for the next chunk are loaded
//    before the current chunk is computed (two chunks in flight per wave).
//    Several wavefronts of a workgroup may share a (row, kv head, split),
//    taking its chunks round-robin, and merge their (max, sum, acc) states
//    in LDS (for wide batches the whole row is one split: one pass, no
//    partials).  With arrival counters the last workgroup of a (row, kv
//    head) to finish merges the split partials in the same launch.
//
//  * Generic (any dtype, head_dim <= 256, group <= 64, any page size).  A
//    straightforward LDS-tiled implementation kept for fp32 and unusual
//    shapes; it is the accuracy reference path on the GPU (fp32 math
//    throughout).
//
// Softmax runs in base 2: scores are multiplied by scale*log2(e) and
// exponentiated with exp2, which is the native v_exp_f32.  Partial maxima are
// therefore base-2 values; only tf_paged_gqa_decode_merge reads them.
//
// Reference semantics:
//   one-pass kernel   triton_attention.py:67-171 (online softmax :116-161)
//   split kernel      triton_attention.py:173-266 (partials :260-266)
//   reduce kernel     triton_attention.py:268-316 (LSE merge :288-316)
//   oracle            kernels/reference.py:46-93
#include <mutex>
#include <type_traits>

#include "tf_common.hpp"

namespace tf {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// 2^x with the native v_exp_f32 (results below 2^-126 flush to zero, which
// is harmless for softmax weights; exp2(-inf) = 0).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

struct AttnParams {
  const void *query;
  const void *key_cache;
  const void *value_cache;
  const int32_t *block_tables;
  const int32_t *context_lengths;
  void *output;
  float *partial_max;
  float *partial_sum;
  float *partial_acc;
  int32_t *split_counters;  // per (row, kv head) arrival counters, or null
  int32_t batch;
  int32_t query_heads;
  int32_t kv_heads;
  int32_t group;
  int32_t head_dim;
  int32_t num_blocks;
  int32_t block_size;
  int32_t page_shift;  // log2(block_size) when a power of two, else -1
  int32_t table_width;
  int32_t split_size;
  int32_t num_splits;
  int32_t partial_stride;
  int32_t max_tokens;  // min(num_splits * split_size, table_width * block_size)
  int64_t partial_rows;    // rows the partial buffers hold
  int32_t heads_per_wg;    // MFMA grid kernel: kv heads served by one workgroup
  int32_t waves_per_head;  // MFMA grid kernel: wavefronts sharing one kv head
  int32_t tokens_per_wave; // MFMA grid kernel: > 0 uses ceil(tokens / this) of them per row
  int32_t balanced;        // MFMA grid kernel: partition size from the lengths (FLAG_BALANCED)
  float scale_log2;
  // Fused RoPE + append (MFMA grid kernel, tf_paged_gqa_decode_rope_append):
  // the query group is rotated from row b of `rope_qkv` ([q heads | k heads
  // | v heads], head_dim each) instead of read from `query`, and the row's
  // new token (rotated k, v) is written to its page slot before the row's
  // tokens are read.  Null for the plain call.
  const void *rope_qkv;
  int64_t rope_row_stride;
  const int64_t *rope_positions;
  const void *rope_cos;
  const void *rope_sin;
  int32_t rope_table_rows;
  const int32_t *append_pages;
  const int32_t *append_offsets;
  const int32_t *append_active;
};

__device__ __forceinline__ int32_t clamp_context(const AttnParams &p, int32_t b) {
  int32_t ctx = p.context_lengths[b];
  if (ctx < 0) ctx = 0;
  if (ctx > p.max_tokens) ctx = p.max_tokens;
  return ctx;
}

// Integer wavefront reductions by DPP lane moves within each 16-lane row and
// lane reads across the four rows (no LDS-routed shuffles; the whole
// wavefront must be active).  A DPP source lane outside the row reads 0.
template <int CTRL>
__device__ __forceinline__ int32_t dpp_int(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
// Sum over the 64 lanes (every lane gets it): quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror and row_mirror give each lane its row's sum.
__device__ __forceinline__ int32_t wave64_isum(int32_t v) {
  v += dpp_int<0xb1>(v);
  v += dpp_int<0x4e>(v);
  v += dpp_int<0x141>(v);
  v += dpp_int<0x140>(v);
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}
// Inclusive prefix sum over lanes 0..63: row_shr 1, 2, 4, 8 within each row
// (Hillis-Steele), then the earlier rows' totals added.
__device__ __forceinline__ int32_t wave64_iscan(int32_t v) {
  v += dpp_int<0x111>(v);
  v += dpp_int<0x112>(v);
  v += dpp_int<0x114>(v);
  v += dpp_int<0x118>(v);
  const int32_t r0 = __builtin_amdgcn_readlane(v, 15);
  const int32_t r01 = r0 + __builtin_amdgcn_readlane(v, 31);
  const int32_t r012 = r01 + __builtin_amdgcn_readlane(v, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return v + (row == 0 ? 0 : (row == 1 ? r0 : (row == 2 ? r01 : r012)));
}

// Partition size of a balanced split-KV call (TF_ATTENTION_FLAG_BALANCED),
// the same in every workgroup and in the merge: with total = the sum of the
// batch's clamped lengths, max(split_size, ceil32(ceil(total / (num_splits
// - batch)))), capped at the largest length a row can have.  A nonempty
// row of length L then needs ceil(L / size) <= L / size + 1 partitions, so
// the rows together need at most total / size + batch <= num_splits.
// Called by a whole wavefront (batch <= 64, num_splits > batch); lane b <
// batch returns row b's clamped length in `len` (0 on the other lanes).
__device__ __forceinline__ int32_t balanced_partition(const int32_t *lengths, int32_t batch,
                                                      int32_t max_tokens, int32_t split_size,
                                                      int32_t num_splits, int32_t &len) {
  const int lane = threadIdx.x & 63;
  int32_t v = lane < batch ? lengths[lane] : 0;
  v = v < 0 ? 0 : (v > max_tokens ? max_tokens : v);
  len = v;
  // The lengths' sum in two 16-bit halves (each half's sum over 64 lanes
  // fits in 32 bits), reduced with DPP moves and lane reads.
  const int64_t total = (static_cast<int64_t>(wave64_isum(v >> 16)) << 16) + wave64_isum(v & 0xffff);
  const int64_t spare = num_splits - batch;
  int64_t size = ((total + spare - 1) / spare + 31) / 32 * 32;
  const int64_t longest = (static_cast<int64_t>(max_tokens) + 31) / 32 * 32;
  if (size > longest) size = longest;
  if (size < split_size) size = split_size;
  return __builtin_amdgcn_readfirstlane(static_cast<int32_t>(size));
}

// Row and partition of slot `slot` of a balanced call: the rows'
// partitions, ceil(length / size) each, are numbered in row order, and
// slots past the last one have none (row -1).  Whole-wavefront call; the
// results are wavefront-uniform.
__device__ __forceinline__ void balanced_slot(const AttnParams &p, int32_t slot, int32_t &size,
                                              int32_t &row, int32_t &part) {
  int32_t len;
  size = balanced_partition(p.context_lengths, p.batch, p.max_tokens, p.split_size,
                            p.num_splits, len);
  const int32_t n = (len + size - 1) / size;
  const int32_t incl = wave64_iscan(n);  // inclusive prefix sum of the partition counts over rows (lanes)
  const int32_t excl = incl - n;
  const unsigned long long hit = __ballot(slot >= excl && slot < incl);
  row = -1;
  part = 0;
  if (hit != 0) {
    const int r = __builtin_ctzll(hit);
    row = r;
    part = slot - __builtin_amdgcn_readlane(excl, r);
  }
  row = __builtin_amdgcn_readfirstlane(row);
  part = __builtin_amdgcn_readfirstlane(part);
}

// Element offset of token `t` of sequence row `table` for kv head 0, or -1
// when the token's page entry is outside the cache.
__device__ __forceinline__ int64_t token_offset(const AttnParams &p, const int32_t *table,
                                                int32_t t) {
  int32_t logical, offset;
  if (p.page_shift >= 0) {
    logical = t >> p.page_shift;
    offset = t & (p.block_size - 1);
  } else {
    logical = t / p.block_size;
    offset = t - logical * p.block_size;
  }
  const int32_t page = table[logical];
  if (page < 0 || page >= p.num_blocks) return -1;
  return (static_cast<int64_t>(page) * p.block_size + offset) *
         static_cast<int64_t>(p.kv_heads) * p.head_dim;
}

// True when no separate merge launch follows the split stage: one pass, or
// split mode with arrival counters (the last workgroup of a row merges).
__device__ __forceinline__ bool writes_output(const AttnParams &p) {
  return p.num_splits == 1 || p.split_counters != nullptr;
}

// Rows of length zero produce zeros, written by their split-0 workgroup
// whenever no merge launch follows: query heads [qh0, qh0 + nheads).
template <typename T>
__device__ void zero_rows(const AttnParams &p, int32_t b, int32_t qh0, int32_t nheads) {
  if (!writes_output(p)) return;
  T *out = static_cast<T *>(p.output) +
           (static_cast<int64_t>(b) * p.query_heads + qh0) * p.head_dim;
  for (int i = threadIdx.x; i < nheads * p.head_dim; i += blockDim.x) out[i] = from_float<T>(0.f);
}

template <typename T>
__device__ __forceinline__ T *output_row(const AttnParams &p, int32_t b, int32_t qh) {
  return static_cast<T *>(p.output) + (static_cast<int64_t>(b) * p.query_heads + qh) * p.head_dim;
}

// Epilogue shared by both kernel families.  A workgroup finishes the query
// heads [qh0, qh0 + nheads) of row b for its split.  Every thread calls it;
// thread t owns items idx = t + k * blockDim.x (k < MAXK) of the
// nheads x head_dim result, and value_of(k, idx, m, l, num) yields the
// workgroup's base-2 max, sum and unnormalised numerator for that item.
//
//  * one pass, or a row with a single non-empty split in counter mode:
//    write num / l to the output directly;
//  * otherwise store the partial; in counter mode the workgroup then counts
//    itself in at split_counters[counter] and the last of the row's
//    ceil(ctx / split_size) workgroups merges all partials of its heads by
//    log-sum-exp and resets the counter to zero, leaving it ready for the
//    next call (no memset, so the call is graph-replay safe).
//
// Cross-workgroup ordering follows the HIP memory model at agent scope:
// every lane stores its partials (agent-scope atomic stores) and issues an
// agent-scope release fence before the workgroup barrier, so those stores
// happen before thread 0's counter increment, itself an acquire-release RMW
// at agent scope; the last arrival's threads pass a barrier and an
// agent-scope acquire fence before reading any other workgroup's partials.
// The fences write back / invalidate the per-XCD L2 (the price of formal
// ordering on a multi-XCD part); this mode is opt-in and the default path
// merges in a second launch instead.
template <typename T, int MAXK, typename F>
__device__ __forceinline__ void finish(const AttnParams &p, int32_t b, int32_t qh0,
                                       int32_t nheads, int64_t counter, int32_t split,
                                       int32_t ctx, F value_of) {
  const int D = p.head_dim;
  const int items = nheads * D;
  const int32_t nvalid = (ctx + p.split_size - 1) / p.split_size;
  const bool counters = p.num_splits > 1 && p.split_counters != nullptr;
  const bool direct = p.num_splits == 1 || (counters && nvalid == 1);
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    const int idx = threadIdx.x + k * blockDim.x;
    if (idx < items) {
      float m, l, num;
      value_of(k, idx, m, l, num);
      const int g = idx / D;
      const int d = idx - g * D;
      const int32_t qh = qh0 + g;
      if (direct) {
        output_row<T>(p, b, qh)[d] = from_float<T>(l > 0.f ? num / l : 0.f);
      } else {
        const int64_t row = (static_cast<int64_t>(b) * p.query_heads + qh) * p.num_splits + split;
        if (counters) {
          __hip_atomic_store(p.partial_acc + row * p.partial_stride + d, num, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          if (d == 0) {
            __hip_atomic_store(p.partial_max + row, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.partial_sum + row, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        } else {
          p.partial_acc[row * p.partial_stride + d] = num;
          if (d == 0) {
            p.partial_max[row] = m;
            p.partial_sum[row] = l;
          }
        }
      }
    }
  }
  if (!counters || direct) return;

  __shared__ int32_t is_last;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // this lane's partials, published
  __syncthreads();                                    // ... and every other lane's
  if (threadIdx.x == 0) {
    int32_t *slot = p.split_counters + counter;
    const int32_t prev =
        __hip_atomic_fetch_add(slot, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == nvalid - 1;
    if (is_last) __hip_atomic_store(slot, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!is_last) return;
  // The other workgroups' partials happen before this point (their release,
  // the counter RMW, thread 0's acquire, the barrier); make them visible to
  // every lane of this one.
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // Merge: all loads of an item (nvalid <= 8 at a time) are issued before
  // any is used, so the merge costs one round trip per 8 splits.
  constexpr int kBatch = 8;
  for (int idx = threadIdx.x; idx < items; idx += blockDim.x) {
    const int g = idx / D;
    const int d = idx - g * D;
    const int32_t qh = qh0 + g;
    const int64_t base = (static_cast<int64_t>(b) * p.query_heads + qh) * p.num_splits;
    float gmax = kNegInf, num = 0.f, den = 0.f;
    for (int32_t s0 = 0; s0 < nvalid; s0 += kBatch) {
      float ms[kBatch], ls[kBatch], as[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int32_t sj = min(s0 + j, nvalid - 1);
        ms[j] = __hip_atomic_load(p.partial_max + base + sj, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        ls[j] = __hip_atomic_load(p.partial_sum + base + sj, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        as[j] = __hip_atomic_load(p.partial_acc + (base + sj) * p.partial_stride + d,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (s0 + j >= nvalid || ms[j] == kNegInf) continue;
        // Running log-sum-exp over the batches (base 2).
        if (ms[j] > gmax) {
          const float r = fast_exp2(gmax - ms[j]);
          num *= r;
          den *= r;
          gmax = ms[j];
        }
        const float e = fast_exp2(ms[j] - gmax);
        den += e * ls[j];
        num += e * as[j];
      }
    }
    output_row<T>(p, b, qh)[d] = from_float<T>(den > 0.f ? num / den : 0.f);
  }
}

// Log-sum-exp merge of the nvalid split partials of (row b, kv head kvh) by
// one wavefront, for the G query heads of the head.  Pass 1 loads every
// (head, split) max and sum at once and leaves the normalised weights
// exp2(m_s - M) / den in `scratch` (wavefront-private LDS, `capacity`
// floats).  Pass 2 accumulates the weighted partial rows, 4 items x 8
// splits of loads in flight per lane.  Partials are read with agent-scope
// atomic loads (coherent across XCDs).  When the weights do not fit the
// scratch, each item is merged on its own (slower, same result).
template <typename T, int D>
__device__ __forceinline__ void merge_head_partials(const AttnParams &p, int32_t b, int32_t kvh,
                                                 int32_t nvalid, float *scratch,
                                                 int32_t capacity) {
  const int lane = threadIdx.x & 63;
  const int32_t G = p.group;
  const int64_t head0 = (static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(kvh) * G) *
                        p.num_splits;  // partial row of (head 0 of the group, split 0)
  const int32_t pairs = G * nvalid;
  const int items = G * D;
  if (2 * pairs <= capacity) {
    float *wm = scratch;          // [G][nvalid] maxima, then weights
    float *wl = scratch + pairs;  // [G][nvalid] sums
    constexpr int kItems = 8, kSplits = 8;
    float v[kItems][kSplits];
    // Accumulator loads of items [64 k0, 64 (k0 + kItems)) x splits
    // [s0, s0 + kSplits) of this lane (independent of the weights).
    auto load_acc = [&](int k0, int32_t s0) {
#pragma unroll
      for (int i = 0; i < kItems; ++i) {
        const int idx = min(lane + 64 * (k0 + i), items - 1);
        const int g = idx / D;
        const int d = idx - g * D;
#pragma unroll
        for (int j = 0; j < kSplits; ++j) {
          const int32_t sj = min(s0 + j, nvalid - 1);
          v[i][j] = __hip_atomic_load(
              p.partial_acc + (head0 + static_cast<int64_t>(g) * p.num_splits + sj) *
                                  p.partial_stride + d,
              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    };
    // Pass 1: the (head, split) maxima and sums, issued first; the first
    // accumulator batch follows at once, so for G * D <= 512 and
    // nvalid <= 8 the whole merge waits for memory once.
    for (int32_t q0 = 0; q0 < pairs; q0 += 4 * 64) {
      float mv[4], lv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int32_t q = min(q0 + j * 64 + lane, pairs - 1);
        const int32_t g = q / nvalid;
        const int64_t at = head0 + static_cast<int64_t>(g) * p.num_splits + (q - g * nvalid);
        mv[j] = __hip_atomic_load(p.partial_max + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lv[j] = __hip_atomic_load(p.partial_sum + at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (q0 == 0) load_acc(0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int32_t q = q0 + j * 64 + lane;
        if (q < pairs) {
          wm[q] = mv[j];
          wl[q] = lv[j];
        }
      }
    }
    __asm__ volatile("" ::: "memory");
    if (lane < G) {
      float mmax = kNegInf;
      for (int32_t s = 0; s < nvalid; ++s) mmax = fmaxf(mmax, wm[lane * nvalid + s]);
      float den = 0.f;
      if (mmax != kNegInf)
        for (int32_t s = 0; s < nvalid; ++s)
          den += wl[lane * nvalid + s] * fast_exp2(wm[lane * nvalid + s] - mmax);
      const float inv = den > 0.f ? 1.f / den : 0.f;
      for (int32_t s = 0; s < nvalid; ++s) {
        const float m = wm[lane * nvalid + s];
        wm[lane * nvalid + s] = m == kNegInf ? 0.f : fast_exp2(m - mmax) * inv;
      }
    }
    __asm__ volatile("" ::: "memory");
    for (int k0 = 0; k0 * 64 < items; k0 += kItems) {
      float num[kItems];
#pragma unroll
      for (int i = 0; i < kItems; ++i) num[i] = 0.f;
      for (int32_t s0 = 0; s0 < nvalid; s0 += kSplits) {
        if (k0 > 0 || s0 > 0) load_acc(k0, s0);
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
          const int idx = min(lane + 64 * (k0 + i), items - 1);
          const int g = idx / D;
#pragma unroll
          for (int j = 0; j < kSplits; ++j)
            if (s0 + j < nvalid) num[i] += wm[g * nvalid + s0 + j] * v[i][j];
        }
      }
#pragma unroll
      for (int i = 0; i < kItems; ++i) {
        const int idx = lane + 64 * (k0 + i);
        if (idx < items) {
          const int g = idx / D;
          output_row<T>(p, b, kvh * G + g)[idx - g * D] = from_float<T>(num[i]);
        }
      }
    }
    return;
  }
  // Fallback: one item at a time, all splits of the item in flight.
  for (int idx = lane; idx < items; idx += 64) {
    const int g = idx / D;
    const int d = idx - g * D;
    const int64_t base = head0 + static_cast<int64_t>(g) * p.num_splits;
    float gmax = kNegInf, num = 0.f, den = 0.f;
    for (int32_t s = 0; s < nvalid; ++s) {
      const float m = __hip_atomic_load(p.partial_max + base + s, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
      const float l = __hip_atomic_load(p.partial_sum + base + s, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
      const float a = __hip_atomic_load(p.partial_acc + (base + s) * p.partial_stride + d,
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (m == kNegInf) continue;
      if (m > gmax) {
        const float r = fast_exp2(gmax - m);
        num *= r;
        den *= r;
        gmax = m;
      }
      const float e = fast_exp2(m - gmax);
      den += e * l;
      num += e * a;
    }
    output_row<T>(p, b, kvh * G + g)[d] = from_float<T>(den > 0.f ? num / den : 0.f);
  }
}

// ===========================================================================
// MFMA kernel
// ===========================================================================
template <typename T>
struct Mfma;

template <>
struct Mfma<__bf16> {
  typedef __bf16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<_Float16> {
  typedef _Float16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kChunk = 32;  // tokens per wavefront step (two 16-row tiles)

// LDS row of the staged V tile: head_dim elements plus 16 bytes, which
// staggers the rows of one transpose read over the banks.
template <int D>
constexpr int v_row_bytes() { return D * 2 + 16; }

// LDS of the MFMA grid kernel for `waves` wavefronts: max(per-wave V tiles,
// cross-wave merge buffers for 16 heads).
__host__ __device__ constexpr int mfma_lds_bytes(int head_dim, int waves) {
  return (waves * kChunk * (head_dim * 2 + 16)) > (waves * (16 * head_dim + 32) * 4)
             ? (waves * kChunk * (head_dim * 2 + 16))
             : (waves * (16 * head_dim + 32) * 4);
}

// Rescale threshold of the lazy online softmax (base-2 units): the running
// max of a head is only raised -- and the accumulator rescaled -- when a
// score exceeds it by more than this, so weights stay below 2^8 and the
// rescale (with its cross-lane max) runs a handful of times per split.
constexpr float kRescaleThreshold = 8.f;
constexpr int kSegmentTiles = 64;  // page-window capacity: 64 tiles = 1024 tokens

// Max / sum over the 16 lanes of a DPP row (every lane gets the result):
// quad_perm [1,0,3,2] and [2,3,0,1] combine within quads, row_half_mirror
// (lane i <-> 7 - i of each half row) pairs the two quads of a half row and
// row_mirror (i <-> 15 - i) the two halves -- in-register lane moves instead
// of LDS-routed shuffles.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_move<0xb1>(v));
  v = fmaxf(v, dpp_move<0x4e>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  return fmaxf(v, dpp_move<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_move<0xb1>(v);
  v += dpp_move<0x4e>(v);
  v += dpp_move<0x141>(v);
  return v + dpp_move<0x140>(v);
}
// Lane `l` of v (l wavefront-uniform).
__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Max / sum over the 64 lanes: the rows' results combined by lane reads
// (the same value on every lane).
__device__ __forceinline__ float wave64_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave64_sum(float v) {
  v = row16_sum(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// Wave-level layout of one 32-token chunk (tiles j = 0, 1 of 16 tokens):
//   loads    LINES: lane holds bytes [16 (lane % (D/8)), +16) of the K / V
//            slice of token 16j + lane / (D/8) + (512/D) ks (whole token
//            rows), and K is staged in LDS and read back in the A-operand
//            layout; otherwise lane (l16, q4) loads K / V of token 16j + l16,
//            head_dim elements [32ks + 8q4, +8) -- the A operand directly;
//   scores   lane holds S[token 16j + 4q4 + r][head l16], r = 0..3;
//   P        B operand of the P.V MFMA, k = 8q4 + i <-> token 4q4 + i of
//            tile 0 (i < 4) or 4q4 + i - 4 of tile 1 (i >= 4);
//   V^T      A operand of the P.V MFMA (row = dim 16n + l16, same k order),
//            produced by ds_read_b64_tr_b16 from V staged token-major: in a
//            16-lane group, lane jj addresses the 4 elements
//            V[4q4 + jj/4][16n + 4(jj%4) .. +4] and lane i receives
//            V[4q4 + e][16n + i] for e = 0..3.
// Requires block_size % 16 == 0 and split_size % 32 == 0 (a tile never
// straddles a page), so each tile's page is wave-uniform.
template <typename T, int D, int NW, bool ROPE, bool LINES, bool VALU = false>
__global__ void __launch_bounds__(NW * 64)
paged_decode_mfma_kernel(AttnParams p) {
  using M = Mfma<T>;
  using vec8 = typename M::vec8;
  constexpr int KS = D / 32;  // k-steps of the score product
  constexpr int NB = D / 16;  // 16-dim blocks of the output
  constexpr int kRow = v_row_bytes<D>();
  // Dynamic LDS sized for the launch's wavefronts (mfma_lds_bytes).
  extern __shared__ __attribute__((aligned(16))) unsigned char mfma_smem[];
  unsigned char *lds = mfma_smem;

  // blockIdx.x enumerates (row, kv-head group) and the split index is the
  // slow dimension: the first dispatches cover split 0 of every row (present
  // in every non-empty row) before any later split, and the round-robin
  // deal over the 8 XCDs gives each XCD an even mix of rows and splits.
  // Wavefront w serves kv head (group * HPW + w % HPW) and takes every
  // WPH-th chunk of the split starting at w / HPW, so the HPW wavefronts of
  // one sub-index read the slices of the same token rows at the same time:
  // the cache row [token, kv head, head_dim] is fetched as a whole, not one
  // head slice at a time from different workgroups.
  //
  // Balanced calls launch one compact grid instead: blockIdx.x = slot * NG +
  // group, the slot naming a (row, partition) by balanced_slot, and slots
  // without a partition exit at once.
  const int32_t HPW = p.heads_per_wg;
  const int32_t WPH = p.waves_per_head;
  const int32_t NG = p.kv_heads / HPW;
  int32_t b, grp, split, split_size;
  if (p.balanced) {
    grp = blockIdx.x % NG;
    balanced_slot(p, blockIdx.x / NG, split_size, b, split);
    if (b < 0) return;  // the same on every wavefront of the workgroup
  } else {
    b = blockIdx.x / NG;
    grp = blockIdx.x - b * NG;
    split = blockIdx.y;
    split_size = p.split_size;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t hl = wave % HPW;   // head within the group
  const int32_t sub = wave / HPW;  // chunk phase within the head
  const int32_t kvh = grp * HPW + hl;
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int32_t s0 = split * split_size;
  const int32_t *table = p.block_tables + static_cast<int64_t>(b) * p.table_width;

  // Page ids of up to 64 tiles starting at `first` (lane i: tile first + i).
  auto load_window = [&](int32_t first) -> int32_t {
    const int32_t t = s0 + 16 * (first + lane);
    const int32_t logical = p.page_shift >= 0 ? (t >> p.page_shift) : (t / p.block_size);
    return logical < p.table_width ? table[logical] : -1;
  };
  // Byte offsets of the same tiles' K / V head slices from the cache bases
  // (lane i: tile first + i), -1 where the tile has no valid page: computed
  // once per window on the vector lanes, so a tile's loads need only two
  // lane reads and a few scalar adds (the scalar unit, one instruction per
  // cycle for the whole compute unit, was the long rows' bound).
  const uint32_t token_bytes = static_cast<uint32_t>(p.kv_heads) * D * sizeof(T);
  const int64_t head_bytes = static_cast<int64_t>(kvh) * D * sizeof(T);
  auto window_offsets = [&](int32_t first, int32_t page, uint32_t &lo, int32_t &hi) {
    const int32_t t = s0 + 16 * (first + lane);
    const int32_t in_page = p.page_shift >= 0 ? (t & (p.block_size - 1))
                                              : (t - (t / p.block_size) * p.block_size);
    const int64_t off = page >= 0 && page < p.num_blocks
                            ? (static_cast<int64_t>(page) * p.block_size + in_page) * token_bytes + head_bytes
                            : int64_t{-1};
    lo = static_cast<uint32_t>(off);
    hi = static_cast<int32_t>(off >> 32);
  };
  uint32_t win_lo = 0;  // the current segment's window_offsets
  int32_t win_hi = -1;

  // Independent start-up loads, all issued before anything waits for one:
  // the first page window, the query group, then the row length (below;
  // with RoPE the length is read together with the row's position).
  int32_t page_win = load_window(0);
  int32_t length = 0;
  vec8 qf[KS];  // B operand of the score MFMA: q[head l16][32ks + 8q4 .. +8]
  constexpr int kHalf = D / 2;
  // RoPE inputs of this row: the QKV row and the cos / sin rows of its position.
  const T *rope_row = nullptr;
  const T *rope_cs = nullptr;
  const T *rope_sn = nullptr;
  if constexpr (ROPE) {
    rope_row = static_cast<const T *>(p.rope_qkv) + static_cast<int64_t>(b) * p.rope_row_stride;
    length = p.context_lengths[b];
    int64_t pos = p.rope_positions[b];
    // Both reads issued before either is waited for (the empty-row test on
    // the length would otherwise be placed between them).
    __asm__ volatile("" ::: "memory");
    pos = pos < 0 ? 0 : (pos >= p.rope_table_rows ? p.rope_table_rows - 1 : pos);
    rope_cs = static_cast<const T *>(p.rope_cos) + pos * D;
    rope_sn = static_cast<const T *>(p.rope_sin) + pos * D;
  }
  // 8 rotated elements [i0, i0 + 8) of the head at `src` (i0 a multiple of 8;
  // the pair partner of element i is i + D/2 or i - D/2).
  auto rotate8 = [&](const T *src, int i0) -> vec8 {
    const int ip = i0 < kHalf ? i0 + kHalf : i0 - kHalf;
    const vec8 x = *reinterpret_cast<const vec8 *>(src + i0);
    const vec8 xp = *reinterpret_cast<const vec8 *>(src + ip);
    const vec8 c = *reinterpret_cast<const vec8 *>(rope_cs + i0);
    const vec8 sn = *reinterpret_cast<const vec8 *>(rope_sn + i0);
    vec8 out;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float o = i0 < kHalf ? rope_lo(to_float(x[j]), to_float(xp[j]), to_float(c[j]), to_float(sn[j]))
                                 : rope_hi(to_float(xp[j]), to_float(x[j]), to_float(c[j]), to_float(sn[j]));
      out[j] = from_float<T>(o);
    }
    return out;
  };
  {
    // Lanes past the group (l16 >= group) take the group's last head: their
    // score and output columns are never stored, and their maxima follow
    // that head's, so the wavefront's rescale decisions and every stored
    // bit are unchanged.  Loads with no branch around them leave the
    // compiler no reason to wait for them here (a branch's phi copy did, and
    // with it the window and row-length loads behind them lost a round trip).
    const int64_t head = static_cast<int64_t>(kvh) * p.group + min(l16, p.group - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (ROPE) {
        qf[ks] = rotate8(rope_row + head * D, 32 * ks + 8 * q4);
      } else {
        const T *qrow = static_cast<const T *>(p.query) +
                        (static_cast<int64_t>(b) * p.query_heads + head) * D;
        qf[ks] = *reinterpret_cast<const vec8 *>(qrow + 32 * ks + 8 * q4);
      }
    }
  }
  // The row length is read after the loads above are issued: its test (an
  // empty partition returns) would otherwise be placed first, holding the
  // query loads behind the length's round trip.
  if constexpr (!ROPE) {
    __asm__ volatile("" ::: "memory");
    length = p.context_lengths[b];
  }
  const int32_t ctx = length < 0 ? 0 : (length > p.max_tokens ? p.max_tokens : length);
  // VALU form (head_dim 64, group <= 8): lane (t16, qd) holds dims
  // [16 qd, 16 qd + 16) of every query head of the group (zeros past it).
  constexpr int kValuHeads = 8;
  vec8 qq[VALU ? kValuHeads : 1][2];
  if constexpr (VALU) {
    const T *qgroup = static_cast<const T *>(p.query) +
                      (static_cast<int64_t>(b) * p.query_heads +
                       static_cast<int64_t>(kvh) * p.group) * D + 16 * q4;
#pragma unroll
    for (int h = 0; h < kValuHeads; ++h) {
      const bool own = h < p.group;
      qq[h][0] = own ? *reinterpret_cast<const vec8 *>(qgroup + h * D) : vec8{};
      qq[h][1] = own ? *reinterpret_cast<const vec8 *>(qgroup + h * D + 8) : vec8{};
    }
  }

  if (s0 >= ctx) {
    if (split == 0) zero_rows<T>(p, b, grp * HPW * p.group, HPW * p.group);
    return;
  }
  if constexpr (ROPE) {
    // The row's new token: every wavefront writes the whole token row --
    // rotated k and v of every kv head, the same bytes from every
    // wavefront of the row -- and waits for its own stores before its
    // first K/V load.  Any cache line of the row that a wavefront later
    // reads (kv heads of 64 bytes or less share a line) then already holds
    // the token in L2 when it reads it, whichever wavefront of the compute
    // unit brought the line into L1: no wavefront loads a line of any
    // appended row before its own wait (stand-in loads read the QKV row,
    // and the chunk deal reads a row's new token only in that row's own
    // wavefronts), the vector L1 is write-through, and L1 holds nothing
    // from before the launch.  Pieces [0, Hkv D/8) rotate 8 key elements
    // each, the next Hkv D/8 copy 8 value elements.
    //
    // Issuing a wavefront's first K/V chunks before this store (when they
    // do not hold the new token) once gave results that differed from the
    // two launches at head_dim 32, although no such load touches an
    // appended line (tests/test_fused_append_schedule.py restates the
    // addresses).  The same symptom -- a few last-bit differences, both
    // forms deterministic -- came back with another change of this
    // prologue and went away when the wavefronts' combine below was written
    // with explicit fused multiply-adds: the compiler had fused a different
    // product of `x * a + y * c` in the two instantiations.
    const int32_t page = p.append_pages[b];
    const int32_t off = p.append_offsets[b];
    const bool append = p.append_active[b] != 0 && page >= 0 && page < p.num_blocks && off >= 0 &&
                        off < p.block_size;
    if (append) {
      const int64_t row0 = (static_cast<int64_t>(page) * p.block_size + off) * p.kv_heads * D;
      const int32_t pieces = p.kv_heads * (D / 8);
      for (int32_t i = lane; i < 2 * pieces; i += 64) {
        const int32_t j = i < pieces ? i : i - pieces;
        const int32_t h = j / (D / 8);
        const int e0 = 8 * (j - h * (D / 8));
        if (i < pieces) {
          const vec8 k = rotate8(rope_row + static_cast<int64_t>(p.query_heads + h) * D, e0);
          *reinterpret_cast<vec8 *>(static_cast<T *>(const_cast<void *>(p.key_cache)) + row0 +
                                    static_cast<int64_t>(h) * D + e0) = k;
        } else {
          const vec8 v = *reinterpret_cast<const vec8 *>(
              rope_row + static_cast<int64_t>(p.query_heads + p.kv_heads + h) * D + e0);
          *reinterpret_cast<vec8 *>(static_cast<T *>(const_cast<void *>(p.value_cache)) + row0 +
                                    static_cast<int64_t>(h) * D + e0) = v;
        }
      }
    }
    // vmcnt counts stores on gfx9-family parts: after the wait this
    // wavefront's stores have reached L2.  The empty asm statements are
    // compiler memory barriers, so no load below is scheduled above it.
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);
    __asm__ volatile("" ::: "memory");
  }
  const int32_t s1 = min(s0 + split_size, ctx);
  // Wavefronts of the head that take chunks of this row: all WPH, or with a
  // token budget per wavefront only as many as the row's length needs (the
  // rest stay idle), so short rows do not load the memory system with
  // near-empty streams while long rows still get WPH.
  int32_t active = WPH;
  if (p.tokens_per_wave > 0) {
    active = (s1 - s0 + p.tokens_per_wave - 1) / p.tokens_per_wave;
    active = active < 1 ? 1 : (active > WPH ? WPH : active);
  }

  const unsigned char *kbytes = static_cast<const unsigned char *>(p.key_cache);
  const unsigned char *vbytes = static_cast<const unsigned char *>(p.value_cache);
  // Stand-in row of absent tokens (read, masked out): this row's query
  // input, at least D elements long.
  const unsigned char *stand_in =
      ROPE ? reinterpret_cast<const unsigned char *>(rope_row)
           : static_cast<const unsigned char *>(p.query) +
                 static_cast<int64_t>(b) * p.query_heads * D * sizeof(T);
  // Operand-layout loads: lane (l16, q4) reads 16 bytes of token l16.
  const uint32_t lane_full = static_cast<uint32_t>(l16) * token_bytes + 16u * q4;
  const uint32_t lane_first = 16u * q4;  // stand-in row for absent tokens
  // LINES: K and V pass through LDS, so their loads need not follow the
  // MFMA operand layout: D/8 lanes cover one token's head slice and one
  // load covers 512/D whole tokens (whole cache lines), where a load in
  // operand layout touches 16 tokens with half a line each.  A compute
  // unit issues loads of fewer lines faster (its ceiling rises from about
  // 36 to 55 GB/s), at the price of an LDS round trip for K on every
  // chunk: the form for several wavefronts per kv head.
  constexpr int kVLanes = D / 8;
  constexpr int kVTokens = 64 / kVLanes;
  const int v_tok = lane / kVLanes;  // token of load ks: v_tok + kVTokens * ks
  const uint32_t v_piece = 16u * static_cast<uint32_t>(lane % kVLanes);

  f32x4 acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;  // reference max of head l16 (base 2, scaled)
  float l_run = 0.f;      // lane-partial sum of head l16
  unsigned char *vt = lds + wave * kChunk * kRow;
  // VALU form state: per head h of the group the reference max and sum
  // (the same on every lane) and the accumulator of output dimension `lane`.
  float vm[VALU ? kValuHeads : 1], vl[VALU ? kValuHeads : 1], vacc[VALU ? kValuHeads : 1];
#pragma unroll
  for (int h = 0; h < (VALU ? kValuHeads : 1); ++h) {
    vm[h] = kNegInf;
    vl[h] = 0.f;
    vacc[h] = 0.f;
  }
  // The wavefront's VALU slice: P as [32 tokens][8 heads] floats, at the end
  // the accumulators as [8 heads][64 dims].
  float *vslice = VALU ? reinterpret_cast<float *>(lds + mfma_lds_bytes(D, blockDim.x >> 6)) +
                             wave * kValuHeads * 64
                       : nullptr;

  // Issue the K/V loads of segment-relative chunk c (valid or not: absent
  // tokens and chunks past the end read a stand-in row, so every load is
  // unconditional and the wait counts stay exact).  Bit t of valid[j]
  // marks token 16j + t present.
  auto load_kv = [&](int32_t seg_s0, int32_t seg_s1, int32_t c, vec8(&kf)[2][KS], vec8(&vf)[2][KS],
                     uint32_t(&valid)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int32_t t0 = seg_s0 + c * kChunk + 16 * j;
      // Tile 2c + j of the segment's window (past the segment's end the
      // tile is absent whatever the slot holds).
      const int32_t slot = min(2 * c + j, kSegmentTiles - 1);
      const uint32_t off_lo = __builtin_amdgcn_readlane(win_lo, slot);
      const int32_t off_hi = __builtin_amdgcn_readlane(win_hi, slot);
      const bool tile_ok = t0 < seg_s1 && off_hi >= 0;
      const int32_t ntok = tile_ok ? min(16, seg_s1 - t0) : 0;
      valid[j] = ntok >= 16 ? 0xffffu : ((1u << ntok) - 1u);
      // Absent tiles read a stand-in row: the row's query (or QKV) input,
      // which nothing writes while the kernel runs, so that a stand-in load
      // never brings a cache page's line into L1 while another workgroup
      // on this compute unit may be appending to it.
      const int64_t tile_off = static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(off_hi)) << 32) | off_lo);
      const unsigned char *kp = tile_ok ? kbytes + tile_off : stand_in;
      const unsigned char *vp = tile_ok ? vbytes + tile_off : stand_in;
      const uint32_t lane_off = l16 < ntok ? lane_full : lane_first;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int tt = v_tok + kVTokens * ks;
        const uint32_t t_off =
            LINES ? (tt < ntok ? static_cast<uint32_t>(tt) * token_bytes : 0u) + v_piece
                  : lane_off + 64u * ks;
        kf[j][ks] = load_stream16<vec8>(kp + t_off);
        vf[j][ks] = load_stream16<vec8>(vp + t_off);
      }
    }
  };

  // VALU form of one chunk, K staged token-major in vt.  Scores: lane
  // (t16, qd) takes token 16j + t16 and dims [16 qd, +16) of every head
  // (packed two-element dot products), summed over the four dimension
  // quarters by two cross-lane adds.  Per-head online softmax with the same
  // lazy rescale as the MFMA form; P (rounded to T, as the MFMA form feeds
  // it) goes through the wavefront's slice as [token][head], and P.V runs
  // with lane = output dimension: one conversion per V element and G fp32
  // FMAs per token.
  auto valu_chunk = [&](vec8(&vf)[2][KS], const uint32_t(&valid)[2]) {
    const bool wide = p.group > 4;  // uniform: heads 4..7 in use
    float sj[2][kValuHeads];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const unsigned char *krow = vt + (16 * j + l16) * kRow + 32 * q4;
      const vec8 k0 = *reinterpret_cast<const vec8 *>(krow);
      const vec8 k1 = *reinterpret_cast<const vec8 *>(krow + 16);
      const bool present = (valid[j] >> l16) & 1u;
#pragma unroll
      for (int h = 0; h < kValuHeads; ++h) {
        float d = 0.f;
        if (h < 4 || wide) d = dot8<T>(qq[h][1], k1, dot8<T>(qq[h][0], k0, 0.f));
        d += __shfl_xor(d, 16, 64);
        d += __shfl_xor(d, 32, 64);
        sj[j][h] = present ? d : kNegInf;
      }
    }
    float cm[kValuHeads];
#pragma unroll
    for (int h = 0; h < kValuHeads; ++h) {
      cm[h] = row16_max(fmaxf(sj[0][h], sj[1][h])) * p.scale_log2;  // scale > 0 commutes with max
    }
    if (cm[0] == kNegInf) return;  // uniform: no token of the chunk is present
    bool raise = false;
#pragma unroll
    for (int h = 0; h < kValuHeads; ++h) raise |= cm[h] > vm[h] + kRescaleThreshold;
    if (raise) {  // uniform
#pragma unroll
      for (int h = 0; h < kValuHeads; ++h) {
        const float mn = fmaxf(vm[h], cm[h]);
        const float alpha = fast_exp2(vm[h] - mn);
        vm[h] = mn;
        vl[h] *= alpha;
        vacc[h] *= alpha;
      }
    }
    float pj[2][kValuHeads];
#pragma unroll
    for (int h = 0; h < kValuHeads; ++h) {
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float pr = fast_exp2(__builtin_fmaf(sj[j][h], p.scale_log2, -vm[h]));
        ps += pr;
        pj[j][h] = to_float(from_float<T>(pr));
      }
      vl[h] += row16_sum(ps);
    }
    __asm__ volatile("" ::: "memory");
    if (q4 == 0) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float *dst = vslice + (16 * j + l16) * kValuHeads;
        *reinterpret_cast<f32x4 *>(dst) = f32x4{pj[j][0], pj[j][1], pj[j][2], pj[j][3]};
        *reinterpret_cast<f32x4 *>(dst + 4) = f32x4{pj[j][4], pj[j][5], pj[j][6], pj[j][7]};
      }
    }
    // V replaces K in the tile (the wavefront's LDS requests are served in
    // order); stand-in rows of absent tokens are cleared so that
    // 0 * (non-finite) cannot leak into the accumulators.
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bool mine = (valid[j] >> (v_tok + kVTokens * ks)) & 1u;
        *reinterpret_cast<vec8 *>(vt + (16 * j + v_tok + kVTokens * ks) * kRow + v_piece) =
            mine ? vf[j][ks] : vec8{};
      }
    __asm__ volatile("" ::: "memory");
    const unsigned char *vcol = vt + 2 * lane;
    if (wide) {
#pragma unroll 8
      for (int t = 0; t < kChunk; ++t) {
        const f32x4 p0 = *reinterpret_cast<const f32x4 *>(vslice + t * kValuHeads);
        const f32x4 p1 = *reinterpret_cast<const f32x4 *>(vslice + t * kValuHeads + 4);
        const float v = to_float(*reinterpret_cast<const T *>(vcol + t * kRow));
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          vacc[h] = __builtin_fmaf(p0[h], v, vacc[h]);
          vacc[4 + h] = __builtin_fmaf(p1[h], v, vacc[4 + h]);
        }
      }
    } else {
#pragma unroll 8
      for (int t = 0; t < kChunk; ++t) {
        const f32x4 p0 = *reinterpret_cast<const f32x4 *>(vslice + t * kValuHeads);
        const float v = to_float(*reinterpret_cast<const T *>(vcol + t * kRow));
#pragma unroll
        for (int h = 0; h < 4; ++h) vacc[h] = __builtin_fmaf(p0[h], v, vacc[h]);
      }
    }
    __asm__ volatile("" ::: "memory");
  };

  auto compute = [&](vec8(&kf)[2][KS], vec8(&vf)[2][KS], const uint32_t(&valid)[2]) {
    if constexpr (LINES) {
      // Stage K token-major in the wavefront's LDS tile and read it back in
      // the A-operand layout; the V tile below reuses the same bytes (the
      // wavefront's LDS requests are served in order).
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          *reinterpret_cast<vec8 *>(vt + (16 * j + v_tok + kVTokens * ks) * kRow + v_piece) = kf[j][ks];
      __asm__ volatile("" ::: "memory");
      if constexpr (VALU) {
        valu_chunk(vf, valid);
        return;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          kf[j][ks] =
              *reinterpret_cast<const vec8 *>(vt + (16 * j + l16) * kRow + (32 * ks + 8 * q4) * 2);
      __asm__ volatile("" ::: "memory");
    }
    float sc[8];  // raw q.k of token 16j + 4q4 + r, head l16
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) s = M::mma(kf[j][ks], qf[ks], s);
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[4 * j + r] = s[r];
    }
    if ((valid[0] & valid[1]) != 0xffffu) {  // uniform: partial chunk
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (!((valid[j] >> (4 * q4 + r)) & 1u)) sc[4 * j + r] = kNegInf;
      // Stand-in V rows of absent tokens are cleared so that 0 * (non-finite)
      // cannot leak into the accumulator.
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bool mine = (valid[j] >> (LINES ? v_tok + kVTokens * ks : l16)) & 1u;
          vf[j][ks] = mine ? vf[j][ks] : vec8{};
        }
    }
    float mx = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                     fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
    mx *= p.scale_log2;  // scale > 0 commutes with max
    // Raise the reference max only when some score overshoots it by more
    // than the threshold (uniform decision).
    if (__ballot(mx > m_run + kRescaleThreshold) != 0) {
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      if (mx == kNegInf) return;  // uniform: no token of the chunk is present
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int n = 0; n < NB; ++n) acc[n] *= alpha;
    }
    vec8 pf;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pr = fast_exp2(__builtin_fmaf(sc[i], p.scale_log2, -m_run));
      psum += pr;
      pf[i] = static_cast<T>(pr);
    }
    l_run += psum;

    // Stage V token-major (one 16-byte LDS write per load, each to its
    // token's row), then read V^T fragments with the transpose read.  LDS
    // requests of one wavefront are served in order, so compiler barriers
    // are the only ordering needed.
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        *reinterpret_cast<vec8 *>(
            vt + (LINES ? (16 * j + v_tok + kVTokens * ks) * kRow + v_piece
                        : (16 * j + l16) * kRow + (32 * ks + 8 * q4) * 2)) = vf[j][ks];
    __asm__ volatile("" ::: "memory");
    {
      const unsigned char *rd = vt + (4 * q4 + (l16 >> 2)) * kRow + (l16 & 3) * 8;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(rd + 32 * n));
        const i16x4 hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(rd + 16 * kRow + 32 * n));
        const i16x8 a16 = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        acc[n] = M::mma(__builtin_bit_cast(vec8, a16), pf, acc[n]);
      }
    }
    __asm__ volatile("" ::: "memory");
  };

  // Segments of up to 1024 tokens share one page window; inside a segment
  // two register sets alternate so the next chunk's K/V are in flight while
  // the current one is computed (a third set, two chunks ahead, measured
  // slower: 16 KB more in flight per wavefront lowers a compute unit's
  // read rate).
  vec8 ka[2][KS], va[2][KS], kb[2][KS], vb[2][KS];
  uint32_t vala[2], valb[2];
  for (int32_t seg_s0 = s0; seg_s0 < s1; seg_s0 += 16 * kSegmentTiles) {
    const int32_t seg_first_tile = (seg_s0 - s0) >> 4;
    if (seg_first_tile != 0) page_win = load_window(seg_first_tile);
    const int32_t seg_s1 = min(seg_s0 + 16 * kSegmentTiles, s1);
    const int32_t seg_chunks = (seg_s1 - seg_s0 + kChunk - 1) / kChunk;
    const int32_t mine =
        sub < active && seg_chunks > sub ? (seg_chunks - sub + active - 1) / active : 0;
    if (mine == 0) continue;
    window_offsets(seg_first_tile, page_win, win_lo, win_hi);
    auto chunk = [&](int32_t i) { return i < mine ? sub + i * active : seg_chunks; };
    load_kv(seg_s0, seg_s1, chunk(0), ka, va, vala);
    for (int32_t i = 0; i < mine; i += 2) {
      load_kv(seg_s0, seg_s1, chunk(i + 1), kb, vb, valb);
      compute(ka, va, vala);
      if (i + 1 >= mine) break;
      load_kv(seg_s0, seg_s1, chunk(i + 2), ka, va, vala);
      compute(kb, vb, valb);
    }
  }

  if constexpr (VALU) {
    // Into the MFMA form's lane layout (head l16, dims 16n + 4q4 + r, the
    // sum of head l16 on its q4 = 0 lane) through the slice, for the shared
    // combine and epilogue; lanes of heads past the group are never stored.
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int h = 0; h < kValuHeads; ++h) vslice[h * 64 + lane] = vacc[h];
    __asm__ volatile("" ::: "memory");
    const bool own = l16 < kValuHeads;
    const int hh = own ? l16 : 0;
#pragma unroll
    for (int n = 0; n < NB; ++n)
      acc[n] = own ? *reinterpret_cast<const f32x4 *>(vslice + hh * 64 + 16 * n + 4 * q4)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
    float m = vm[0], l = vl[0];
#pragma unroll
    for (int h = 1; h < kValuHeads; ++h) {
      m = hh == h ? vm[h] : m;
      l = hh == h ? vl[h] : l;
    }
    m_run = m;
    l_run = own && q4 == 0 ? l : 0.f;
  }

  // Lane-partial sums -> per-head sums within the wave.
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);

  // Several wavefronts per head: the ones with sub > 0 hand their state to
  // the sub == 0 wavefront of their head through LDS (the V tiles are dead
  // after the first barrier).  Each lane combines the elements it owns, so
  // the reads are independent.  The second barrier frees LDS again.
  if (WPH > 1) {  // workgroup-uniform
    __syncthreads();
    float *xm = reinterpret_cast<float *>(lds);  // [waves][32]: m of 16 heads, then l
    float *xa = xm + HPW * WPH * 32;             // [waves][64 lanes][D / 4]
    constexpr int kLaneFloats = D / 4;
    if (sub > 0) {
      if (q4 == 0) {
        xm[wave * 32 + l16] = m_run;
        xm[wave * 32 + 16 + l16] = l_run;
      }
#pragma unroll
      for (int n = 0; n < NB; ++n)
        *reinterpret_cast<f32x4 *>(xa + (wave * 64 + lane) * kLaneFloats + 4 * n) = acc[n];
    }
    __syncthreads();
    if (sub == 0) {
      for (int32_t s = 1; s < active; ++s) {
        const int w = hl + s * HPW;
        const float mo = xm[w * 32 + l16];
        const float lo = xm[w * 32 + 16 + l16];
        f32x4 ao[NB];
#pragma unroll
        for (int n = 0; n < NB; ++n)
          ao[n] = *reinterpret_cast<const f32x4 *>(xa + (w * 64 + lane) * kLaneFloats + 4 * n);
        const float mn = fmaxf(m_run, mo);
        const float a = m_run == kNegInf ? 0.f : fast_exp2(m_run - mn);
        const float c = mo == kNegInf ? 0.f : fast_exp2(mo - mn);
        m_run = mn;
        // Explicit fused multiply-adds: `x * a + y * c` leaves the compiler
        // free to fuse either product, and its choice differed between
        // instantiations of this kernel (the fused RoPE launch and the plain
        // one, which must give the same bits) once their other code differed.
        l_run = __builtin_fmaf(lo, c, l_run * a);
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[n][r] = __builtin_fmaf(ao[n][r], c, acc[n][r] * a);
      }
    }
    __syncthreads();
    if (sub > 0) return;
  }

  // ---- per-wavefront epilogue for kv head kvh ----------------------------
  // Lane (l16, q4) owns head l16 (if < G), dims 16n + 4q4 + r.
  const int32_t G = p.group;
  const int32_t nvalid = (ctx + split_size - 1) / split_size;
  const bool counters = p.num_splits > 1 && p.split_counters != nullptr;
  const bool direct = p.num_splits == 1 || (counters && nvalid == 1);
  const bool head_ok = l16 < G;
  const int32_t qh = kvh * G + l16;
  if (direct) {
    if (head_ok) {
      const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
      T *out = output_row<T>(p, b, qh);
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        const t4 v = {from_float<T>(acc[n][0] * inv), from_float<T>(acc[n][1] * inv),
                      from_float<T>(acc[n][2] * inv), from_float<T>(acc[n][3] * inv)};
        *reinterpret_cast<t4 *>(out + 16 * n + 4 * q4) = v;
      }
    }
    return;
  }
  // Partials: the accumulator tile goes through this wavefront's LDS area
  // ([G][D] floats, <= 64 * D bytes, within the V staging tile) so that
  // each store instruction writes consecutive floats of one partial row.
  {
    float *tile = reinterpret_cast<float *>(vt);
    if (head_ok) {
#pragma unroll
      for (int n = 0; n < NB; ++n)
        *reinterpret_cast<f32x4 *>(tile + l16 * D + 16 * n + 4 * q4) = acc[n];
    }
    __asm__ volatile("" ::: "memory");
    const int64_t row0 = (static_cast<int64_t>(b) * p.query_heads + kvh * G) * p.num_splits + split;
    for (int idx = lane; idx < G * D; idx += 64) {
      const int g = idx / D;
      const int d = idx - g * D;
      float *dst = p.partial_acc + (row0 + static_cast<int64_t>(g) * p.num_splits) * p.partial_stride + d;
      if (counters)
        __hip_atomic_store(dst, tile[idx], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else
        *dst = tile[idx];
    }
    if (head_ok && q4 == 0) {
      const int64_t row = row0 + static_cast<int64_t>(l16) * p.num_splits;
      if (counters) {
        __hip_atomic_store(p.partial_max + row, m_run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.partial_sum + row, l_run, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        p.partial_max[row] = m_run;
        p.partial_sum[row] = l_run;
      }
    }
    __asm__ volatile("" ::: "memory");
  }
  if (!counters) return;
  // Publish this wavefront's partials at agent scope before its counter
  // increment (an acquire-release RMW); the last arrival acquires at agent
  // scope before reading the other wavefronts' partials (the ordering of
  // `finish` above, with the wavefront as the unit).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  int32_t last = 0;
  if (lane == 0) {
    int32_t *slot = p.split_counters + static_cast<int64_t>(b) * p.kv_heads + kvh;
    const int32_t prev =
        __hip_atomic_fetch_add(slot, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == nvalid - 1;
    if (last) __hip_atomic_store(slot, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (__builtin_amdgcn_readfirstlane(last) == 0) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  merge_head_partials<T, D>(p, b, kvh, nvalid, reinterpret_cast<float *>(vt),
                            kChunk * kRow / static_cast<int>(sizeof(float)));
}

// ===========================================================================
// Generic kernel (fp32 math, LDS tiles)
// ===========================================================================
constexpr int kGenericThreads = 256;
constexpr int kGenericTile = 16;
constexpr int kGenericMaxAcc = 32;  // group * head_dim <= 256 * 32

template <typename T>
__global__ void __launch_bounds__(kGenericThreads)
paged_decode_generic_kernel(AttnParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char generic_smem[];
  float *smem = reinterpret_cast<float *>(generic_smem);
  const int D = p.head_dim;
  const int G = p.group;
  float *ks = smem;                            // [tile][D + 1]
  float *vs = ks + kGenericTile * (D + 1);     // [tile][D]
  float *sc = vs + kGenericTile * D;           // [G][tile]
  float *m_run = sc + G * kGenericTile;        // [G]
  float *l_run = m_run + G;                    // [G]
  float *alpha = l_run + G;                    // [G]
  int *tok_ok = reinterpret_cast<int *>(alpha + G);  // [tile]

  const int32_t b = blockIdx.x / p.kv_heads;
  const int32_t kvh = blockIdx.x - b * p.kv_heads;
  const int32_t split = blockIdx.y;
  const int32_t ctx = clamp_context(p, b);
  const int32_t s0 = split * p.split_size;
  if (s0 >= ctx) {
    if (split == 0) zero_rows<T>(p, b, kvh * p.group, p.group);
    return;
  }
  const int32_t s1 = min(s0 + p.split_size, ctx);
  const int32_t *table = p.block_tables + static_cast<int64_t>(b) * p.table_width;
  const T *q = static_cast<const T *>(p.query) +
               (static_cast<int64_t>(b) * p.query_heads + static_cast<int64_t>(kvh) * G) * D;
  const T *kbase = static_cast<const T *>(p.key_cache) + static_cast<int64_t>(kvh) * D;
  const T *vbase = static_cast<const T *>(p.value_cache) + static_cast<int64_t>(kvh) * D;

  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    m_run[g] = kNegInf;
    l_run[g] = 0.f;
  }
  float acc[kGenericMaxAcc];
#pragma unroll
  for (int i = 0; i < kGenericMaxAcc; ++i) acc[i] = 0.f;

  for (int32_t t0 = s0; t0 < s1; t0 += kGenericTile) {
    __syncthreads();
    for (int idx = threadIdx.x; idx < kGenericTile * D; idx += blockDim.x) {
      const int tt = idx / D;
      const int d = idx - tt * D;
      const int32_t t = t0 + tt;
      int64_t off = -1;
      if (t < s1) off = token_offset(p, table, t);
      float kv = 0.f, vv = 0.f;
      if (off >= 0) {
        kv = to_float(kbase[off + d]);
        vv = to_float(vbase[off + d]);
      }
      ks[tt * (D + 1) + d] = kv;
      vs[tt * D + d] = vv;
      if (d == 0) tok_ok[tt] = off >= 0;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * kGenericTile; idx += blockDim.x) {
      const int g = idx / kGenericTile;
      const int tt = idx - g * kGenericTile;
      float s = kNegInf;
      if (tok_ok[tt]) {
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot += to_float(q[g * D + d]) * ks[tt * (D + 1) + d];
        s = dot * p.scale_log2;
      }
      sc[idx] = s;
    }
    __syncthreads();
    for (int g = threadIdx.x; g < G; g += blockDim.x) {
      float mx = kNegInf;
      for (int tt = 0; tt < kGenericTile; ++tt) mx = fmaxf(mx, sc[g * kGenericTile + tt]);
      const float m_new = fmaxf(m_run[g], mx);
      float a = 1.f, sum = 0.f;
      if (m_new != kNegInf) {
        a = exp2f(m_run[g] - m_new);
        for (int tt = 0; tt < kGenericTile; ++tt) {
          const float pr = exp2f(sc[g * kGenericTile + tt] - m_new);
          sc[g * kGenericTile + tt] = pr;
          sum += pr;
        }
      } else {
        for (int tt = 0; tt < kGenericTile; ++tt) sc[g * kGenericTile + tt] = 0.f;
      }
      l_run[g] = l_run[g] * a + sum;
      m_run[g] = m_new;
      alpha[g] = a;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kGenericMaxAcc; ++i) {
      const int idx = threadIdx.x + i * kGenericThreads;
      if (idx < G * D) {
        const int g = idx / D;
        const int d = idx - g * D;
        float a = acc[i] * alpha[g];
        for (int tt = 0; tt < kGenericTile; ++tt) a += sc[g * kGenericTile + tt] * vs[tt * D + d];
        acc[i] = a;
      }
    }
  }
  __syncthreads();
  finish<T, kGenericMaxAcc>(p, b, kvh * G, G, static_cast<int64_t>(b) * p.kv_heads + kvh, split, ctx,
                            [&](int k, int idx, float &m, float &l, float &num) {
                              const int g = idx / D;
                              m = m_run[g];
                              l = l_run[g];
                              num = acc[k];
                            });
}

size_t generic_lds_bytes(int D, int G) {
  return sizeof(float) * (static_cast<size_t>(kGenericTile) * (D + 1) +
                          static_cast<size_t>(kGenericTile) * D + static_cast<size_t>(G) * kGenericTile +
                          3 * static_cast<size_t>(G) + kGenericTile);
}

// ===========================================================================
// Log-sum-exp merge of split partials
// ===========================================================================
template <typename T, int NDIM>
__global__ void __launch_bounds__(256)
merge_partials_kernel(const float *__restrict__ partial_max, const float *__restrict__ partial_sum,
                      const float *__restrict__ partial_acc,
                      const int32_t *__restrict__ context_lengths, T *__restrict__ output,
                      int32_t query_heads, int32_t head_dim, int32_t split_size,
                      int32_t num_splits, int32_t partial_stride, int32_t max_tokens,
                      int32_t balanced) {
  // One workgroup of W wavefronts per (row, query head); NDIM = ceil(head_dim
  // / 64) accumulator elements per lane (dims lane + 64 k).  Lane s holds the
  // max and sum of split s (64 splits per pass) and, once the row's max and
  // denominator are known, the weight of split s; the weighted rows are
  // summed in batches of kBatch splits, every load of a batch in flight
  // together, each split's weight taken from its lane with a lane read.
  // Wavefront w takes batches w, w + W, ...; each batch's weighted sum
  // starts from zero and the batch sums are added in batch order (by
  // wavefront 0 through LDS when W > 1), so the result does not depend on W,
  // and a row of <= kBatch splits gives exactly the one batch's sum.  The
  // first batch of each wavefront is issued together with the max/sum loads
  // (before the row length is known), so a row with <= W kBatch splits costs
  // one memory round trip; loads of splits past the row's last one (clamped
  // to the last slot) are never used.
  constexpr int kBatch = 16;
  extern __shared__ float batch_sums[];  // [batches][NDIM][64] when W > 1
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int32_t qh = blockIdx.x;
  const int32_t b = blockIdx.y;
  const int64_t base = (static_cast<int64_t>(b) * query_heads + qh) * num_splits;
  T *out = output + (static_cast<int64_t>(b) * query_heads + qh) * head_dim;
  const float *acc_rows = partial_acc + base * partial_stride;
  int dim[NDIM];
#pragma unroll
  for (int k = 0; k < NDIM; ++k) dim[k] = min(lane + 64 * k, head_dim - 1);
  float v[kBatch][NDIM];
  auto load_batch = [&](int32_t s0) {
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const float *row = acc_rows + static_cast<int64_t>(min(s0 + j, num_splits - 1)) * partial_stride;
#pragma unroll
      for (int k = 0; k < NDIM; ++k) v[j][k] = row[dim[k]];
    }
  };
  const int32_t first = min(lane, num_splits - 1);
  const float m0 = partial_max[base + first];
  const float l0 = partial_sum[base + first];
  load_batch(kBatch * wave);
  int32_t ctx = context_lengths[b];
  ctx = ctx < 0 ? 0 : (ctx > max_tokens ? max_tokens : ctx);
  if (balanced) {
    int32_t unused;
    split_size = balanced_partition(context_lengths, static_cast<int32_t>(gridDim.y), max_tokens,
                                    split_size, num_splits, unused);
  }
  const int32_t nvalid = (ctx + split_size - 1) / split_size;
  // Max and sum over the valid splits (lanes beyond 64 splits in later passes).
  float gmax = kNegInf;
  for (int32_t s0 = 0; s0 < nvalid; s0 += 64) {
    const float ms = s0 == 0 ? m0 : partial_max[base + min(s0 + lane, num_splits - 1)];
    gmax = fmaxf(gmax, s0 + lane < nvalid ? ms : kNegInf);
  }
  gmax = wave64_max(gmax);
  float den = 0.f;
  if (gmax != kNegInf) {
    for (int32_t s0 = 0; s0 < nvalid; s0 += 64) {
      const int32_t sl = min(s0 + lane, num_splits - 1);
      const float ms = s0 == 0 ? m0 : partial_max[base + sl];
      const float ls = s0 == 0 ? l0 : partial_sum[base + sl];
      if (s0 + lane < nvalid && ms != kNegInf) den += ls * fast_exp2(ms - gmax);
    }
  }
  den = wave64_sum(den);
  const float inv = den > 0.f ? 1.f / den : 0.f;
  // Lane s's weight of split 64 pass + s (0 for a partial with no tokens).
  auto pass_weight = [&](int32_t pass) -> float {
    const float ms = pass == 0 ? m0 : partial_max[base + min(64 * pass + lane, num_splits - 1)];
    return ms == kNegInf ? 0.f : fast_exp2(ms - gmax) * inv;
  };
  int32_t pass = 0;
  float weight = pass_weight(0);
  const int32_t batches = (nvalid + kBatch - 1) / kBatch;
  float total[NDIM];
#pragma unroll
  for (int k = 0; k < NDIM; ++k) total[k] = 0.f;
  for (int32_t bi = wave; bi < batches; bi += W) {
    const int32_t s0 = bi * kBatch;
    if (bi != wave) load_batch(s0);
    if (s0 / 64 != pass) {
      pass = s0 / 64;
      weight = pass_weight(pass);
    }
    float num[NDIM];
#pragma unroll
    for (int k = 0; k < NDIM; ++k) num[k] = 0.f;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (s0 + j >= nvalid) break;
      const float w = lane_value(weight, (s0 + j) & 63);
#pragma unroll
      for (int k = 0; k < NDIM; ++k) num[k] = fmaf(w, v[j][k], num[k]);
    }
    if (W == 1) {
#pragma unroll
      for (int k = 0; k < NDIM; ++k) total[k] += num[k];
    } else {
#pragma unroll
      for (int k = 0; k < NDIM; ++k) batch_sums[(bi * NDIM + k) * 64 + lane] = num[k];
    }
  }
  if (W > 1) {  // workgroup-uniform
    __syncthreads();
    if (wave != 0) return;
    for (int32_t bi = 0; bi < batches; ++bi)
#pragma unroll
      for (int k = 0; k < NDIM; ++k) total[k] += batch_sums[(bi * NDIM + k) * 64 + lane];
  }
#pragma unroll
  for (int k = 0; k < NDIM; ++k) {
    const int d = lane + 64 * k;
    if (d < head_dim) out[d] = from_float<T>(total[k]);
  }
}

// ===========================================================================
// Host side
// ===========================================================================
int32_t choose_variant(int32_t dtype, int32_t head_dim, int32_t group, int32_t block_size,
                       int32_t flags) {
  if (flags & TF_ATTENTION_FLAG_FORCE_GENERIC) return TF_ATTENTION_GENERIC;
  if (dtype == TF_DTYPE_FLOAT32) return TF_ATTENTION_GENERIC;
  if (group > 16) return TF_ATTENTION_GENERIC;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return TF_ATTENTION_GENERIC;
  if (block_size % 16 != 0) return TF_ATTENTION_GENERIC;
  return TF_ATTENTION_MFMA;
}

// Wavefronts per MFMA grid workgroup (upper bound; the launch uses
// heads_per_wg * waves_per_head of them).
constexpr int kMfmaWaves = 8;

// Work split of the MFMA grid kernel: a workgroup serves HPW kv heads with
// WPH wavefronts per head (HPW * WPH <= 8), and with a token budget per
// wavefront (flag bits 24-30) a row uses only as many of the WPH as its
// length needs.  Without flags: one wavefront per (row, kv head, split),
// the fastest split-KV form.  The host plan of the Python entry point asks
// for one pass with WPH = ceil(L / 576) and a 576-token budget for wide
// batches (bits 20-23 / 8-15 / 24-30; HPW must divide kv_heads).
void mfma_geometry(AttnParams &p, int32_t flags) {
  int32_t hpw = 1;
  const int32_t want_hpw = (flags >> TF_ATTENTION_HEADS_PER_WG_SHIFT) & 0xf;
  if (want_hpw > 0 && want_hpw <= kMfmaWaves && p.kv_heads % want_hpw == 0) hpw = want_hpw;
  int32_t wph = 1;
  const int32_t want_wph = (flags >> TF_ATTENTION_WAVES_PER_CU_SHIFT) & 0xff;
  if (want_wph > 0 && want_wph * hpw <= kMfmaWaves) wph = want_wph;
  p.heads_per_wg = hpw;
  p.waves_per_head = wph;
  p.tokens_per_wave = ((flags >> TF_ATTENTION_TOKENS_PER_WAVE_SHIFT) & 0x7f) * 64;
}

// Whole-row loads (LINES) when several wavefronts stream one kv head: there
// a compute unit's load issue rate bounds the longest rows.  One wavefront
// per (row, kv head, split) is latency-bound and keeps the operand-layout
// loads, which need no LDS round trip for K.
template <typename T, int D, bool ROPE>
void launch_mfma_form(const AttnParams &p, dim3 grid, hipStream_t stream) {
  const int waves = p.heads_per_wg * p.waves_per_head;
  const size_t lds = static_cast<size_t>(mfma_lds_bytes(D, waves));
  if (p.waves_per_head > 1)
    hipLaunchKernelGGL((paged_decode_mfma_kernel<T, D, kMfmaWaves, ROPE, true>), grid,
                       dim3(waves * 64), lds, stream, p);
  else
    hipLaunchKernelGGL((paged_decode_mfma_kernel<T, D, kMfmaWaves, ROPE, false>), grid,
                       dim3(waves * 64), lds, stream, p);
}

// The VALU form of the one-pass / split kernel (TF_ATTENTION_FLAG_VALU): the
// same grid, loads and LDS staging (whole token rows, K staged token-major),
// with the score and P.V products on the VALU; head_dim 64 without RoPE.
template <typename T>
void launch_valu(const AttnParams &p, dim3 grid, hipStream_t stream) {
  const int waves = p.heads_per_wg * p.waves_per_head;
  const size_t lds = static_cast<size_t>(mfma_lds_bytes(64, waves)) +
                     static_cast<size_t>(waves) * 16 * kChunk * sizeof(float);
  hipLaunchKernelGGL((paged_decode_mfma_kernel<T, 64, kMfmaWaves, false, true, true>), grid,
                     dim3(waves * 64), lds, stream, p);
}

template <typename T, int D>
void launch_mfma(const AttnParams &p, dim3 grid, hipStream_t stream) {
  if (p.rope_qkv)
    launch_mfma_form<T, D, true>(p, grid, stream);
  else
    launch_mfma_form<T, D, false>(p, grid, stream);
}

template <typename T>
void launch_mfma_dim(const AttnParams &p, dim3 grid, hipStream_t stream) {
  switch (p.head_dim) {
    case 32: launch_mfma<T, 32>(p, grid, stream); break;
    case 64: launch_mfma<T, 64>(p, grid, stream); break;
    default: launch_mfma<T, 128>(p, grid, stream); break;
  }
}

int32_t validate(const void *query, const void *key_cache, const void *value_cache,
                 const int32_t *block_tables, const int32_t *context_lengths, int32_t batch,
                 int32_t query_heads, int32_t kv_heads, int32_t head_dim, int32_t num_blocks,
                 int32_t block_size, int32_t table_width, int32_t split_size, int32_t num_splits,
                 int32_t dtype) {
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (batch < 0 || query_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || num_blocks <= 0 ||
      block_size <= 0 || table_width <= 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "attention dimensions must be positive");
  if (query_heads % kv_heads != 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "query heads must be a multiple of kv heads");
  if (head_dim > 256) return fail(TF_ERROR_INVALID_ARGUMENT, "head_dim must be <= 256");
  if (split_size <= 0 || num_splits <= 0 || num_splits > 65535)
    return fail(TF_ERROR_INVALID_ARGUMENT, "split_size and num_splits must be positive");
  if (batch > 65535 || kv_heads > 65535) return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  if (batch > 0 && (!query || !key_cache || !value_cache || !block_tables || !context_lengths))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  return TF_SUCCESS;
}

int32_t make_params(AttnParams &p, const void *query, const void *key_cache,
                    const void *value_cache, const int32_t *block_tables,
                    const int32_t *context_lengths, void *output, float *partial_max,
                    float *partial_sum, float *partial_acc, int32_t *split_counters,
                    int64_t partial_capacity, int32_t partial_row_stride, int32_t batch,
                    int32_t query_heads,
                    int32_t kv_heads, int32_t head_dim, int32_t num_blocks, int32_t block_size,
                    int32_t table_width, int32_t split_size, int32_t num_splits, float scale,
                    int32_t dtype) {
  if (int32_t s = validate(query, key_cache, value_cache, block_tables, context_lengths, batch,
                           query_heads, kv_heads, head_dim, num_blocks, block_size, table_width,
                           split_size, num_splits, dtype))
    return s;
  if (num_splits > 1) {
    if (!partial_max || !partial_sum || !partial_acc)
      return fail(TF_ERROR_INVALID_ARGUMENT, "split attention needs partial buffers");
    if (partial_row_stride < head_dim)
      return fail(TF_ERROR_INVALID_ARGUMENT, "partial row stride is smaller than head_dim");
    if (partial_capacity < static_cast<int64_t>(batch) * query_heads * num_splits)
      return fail(TF_ERROR_INVALID_ARGUMENT, "partial buffers are too small");
  }
  p.query = query;
  p.key_cache = key_cache;
  p.value_cache = value_cache;
  p.block_tables = block_tables;
  p.context_lengths = context_lengths;
  p.output = output;
  p.partial_max = partial_max;
  p.partial_sum = partial_sum;
  p.partial_acc = partial_acc;
  p.split_counters = num_splits > 1 ? split_counters : nullptr;
  p.batch = batch;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.group = query_heads / kv_heads;
  p.head_dim = head_dim;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.page_shift = -1;
  if ((block_size & (block_size - 1)) == 0) p.page_shift = __builtin_ctz(block_size);
  p.table_width = table_width;
  p.split_size = split_size;
  p.num_splits = num_splits;
  p.partial_stride = partial_row_stride;
  const int64_t split_tokens = static_cast<int64_t>(num_splits) * split_size;
  const int64_t table_tokens = static_cast<int64_t>(table_width) * block_size;
  int64_t max_tokens = split_tokens < table_tokens ? split_tokens : table_tokens;
  if (max_tokens > 0x7fffffff) max_tokens = 0x7fffffff;
  p.max_tokens = static_cast<int32_t>(max_tokens);
  p.partial_rows = partial_capacity;
  p.heads_per_wg = 1;
  p.waves_per_head = 1;
  p.tokens_per_wave = 0;
  p.balanced = 0;
  p.scale_log2 = scale * kLog2e;
  p.rope_qkv = nullptr;
  p.rope_row_stride = 0;
  p.rope_positions = nullptr;
  p.rope_cos = nullptr;
  p.rope_sin = nullptr;
  p.rope_table_rows = 0;
  p.append_pages = nullptr;
  p.append_offsets = nullptr;
  p.append_active = nullptr;
  return TF_SUCCESS;
}

// Flag bits with no meaning in this ABI (bit 2 once selected a streaming
// kernel that has been removed, bits 16-19 its pipeline depth).
constexpr int32_t kUnknownFlagBits = 0x2 | 0x4 | 0x8 | 0x40 | 0x80 | 0xF0000;

int32_t launch_split_stage(const AttnParams &p, int32_t dtype, int32_t flags, hipStream_t stream) {
  if (flags & kUnknownFlagBits)
    return fail(TF_ERROR_UNSUPPORTED, "unknown attention flag bits");
  if (p.batch == 0) return TF_SUCCESS;
  const bool balanced = (flags & TF_ATTENTION_FLAG_BALANCED) != 0;
  if (balanced &&
      (choose_variant(dtype, p.head_dim, p.group, p.block_size, flags) != TF_ATTENTION_MFMA ||
       (flags & TF_ATTENTION_FLAG_VALU) || p.num_splits <= p.batch ||
       p.batch > 64 || p.split_counters != nullptr || p.split_size % 32 != 0))
    return fail(TF_ERROR_UNSUPPORTED,
                "balanced partitions need the MFMA grid kernel in split-KV mode with the merge "
                "launch (no arrival counters, no VALU flag), num_splits > batch, "
                "batch <= 64 and split_size % 32 == 0");
  const dim3 grid(static_cast<unsigned>(p.batch) * static_cast<unsigned>(p.kv_heads),
                  static_cast<unsigned>(p.num_splits));
  int32_t variant = choose_variant(dtype, p.head_dim, p.group, p.block_size, flags);
  // The MFMA kernel's tiles start at multiples of 16 tokens of a split.
  if (p.num_splits > 1 && p.split_size % 32 != 0) variant = TF_ATTENTION_GENERIC;
  if (variant == TF_ATTENTION_MFMA) {
    AttnParams q = p;
    mfma_geometry(q, flags);
    q.balanced = balanced ? 1 : 0;
    const unsigned groups = static_cast<unsigned>(p.kv_heads / q.heads_per_wg);
    const dim3 mgrid = balanced ? dim3(groups * static_cast<unsigned>(p.num_splits), 1)
                                : dim3(static_cast<unsigned>(p.batch) * groups,
                                       static_cast<unsigned>(p.num_splits));
    if (flags & TF_ATTENTION_FLAG_VALU) {
      if (p.head_dim != 64 || p.rope_qkv != nullptr)
        return fail(TF_ERROR_UNSUPPORTED, "the VALU attention form supports head_dim 64 without RoPE");
      if (dtype == TF_DTYPE_BFLOAT16)
        launch_valu<__bf16>(q, mgrid, stream);
      else
        launch_valu<_Float16>(q, mgrid, stream);
      return check_launch("paged_gqa_decode (valu)");
    }
    if (dtype == TF_DTYPE_BFLOAT16)
      launch_mfma_dim<__bf16>(q, mgrid, stream);
    else
      launch_mfma_dim<_Float16>(q, mgrid, stream);
    return check_launch("paged_gqa_decode (mfma)");
  }
  if (p.group > 64 || p.group * p.head_dim > kGenericThreads * kGenericMaxAcc)
    return fail(TF_ERROR_UNSUPPORTED,
                "generic attention supports group <= 64 and group * head_dim <= 8192");
  const size_t lds = generic_lds_bytes(p.head_dim, p.group);
  switch (dtype) {
    case TF_DTYPE_FLOAT32:
      hipLaunchKernelGGL(paged_decode_generic_kernel<float>, grid, dim3(kGenericThreads), lds,
                         stream, p);
      break;
    case TF_DTYPE_FLOAT16:
      hipLaunchKernelGGL(paged_decode_generic_kernel<_Float16>, grid, dim3(kGenericThreads), lds,
                         stream, p);
      break;
    default:
      hipLaunchKernelGGL(paged_decode_generic_kernel<__bf16>, grid, dim3(kGenericThreads), lds,
                         stream, p);
      break;
  }
  return check_launch("paged_gqa_decode (generic)");
}


int32_t launch_merge(const float *partial_max, const float *partial_sum, const float *partial_acc,
                     const int32_t *context_lengths, void *output, int32_t batch,
                     int32_t query_heads, int32_t head_dim, int32_t split_size, int32_t num_splits,
                     int32_t partial_stride, int32_t max_tokens, int32_t dtype,
                     hipStream_t stream, bool balanced = false) {
  const int32_t bal = balanced ? 1 : 0;
  if (batch == 0) return TF_SUCCESS;
  const dim3 grid(static_cast<unsigned>(query_heads), static_cast<unsigned>(batch));
  // Up to four wavefronts per (row, head) when a row may have more than one
  // 16-split batch, so the batches' loads are in flight together; their
  // batch sums meet in LDS (1 KB per batch and 64 dims), so beyond 16
  // batches one wavefront walks them.
  const int32_t batches = (num_splits + 15) / 16;
  const int waves = batches <= 1 || batches > 16 ? 1 : (batches < 4 ? batches : 4);
  const dim3 block(64u * static_cast<unsigned>(waves));
  const int ndim = (head_dim + 63) / 64;  // accumulator elements per lane
  if (ndim < 1 || ndim > 4) return fail(TF_ERROR_INVALID_ARGUMENT, "merge: head_dim must be in [1, 256]");
  const size_t lds = waves > 1 ? static_cast<size_t>(batches) * ndim * 64 * sizeof(float) : 0;
  auto launch = [&](auto kernel, auto *out) {
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, partial_max, partial_sum, partial_acc,
                       context_lengths, out, query_heads, head_dim, split_size, num_splits,
                       partial_stride, max_tokens, bal);
  };
  auto by_width = [&](auto *out) {
    using T = std::remove_pointer_t<decltype(out)>;
    switch (ndim) {
      case 1: launch(merge_partials_kernel<T, 1>, out); break;
      case 2: launch(merge_partials_kernel<T, 2>, out); break;
      case 3: launch(merge_partials_kernel<T, 3>, out); break;
      default: launch(merge_partials_kernel<T, 4>, out); break;
    }
  };
  switch (dtype) {
    case TF_DTYPE_FLOAT32: by_width(static_cast<float *>(output)); break;
    case TF_DTYPE_FLOAT16: by_width(static_cast<_Float16 *>(output)); break;
    default: by_width(static_cast<__bf16 *>(output)); break;
  }
  return check_launch("paged_gqa_decode merge");
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_paged_gqa_decode_variant(int32_t dtype, int32_t head_dim, int32_t group_size,
                                               int32_t block_size, int32_t flags) {
  return tf::choose_variant(dtype, head_dim, group_size, block_size, flags);
}

extern "C" int32_t tf_paged_gqa_decode(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths, void *output,
    float *partial_max, float *partial_sum, float *partial_accumulator,
    int32_t *split_counters, int64_t partial_capacity, int32_t partial_row_stride, int32_t batch,
    int32_t query_heads, int32_t kv_heads, int32_t head_dim, int32_t num_blocks,
    int32_t block_size, int32_t table_width, int32_t split_size, int32_t num_splits, float scale,
    int32_t dtype, int32_t flags, void *stream) {
  using namespace tf;
  clear_error();
  if (batch > 0 && !output) return fail(TF_ERROR_INVALID_ARGUMENT, "null output pointer");
  AttnParams p;
  if (int32_t s = make_params(p, query, key_cache, value_cache, block_tables, context_lengths,
                              output, partial_max, partial_sum, partial_accumulator,
                              split_counters, partial_capacity, partial_row_stride, batch, query_heads, kv_heads,
                              head_dim, num_blocks, block_size, table_width, split_size,
                              num_splits, scale, dtype))
    return s;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int32_t st = launch_split_stage(p, dtype, flags, s)) return st;
  if (num_splits == 1 || split_counters != nullptr) return TF_SUCCESS;
  return launch_merge(partial_max, partial_sum, partial_accumulator, context_lengths, output,
                      batch, query_heads, head_dim, split_size, num_splits, partial_row_stride,
                      p.max_tokens, dtype, s, (flags & TF_ATTENTION_FLAG_BALANCED) != 0);
}

extern "C" int32_t tf_paged_gqa_decode_rope_append(
    const void *qkv, int64_t qkv_row_stride, const int64_t *positions, const void *cos_table,
    const void *sin_table, int32_t table_rows, void *key_cache, void *value_cache,
    const int32_t *append_pages, const int32_t *append_offsets, const int32_t *active_mask,
    const int32_t *block_tables, const int32_t *context_lengths, void *output,
    float *partial_max, float *partial_sum, float *partial_accumulator,
    int32_t *split_counters, int64_t partial_capacity, int32_t partial_row_stride, int32_t batch,
    int32_t query_heads, int32_t kv_heads, int32_t head_dim, int32_t num_blocks,
    int32_t block_size, int32_t table_width, int32_t split_size, int32_t num_splits, float scale,
    int32_t dtype, int32_t flags, void *stream) {
  using namespace tf;
  clear_error();
  if (batch > 0 && !output) return fail(TF_ERROR_INVALID_ARGUMENT, "null output pointer");
  if (table_rows <= 0 || (head_dim & 1))
    return fail(TF_ERROR_INVALID_ARGUMENT, "table rows must be positive and head_dim even");
  if (qkv_row_stride < static_cast<int64_t>(query_heads + 2 * kv_heads) * head_dim)
    return fail(TF_ERROR_INVALID_ARGUMENT, "qkv row stride is shorter than the q, k, v heads");
  if (batch > 0 && (!qkv || !positions || !cos_table || !sin_table || !append_pages ||
                    !append_offsets || !active_mask))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if (choose_variant(dtype, head_dim, query_heads / (kv_heads > 0 ? kv_heads : 1), block_size,
                     flags) != TF_ATTENTION_MFMA ||
      (num_splits > 1 && split_size % 32 != 0))
    return fail(TF_ERROR_UNSUPPORTED,
                "fused RoPE + append attention needs the MFMA grid kernel (bf16/fp16, head_dim "
                "32/64/128, group <= 16, block_size % 16 == 0, split_size % 32 == 0)");
  AttnParams p;
  // `qkv` stands in for the query pointer in the common validation.
  if (int32_t st = make_params(p, qkv, key_cache, value_cache, block_tables, context_lengths,
                               output, partial_max, partial_sum, partial_accumulator,
                               split_counters, partial_capacity, partial_row_stride, batch,
                               query_heads, kv_heads, head_dim, num_blocks, block_size,
                               table_width, split_size, num_splits, scale, dtype))
    return st;
  p.query = nullptr;
  p.rope_qkv = qkv;
  p.rope_row_stride = qkv_row_stride;
  p.rope_positions = positions;
  p.rope_cos = cos_table;
  p.rope_sin = sin_table;
  p.rope_table_rows = table_rows;
  p.append_pages = append_pages;
  p.append_offsets = append_offsets;
  p.append_active = active_mask;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int32_t st = launch_split_stage(p, dtype, flags, s)) return st;
  if (num_splits == 1 || split_counters != nullptr) return TF_SUCCESS;
  return launch_merge(partial_max, partial_sum, partial_accumulator, context_lengths, output,
                      batch, query_heads, head_dim, split_size, num_splits, partial_row_stride,
                      p.max_tokens, dtype, s, (flags & TF_ATTENTION_FLAG_BALANCED) != 0);
}

extern "C" int32_t tf_paged_gqa_decode_partials(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths, float *partial_max,
    float *partial_sum, float *partial_accumulator, int64_t partial_capacity,
    int32_t partial_row_stride, int32_t batch, int32_t query_heads, int32_t kv_heads,
    int32_t head_dim, int32_t num_blocks, int32_t block_size, int32_t table_width,
    int32_t split_size, int32_t num_splits, float scale, int32_t dtype, int32_t flags,
    void *stream) {
  using namespace tf;
  clear_error();
  if (!partial_max || !partial_sum || !partial_accumulator)
    return fail(TF_ERROR_INVALID_ARGUMENT, "partials stage needs partial buffers");
  if (num_splits < 2) return fail(TF_ERROR_INVALID_ARGUMENT, "partials stage needs num_splits >= 2");
  if (flags & TF_ATTENTION_FLAG_BALANCED)
    return fail(TF_ERROR_UNSUPPORTED,
                "the partials stage takes fixed partitions (tf_paged_gqa_decode_merge has no "
                "balanced form)");
  AttnParams p;
  if (int32_t s = make_params(p, query, key_cache, value_cache, block_tables, context_lengths,
                              nullptr, partial_max, partial_sum, partial_accumulator,
                              nullptr, partial_capacity, partial_row_stride, batch, query_heads, kv_heads,
                              head_dim, num_blocks, block_size, table_width, split_size,
                              num_splits, scale, dtype))
    return s;
  return launch_split_stage(p, dtype, flags, static_cast<hipStream_t>(stream));
}

extern "C" int32_t tf_paged_gqa_decode_merge(
    const float *partial_max, const float *partial_sum, const float *partial_accumulator,
    const int32_t *context_lengths, void *output, int64_t partial_capacity,
    int32_t partial_row_stride, int32_t batch, int32_t query_heads, int32_t head_dim,
    int32_t split_size, int32_t num_splits, int32_t max_tokens, int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (batch < 0 || query_heads <= 0 || head_dim <= 0 || head_dim > 256 || split_size <= 0 ||
      num_splits <= 0 || max_tokens < 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "merge dimensions out of range");
  if (batch > 65535 || query_heads > 65535) return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  if (partial_row_stride < head_dim)
    return fail(TF_ERROR_INVALID_ARGUMENT, "partial row stride is smaller than head_dim");
  if (partial_capacity < static_cast<int64_t>(batch) * query_heads * num_splits)
    return fail(TF_ERROR_INVALID_ARGUMENT, "partial buffers are too small");
  if (batch > 0 && (!partial_max || !partial_sum || !partial_accumulator || !context_lengths ||
                    !output))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const int64_t split_tokens = static_cast<int64_t>(num_splits) * split_size;
  const int32_t clamp =
      static_cast<int32_t>(split_tokens < max_tokens ? split_tokens : max_tokens);
  return launch_merge(partial_max, partial_sum, partial_accumulator, context_lengths, output,
                      batch, query_heads, head_dim, split_size, num_splits, partial_row_stride,
                      clamp, dtype, static_cast<hipStream_t>(stream));
}

// ===========================================================================
// tf_paged_gqa_decode_noalloc: the same call with no caller workspace
// ===========================================================================
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).  The
// split partials live in `scratch`, a fixed array of this library that every
// GPU holds in its own memory until the process ends.  In host code the
// array's name is only a stand-in: the device address comes from
// hipGetSymbolAddress, taken once per device (with that device current) on
// the first call there, and only that address is passed to kernels.  The
// split kernel writes every partial the merge reads (empty splits are never
// read), so nothing in `scratch` has to start at zero; arrival counters are
// not used (no in-kernel merge).  Every call on a GPU shares
// that GPU's array: calls that overlap in time on one GPU race.

static __device__ __align__(256) unsigned char scratch[TF_NOALLOC_SCRATCH_BYTES];

namespace tf {
namespace {

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_lock;
void *g_scratch_address[kScratchMaxDevices] = {};

// Device address of `scratch` on the current device.
int32_t scratch_address(void **out) {
  int device = -1;
  const hipError_t got = hipGetDevice(&device);
  if (got != hipSuccess || device < 0 || device >= kScratchMaxDevices) {
    set_error("no usable current HIP device for the attention scratch (%s)",
              hipGetErrorString(got));
    return TF_ERROR_LAUNCH;
  }
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_address[device] == nullptr) {
    void *address = nullptr;
    const hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess || address == nullptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                hipGetErrorString(err));
      return TF_ERROR_LAUNCH;
    }
    g_scratch_address[device] = address;
  }
  *out = g_scratch_address[device];
  return TF_SUCCESS;
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_paged_gqa_decode_noalloc(
    const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lengths, void *output, int32_t batch,
    int32_t query_heads, int32_t kv_heads, int32_t head_dim, int32_t num_blocks,
    int32_t block_size, int32_t table_width, int32_t split_size, int32_t num_splits, float scale,
    int32_t dtype, int32_t flags, void *stream) {
  using namespace tf;
  clear_error();
  if (flags & kUnknownFlagBits) return fail(TF_ERROR_UNSUPPORTED, "unknown attention flag bits");
  if (batch < 0 || query_heads <= 0 || head_dim <= 0 || head_dim > 256 || num_splits <= 0)
    return fail(TF_ERROR_INVALID_ARGUMENT, "attention dimensions out of range");
  // Partials as the workspace lays them out: accumulator rows of
  // next_pow2(head_dim) floats, then the maxima, then the sums.
  int32_t stride = 1;
  while (stride < head_dim) stride <<= 1;
  const int64_t rows =
      num_splits > 1 ? static_cast<int64_t>(batch) * query_heads * num_splits : 0;
  const int64_t bytes = rows * (stride + 2) * static_cast<int64_t>(sizeof(float));
  if (bytes > TF_NOALLOC_SCRATCH_BYTES) {
    set_error("split partials of %lld rows need %lld bytes; the no-allocation scratch holds "
              "%lld (use fewer splits or tf_paged_gqa_decode with a workspace)",
              static_cast<long long>(rows), static_cast<long long>(bytes),
              static_cast<long long>(TF_NOALLOC_SCRATCH_BYTES));
    return TF_ERROR_INVALID_ARGUMENT;
  }
  if (batch > 0 && !output) return fail(TF_ERROR_INVALID_ARGUMENT, "null output pointer");
  void *base = nullptr;
  if (int32_t st = scratch_address(&base)) return st;
  float *partial_acc = static_cast<float *>(base);
  float *partial_max = partial_acc + rows * stride;
  float *partial_sum = partial_max + rows;
  AttnParams p;
  if (int32_t st = make_params(p, query, key_cache, value_cache, block_tables, context_lengths,
                               output, partial_max, partial_sum, partial_acc, nullptr, rows,
                               stride, batch, query_heads, kv_heads, head_dim, num_blocks,
                               block_size, table_width, split_size, num_splits, scale, dtype))
    return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int32_t st = launch_split_stage(p, dtype, flags, s)) return st;
  if (num_splits == 1) return TF_SUCCESS;
  return launch_merge(partial_max, partial_sum, partial_acc, context_lengths, output, batch,
                      query_heads, head_dim, split_size, num_splits, stride, p.max_tokens, dtype,
                      s, (flags & TF_ATTENTION_FLAG_BALANCED) != 0);
}
