// Decode-shaped linear layers on MFMA for up to 64 rows.  This file holds
//   * tf_linear_partials / tf_linear_partials_sum -- split-K slices with
//     operands loaded in the MFMA operand layout (below);
//   * tf_linear_stream -- the same products (or a one-slice rounded output)
//     with both operands staged through LDS by whole-row loads;
//   * tf_linear_swiglu -- its form for the stacked gate|up weight with the
//     SwiGLU in the epilogue;
//   * tf_linear_kstream / tf_linear_kswiglu -- K split over the wavefronts
//     of 16-column workgroups, for narrow weights and for gate|up + SwiGLU.
//
// Split-K form:
//   partials[s][m][n] = sum over k in slice s of x[m][k] * w[n][k]   (fp32)
// and the row sum y[m][n] = round(sum_s partials[s][m][n]).
//
// At decode batch sizes a projection streams its weight matrix once (each
// element is used M <= 64 times) and is HBM-bound; what a library GEMM
// tiled for large M lacks is parallelism -- a 2048 x 2048 weight in 64 x 64
// output tiles is 32 workgroups.  Here blockIdx.x is a 64-column tile and
// blockIdx.y one of S slices of K, so a launch has (N / 64) * S workgroups
// each streaming a 64-row slab of w that is K / S long.  Inside a workgroup
// the four wavefronts split the slice's 32-wide k-steps between them and
// each accumulates the whole 64 x 64 tile (4 row tiles x 4 column tiles of
// v_mfma_f32_16x16x32), so a wavefront reads as many bytes of x as of w (x
// is small and stays in L2; a 16-column tiling would read x four times as
// often as w).  Up to four k-steps of loads (w and x) are issued together.
// The four wavefront tiles are summed once in LDS and stored as the
// slice's fp32 partial; the reduction over the S slices is left to the
// consumer of y (tf_linear_partials_sum here, or a fused consumer), so the
// launch needs no atomics, counters or second pass of its own.
//
// MFMA v_mfma_f32_16x16x32 (bf16 / f16):
//   A = x rows:  lane (l16, q4) holds x[16 mt + l16][k + 8 q4 .. +8]
//   B = w rows:  lane (l16, q4) holds w[n0 + 16 nt + l16][k + 8 q4 .. +8]
//   C:           lane (l16, q4), register r holds y[16 mt + 4 q4 + r][n0 + 16 nt + l16]
//
// Reference semantics: torch.nn.functional.linear(x, w) without bias (fp32
// accumulation, one rounding to the storage type), the nn.Linear
// projections of tensorforge/model/layers.py:88-95, 144-146 as the decode
// step calls them (tensorforge/runtime/decode_bucket.py:441-447, 470,
// 500-505).
#include "tf_common.hpp"

#include <atomic>

namespace tf {
namespace {

template <typename T>
struct SplitMma;

template <>
struct SplitMma<__bf16> {
  typedef __bf16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct SplitMma<_Float16> {
  typedef _Float16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kSplitWaves = 4;    // wavefronts per workgroup
constexpr int kSplitCols = 64;    // output columns per workgroup
constexpr int kSplitUnroll = 4;   // k-steps of loads in flight per wavefront

template <typename T, int MT>
__global__ void __launch_bounds__(kSplitWaves * 64)
linear_partials_kernel(const T *__restrict__ x, int64_t x_stride, const T *__restrict__ w,
                       int64_t w_stride, float *__restrict__ partials, int32_t m, int32_t n,
                       int32_t k, int32_t k_per_split) {
  using M = SplitMma<T>;
  using vec8 = typename M::vec8;
  constexpr int NT = kSplitCols / 16;
  constexpr int kItems = MT * NT * 4 * 64;  // floats of one wavefront's tile
  extern __shared__ __attribute__((aligned(16))) float tile_sums[];  // [waves][kItems]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int32_t n0 = blockIdx.x * kSplitCols;
  const int32_t split = blockIdx.y;
  const int32_t s0 = split * k_per_split;
  const int32_t s1 = min(s0 + k_per_split, k);
  // k-steps of the slice, dealt to the wavefronts in contiguous runs.
  const int32_t steps = (s1 - s0) / 32;
  const int32_t per_wave = (steps + kSplitWaves - 1) / kSplitWaves;
  const int32_t k0 = s0 + 32 * min(wave * per_wave, steps);
  const int32_t k1 = s0 + 32 * min((wave + 1) * per_wave, steps);

  const T *wrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    wrow[nt] = w + static_cast<int64_t>(min(n0 + 16 * nt + l16, n - 1)) * w_stride + 8 * q4;
  const T *xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = x + static_cast<int64_t>(min(16 * mt + l16, m - 1)) * x_stride + 8 * q4;

  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Batches of kSplitUnroll k-steps: every load of a batch is issued before
  // its MFMAs; steps past k1 load the batch's first step again and are
  // zeroed, so the loads stay unconditional.
  for (int32_t kk = k0; kk < k1; kk += 32 * kSplitUnroll) {
    vec8 wb[kSplitUnroll][NT];
    vec8 xa[kSplitUnroll][MT];
#pragma unroll
    for (int u = 0; u < kSplitUnroll; ++u) {
      const int32_t ku = kk + 32 * u < k1 ? kk + 32 * u : kk;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) wb[u][nt] = *reinterpret_cast<const vec8 *>(wrow[nt] + ku);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xa[u][mt] = *reinterpret_cast<const vec8 *>(xrow[mt] + ku);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kSplitUnroll; ++u) {
      if (kk + 32 * u >= k1) break;  // uniform
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = M::mma(xa[u][mt], wb[u][nt], acc[mt][nt]);
    }
  }

  // Sum the wavefront tiles: item (mt, nt, r, lane).
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        tile_sums[wave * kItems + ((mt * NT + nt) * 4 + r) * 64 + lane] = acc[mt][nt][r];
  __syncthreads();
  float *out = partials + static_cast<int64_t>(split) * m * n;
  for (int item = threadIdx.x; item < kItems; item += blockDim.x) {
    float sum = 0.f;
#pragma unroll
    for (int wv = 0; wv < kSplitWaves; ++wv) sum += tile_sums[wv * kItems + item];
    const int il = item & 63;
    const int r = (item >> 6) & 3;
    const int tile = item >> 8;
    const int mt = tile / NT;
    const int nt = tile - mt * NT;
    const int32_t row = 16 * mt + 4 * (il >> 4) + r;
    const int32_t col = n0 + 16 * nt + (il & 15);
    if (row < m && col < n) out[static_cast<int64_t>(row) * n + col] = sum;
  }
}

// ---------------------------------------------------------------------------
// Weight-streaming form (tf_linear_stream).  A load in the MFMA operand
// layout (lane (l16, q4) reading 16 bytes of row l16) touches 16 rows x half
// a 128-byte line, and a compute unit issues such loads at <= 34 GB/s even
// when they hit L2; whole-row loads run at ~85 GB/s from L2 and stream HBM
// ~10% faster.  Here a workgroup stages 256-wide k chunks of x (16 MT rows)
// and of its 64 weight rows in LDS with whole-row loads (32 threads per
// 512-byte row piece), with the next two chunks' loads in flight in
// registers while the MFMAs read the current one, and each wavefront owns
// 16 output columns over the whole slice -- no cross-wavefront sum.  LDS
// rows are 512 bytes with their 16-byte pieces permuted by
// (piece ^ (row & 15)), so the 16 rows an operand read touches at one k
// fall in distinct banks.
// ---------------------------------------------------------------------------
constexpr int kStreamCols = 64;    // output columns per workgroup (4 wavefronts x 16)
constexpr int kStreamChunk = 256;  // k per LDS chunk (one 512-byte row)

__device__ __forceinline__ int stream_lds_offset(int row, int piece) {
  return row * kStreamChunk + ((piece ^ (row & 15)) << 3);
}

// SWIGLU: the weight stacks gate rows [0, n) over up rows [n, 2n) and the
// workgroup covers 32 output columns j: wavefronts 0-1 compute the gate
// columns and 2-3 the matching up columns, which reach 0-1 through LDS; the
// output is round(swiglu_act(round(g), round(u))), the SwiGLU of the
// rounded projection.
template <typename T, int MT, bool SWIGLU>
__global__ void __launch_bounds__(256)
linear_stream_kernel(const T *__restrict__ x, int64_t x_stride, const T *__restrict__ w,
                     int64_t w_stride, T *__restrict__ y, int64_t y_stride,
                     float *__restrict__ partials, int32_t m, int32_t n, int32_t k,
                     int32_t k_per_split) {
  using M = SplitMma<T>;
  using vec8 = typename M::vec8;
  constexpr int XR = 16 * MT;
  constexpr int kLoadsX = XR / 8;           // 16-byte loads per thread per chunk
  constexpr int kLoadsW = kStreamCols / 8;
  extern __shared__ __attribute__((aligned(16))) unsigned char stream_smem[];
  T *xl = reinterpret_cast<T *>(stream_smem);  // [XR][256], swizzled pieces
  T *wl = xl + XR * kStreamChunk;              // [64][256]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int32_t n0 = blockIdx.x * (SWIGLU ? kStreamCols / 2 : kStreamCols);
  const int32_t split = blockIdx.y;
  const int32_t s0 = split * k_per_split;
  const int32_t s1 = min(s0 + k_per_split, k);
  // Staging map: thread t loads piece t % 32 of row 8 i + t / 32.
  const int lrow = tid >> 5;
  const int lpiece = tid & 31;

  const T *xsrc[kLoadsX];
#pragma unroll
  for (int i = 0; i < kLoadsX; ++i)
    xsrc[i] = x + static_cast<int64_t>(min(8 * i + lrow, m - 1)) * x_stride + 8 * lpiece;
  const T *wsrc[kLoadsW];
#pragma unroll
  for (int i = 0; i < kLoadsW; ++i) {
    const int tr = 8 * i + lrow;  // tile row
    const int64_t row = SWIGLU ? (tr < 32 ? 0 : n) + min(n0 + (tr & 31), n - 1)
                               : min(n0 + tr, n - 1);
    wsrc[i] = w + row * w_stride + 8 * lpiece;
  }

  // Two register sets: while the MFMAs read chunk c from LDS, the loads of
  // chunks c + 1 and c + 2 are in flight (128 KB per workgroup at MT = 4).
  vec8 xa[kLoadsX], wa[kLoadsW], xb[kLoadsX], wb[kLoadsW];
  // Pieces past K (only in a last, partial chunk) read the row's first
  // piece instead; pieces past the slice but inside K are read and unused.
  auto load_chunk = [&](int32_t kk, vec8(&xr)[kLoadsX], vec8(&wr)[kLoadsW]) {
    const int32_t c = kk + 8 * lpiece < k ? kk : -8 * lpiece;
#pragma unroll
    for (int i = 0; i < kLoadsX; ++i) xr[i] = *reinterpret_cast<const vec8 *>(xsrc[i] + c);
#pragma unroll
    for (int i = 0; i < kLoadsW; ++i) wr[i] = *reinterpret_cast<const vec8 *>(wsrc[i] + c);
  };
  auto stage_chunk = [&](const vec8(&xr)[kLoadsX], const vec8(&wr)[kLoadsW]) {
    __syncthreads();  // the previous chunk's operand reads are done
#pragma unroll
    for (int i = 0; i < kLoadsX; ++i)
      *reinterpret_cast<vec8 *>(xl + stream_lds_offset(8 * i + lrow, lpiece)) = xr[i];
#pragma unroll
    for (int i = 0; i < kLoadsW; ++i)
      *reinterpret_cast<vec8 *>(wl + stream_lds_offset(8 * i + lrow, lpiece)) = wr[i];
    __syncthreads();
  };

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute_chunk = [&](int32_t kk) {
    const int32_t steps = min(kStreamChunk, s1 - kk) >> 5;
#pragma unroll
    for (int st = 0; st < kStreamChunk / 32; ++st) {
      if (st >= steps) break;  // uniform
      const int piece = 4 * st + q4;
      const vec8 b = *reinterpret_cast<const vec8 *>(wl + stream_lds_offset(16 * wave + l16, piece));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = M::mma(*reinterpret_cast<const vec8 *>(xl + stream_lds_offset(16 * mt + l16, piece)),
                         b, acc[mt]);
    }
  };

  constexpr int32_t C = kStreamChunk;
  load_chunk(s0, xa, wa);
  if (s0 + C < s1) load_chunk(s0 + C, xb, wb);
  for (int32_t kk = s0; kk < s1; kk += 2 * C) {
    stage_chunk(xa, wa);
    if (kk + 2 * C < s1) load_chunk(kk + 2 * C, xa, wa);
    compute_chunk(kk);
    if (kk + C >= s1) break;
    stage_chunk(xb, wb);
    if (kk + 3 * C < s1) load_chunk(kk + 3 * C, xb, wb);
    compute_chunk(kk + C);
  }

  // C layout: lane (l16, q4), register r holds y[16 mt + 4 q4 + r][n0 + 16 wave + l16].
  if constexpr (SWIGLU) {
    float *up = reinterpret_cast<float *>(stream_smem);  // [2 waves][MT * 4][64 lanes]
    __syncthreads();  // the last chunk's operand reads are done
    if (wave >= 2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          up[((wave - 2) * MT * 4 + mt * 4 + r) * 64 + lane] = to_float(from_float<T>(acc[mt][r]));
    }
    __syncthreads();
    const int32_t col = n0 + 16 * wave + l16;
    if (wave >= 2 || col >= n) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t row = 16 * mt + 4 * q4 + r;
        if (row >= m) continue;
        const float g = to_float(from_float<T>(acc[mt][r]));
        const float u = up[(wave * MT * 4 + mt * 4 + r) * 64 + lane];
        y[static_cast<int64_t>(row) * y_stride + col] = from_float<T>(swiglu_act(g, u));
      }
    return;
  }
  const int32_t col = n0 + 16 * wave + l16;
  if (col >= n) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int32_t row = 16 * mt + 4 * q4 + r;
      if (row >= m) continue;
      if (partials)
        partials[(static_cast<int64_t>(split) * m + row) * n + col] = acc[mt][r];
      else
        y[static_cast<int64_t>(row) * y_stride + col] = from_float<T>(acc[mt][r]);
    }
}

// ---------------------------------------------------------------------------
// K-split form of the weight stream for narrow weights (few 64-column tiles,
// e.g. a 2560-row qkv projection) and for the gate|up + SwiGLU launch: a
// workgroup owns NT 16-column tiles over all of K and its four wavefronts
// take a quarter of K each.  Every wavefront stages its own KC-wide k
// chunks of x (16 MT rows) and of its weight rows in a private LDS region
// with whole-row loads (KC / 8 lanes per row piece), so the x re-reads (once
// per workgroup) run at the L2 rate of whole-line loads, and the four
// tiles meet once in LDS.  Each x operand read from LDS feeds NT (twice NT
// for SwiGLU) products: two tiles halve the workgroups that re-read x, which
// is what a 64-row call of a wide weight spends most on (TinyLlama's gate|up
// at 64 rows: 18.4 -> 16.2 us on MI355X; with 2048-2560 columns one tile
// keeps more workgroups streaming and stays faster).
// ---------------------------------------------------------------------------
// Chunk rows are KC * 2 bytes; pieces are permuted by (piece ^ (row & mask))
// with mask = min(KC / 8, 16) - 1.
template <int KC>
__device__ __forceinline__ int kstream_lds_offset(int row, int piece) {
  constexpr int kMask = (KC / 8 < 16 ? KC / 8 : 16) - 1;
  return row * KC + ((piece ^ (row & kMask)) << 3);
}

// Epilogues of the K-split kernel.
//   kEpiPlain     y = round(sum)
//   kEpiNorm      y = round(rsqrt(mean_k(x[r][k]^2) + eps) * sum): the
//                 RMSNorm of x's rows applied to the product, for a weight
//                 whose columns carry the norm's gain (w'[n][k] = w[n][k] g[k]);
//                 each workgroup sees all of K, so the row sums of squares
//                 come from the x operands it feeds the MFMAs anyway
//   kEpiResidual  y = round(round(sum) + residual[r][n]): the projection
//                 added to the residual stream, rounded as a separate add is
enum KstreamEpi : int { kEpiPlain = 0, kEpiNorm = 1, kEpiResidual = 2 };
template <typename T>
struct KstreamExtra {
  float eps = 0.f;
  const T *residual = nullptr;
  int64_t residual_stride = 0;
};

// SWIGLU: the workgroup's 16 NT columns j are activation columns; the
// weight stacks gate rows [0, n) over up rows [n, 2n), each wavefront
// accumulates both tiles of every column tile over its quarter of K, and
// the output is round(swiglu_act(round(g), round(u))) (g and u scaled by
// the row's norm first under kEpiNorm).
template <typename T, int MT, int KC, bool SWIGLU, int NT, int EPI>
__global__ void __launch_bounds__(256)
linear_kstream_kernel(const T *__restrict__ x, int64_t x_stride, const T *__restrict__ w,
                      int64_t w_stride, T *__restrict__ y, int64_t y_stride, int32_t m,
                      int32_t n, int32_t k, int32_t k_per_wave, KstreamExtra<T> extra) {
  using M = SplitMma<T>;
  using vec8 = typename M::vec8;
  static_assert(!(SWIGLU && EPI == kEpiResidual), "the residual epilogue has no SwiGLU form");
  // blockIdx.y: a block of 16 MT rows of x and y.
  const int32_t r0 = static_cast<int32_t>(blockIdx.y) * 16 * MT;
  x += static_cast<int64_t>(r0) * x_stride;
  y += static_cast<int64_t>(r0) * y_stride;
  if constexpr (EPI == kEpiResidual) extra.residual += static_cast<int64_t>(r0) * extra.residual_stride;
  m = min(m - r0, 16 * MT);
  constexpr int XR = 16 * MT;
  constexpr int CW = 16 * NT;                  // output columns per workgroup
  constexpr int WR = SWIGLU ? 2 * CW : CW;     // weight rows per workgroup
  constexpr int kLanesPerRow = KC / 8;
  constexpr int kRowsPerLoad = 64 / kLanesPerRow;
  constexpr int kLoadsX = XR / kRowsPerLoad;
  constexpr int kLoadsW = WR / kRowsPerLoad;
  constexpr int kWaveElems = (XR + WR) * KC;
  constexpr int kItems = MT * 4 * 64;          // floats of one 16-column tile
  constexpr int kTiles = SWIGLU ? 2 : 1;
  // The tile sums reuse the staging regions.
  static_assert(4 * kTiles * NT * kItems * 4 <= 4 * kWaveElems * static_cast<int>(sizeof(T)),
                "tile sums exceed the staging LDS");
  extern __shared__ __attribute__((aligned(16))) unsigned char kstream_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  T *xl = reinterpret_cast<T *>(kstream_smem) + wave * kWaveElems;  // [XR][KC]
  T *wl = xl + XR * KC;                                             // [WR][KC]
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  const int32_t n0 = blockIdx.x * CW;
  const int32_t k0 = min(wave * k_per_wave, k);
  const int32_t k1 = min(k0 + k_per_wave, k);
  const int lrow = lane / kLanesPerRow;  // staging: piece lane % (KC/8) of row R i + lane / (KC/8)
  const int lpiece = lane % kLanesPerRow;

  const T *xsrc[kLoadsX];
#pragma unroll
  for (int i = 0; i < kLoadsX; ++i)
    xsrc[i] = x + static_cast<int64_t>(min(kRowsPerLoad * i + lrow, m - 1)) * x_stride + 8 * lpiece;
  const T *wsrc[kLoadsW];
#pragma unroll
  for (int i = 0; i < kLoadsW; ++i) {
    const int tr = kRowsPerLoad * i + lrow;  // tile row: gate rows [0, CW), then up rows
    const int64_t row = SWIGLU ? (tr < CW ? 0 : n) + min(n0 + (tr % CW), n - 1)
                               : min(n0 + tr, n - 1);
    wsrc[i] = w + row * w_stride + 8 * lpiece;
  }

  vec8 xa[kLoadsX], wa[kLoadsW], xb[kLoadsX], wb[kLoadsW];
  // Pieces past K read the row's first piece; those past the wavefront's
  // range but inside K are read and unused.
  auto load_chunk = [&](int32_t kk, vec8(&xr)[kLoadsX], vec8(&wr)[kLoadsW]) {
    const int32_t c = kk + 8 * lpiece < k ? kk : -8 * lpiece;
#pragma unroll
    for (int i = 0; i < kLoadsX; ++i) xr[i] = *reinterpret_cast<const vec8 *>(xsrc[i] + c);
#pragma unroll
    for (int i = 0; i < kLoadsW; ++i) wr[i] = *reinterpret_cast<const vec8 *>(wsrc[i] + c);
  };
  f32x4 acc[MT][NT], accu[SWIGLU ? MT : 1][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) acc[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mt = 0; mt < (SWIGLU ? MT : 1); ++mt)
#pragma unroll
    for (int ct = 0; ct < NT; ++ct) accu[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The region is private to the wavefront, whose LDS requests are served in
  // order: compiler barriers order the stores, the operand reads and the
  // next chunk's stores.
  // kEpiNorm: this lane's sums of squares of the x operands it feeds the
  // MFMAs (row 16 mt + l16, eight elements of every k-step in range), taken
  // from the operand registers so they cost no load and overlap the MFMAs.
  float ssq[EPI == kEpiNorm ? MT : 1];
#pragma unroll
  for (int i = 0; i < (EPI == kEpiNorm ? MT : 1); ++i) ssq[i] = 0.f;
  auto stage_compute = [&](int32_t kk, const vec8(&xr)[kLoadsX], const vec8(&wr)[kLoadsW]) {
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < kLoadsX; ++i)
      *reinterpret_cast<vec8 *>(xl + kstream_lds_offset<KC>(kRowsPerLoad * i + lrow, lpiece)) = xr[i];
#pragma unroll
    for (int i = 0; i < kLoadsW; ++i)
      *reinterpret_cast<vec8 *>(wl + kstream_lds_offset<KC>(kRowsPerLoad * i + lrow, lpiece)) = wr[i];
    __asm__ volatile("" ::: "memory");
    const int32_t steps = min(KC, k1 - kk) >> 5;
#pragma unroll
    for (int st = 0; st < KC / 32; ++st) {
      if (st >= steps) break;  // uniform
      const int piece = 4 * st + q4;
      vec8 b[NT], bu[NT];
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) {
        b[ct] = *reinterpret_cast<const vec8 *>(wl + kstream_lds_offset<KC>(16 * ct + l16, piece));
        if constexpr (SWIGLU)
          bu[ct] = *reinterpret_cast<const vec8 *>(wl + kstream_lds_offset<KC>(CW + 16 * ct + l16, piece));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const vec8 a = *reinterpret_cast<const vec8 *>(xl + kstream_lds_offset<KC>(16 * mt + l16, piece));
#pragma unroll
        for (int ct = 0; ct < NT; ++ct) {
          acc[mt][ct] = M::mma(a, b[ct], acc[mt][ct]);
          if constexpr (SWIGLU) accu[mt][ct] = M::mma(a, bu[ct], accu[mt][ct]);
        }
        if constexpr (EPI == kEpiNorm) ssq[mt] = dot8<T>(a, a, ssq[mt]);
      }
    }
    __asm__ volatile("" ::: "memory");
  };

  // Two chunks in flight.  Every iteration issues both register sets'
  // loads, past the wavefront's last chunk re-reading that chunk (unused),
  // so the loop head holds the same loads outstanding from the entry and
  // from the back edge and each set is waited for alone; a load issued on
  // only some paths would make the wait at the head drain both sets.
  if (k0 < k1) {
    const int32_t last = k0 + ((k1 - k0 - 1) / KC) * KC;
    load_chunk(k0, xa, wa);
    load_chunk(min(k0 + KC, last), xb, wb);
    for (int32_t kk = k0; kk < k1; kk += 2 * KC) {
      stage_compute(kk, xa, wa);
      load_chunk(min(kk + 2 * KC, last), xa, wa);
      stage_compute(kk + KC, xb, wb);  // no products past the range
      load_chunk(min(kk + 3 * KC, last), xb, wb);
    }
  }

  // kEpiNorm: a row's sum of squares over its four lanes, then over the
  // four wavefronts' quarters of K.
  // Rows of sums [4 waves][XR] past the staging regions.
  float *ssq_rows = reinterpret_cast<float *>(kstream_smem + 4 * kWaveElems * sizeof(T));
  if constexpr (EPI == kEpiNorm) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float v = ssq[mt];
      v += __shfl_xor(v, 16, 64);  // the four lanes (l16, q4) of row 16 mt + l16
      v += __shfl_xor(v, 32, 64);
      if (q4 == 0) ssq_rows[wave * XR + 16 * mt + l16] = v;
    }
  }
  // Sum the four wavefront tiles: item (mt, r, lane) of column tile ct is
  // y[16 mt + 4 q4 + r][n0 + 16 ct + l16].
  __syncthreads();  // every wavefront's operand reads are done
  float *tiles = reinterpret_cast<float *>(kstream_smem);  // [4 waves][kTiles][NT][kItems]
#pragma unroll
  for (int ct = 0; ct < NT; ++ct)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        tiles[((wave * kTiles) * NT + ct) * kItems + (mt * 4 + r) * 64 + lane] = acc[mt][ct][r];
        if constexpr (SWIGLU)
          tiles[((wave * kTiles + 1) * NT + ct) * kItems + (mt * 4 + r) * 64 + lane] = accu[mt][ct][r];
      }
  __syncthreads();
  for (int it = threadIdx.x; it < NT * kItems; it += 256) {
    const int ct = it / kItems;
    const int item = it - ct * kItems;
    float sum = 0.f, sumu = 0.f;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv) {
      sum += tiles[((wv * kTiles) * NT + ct) * kItems + item];
      if constexpr (SWIGLU) sumu += tiles[((wv * kTiles + 1) * NT + ct) * kItems + item];
    }
    const int mt = item >> 8;
    const int r = (item >> 6) & 3;
    const int il = item & 63;
    const int32_t row = 16 * mt + 4 * (il >> 4) + r;
    const int32_t col = n0 + 16 * ct + (il & 15);
    if (row >= m || col >= n) continue;
    if constexpr (EPI == kEpiNorm) {
      const float sq = ((ssq_rows[row] + ssq_rows[XR + row]) + ssq_rows[2 * XR + row]) +
                       ssq_rows[3 * XR + row];
      const float scale = rsqrtf(sq / static_cast<float>(k) + extra.eps);
      sum *= scale;
      sumu *= scale;
    }
    T out;
    if constexpr (SWIGLU)
      out = from_float<T>(swiglu_act(to_float(from_float<T>(sum)), to_float(from_float<T>(sumu))));
    else if constexpr (EPI == kEpiResidual)
      out = from_float<T>(to_float(from_float<T>(sum)) +
                          to_float(extra.residual[static_cast<int64_t>(row) * extra.residual_stride + col]));
    else
      out = from_float<T>(sum);
    y[static_cast<int64_t>(row) * y_stride + col] = out;
  }
}

// Activation-resident form of the K-split kernel (the SwiGLU + RMSNorm
// launch at 49-64 rows with K = 2048; launch_kstream_mt picks it): each
// wavefront copies its K quarter of the workgroup's 16 MT rows of x into
// LDS once, then streams only weights over the column tiles blockIdx.x,
// blockIdx.x + groups, ... (INFL chunks of 64 k in flight), so a workgroup
// reads x once instead of once per 64-k chunk of every tile.  Per lane and
// k-step the MFMA operands, the order of the k-steps, the sums of squares
// and the epilogue are those of linear_kstream_kernel, so both forms give
// the same bits.  The outputs of a workgroup's tiles wait in LDS and are
// stored after the stream (a store inside it would leave the loads' wait
// counts unknown at the loop head).
template <typename T, int MT, int NT, bool SWIGLU, int EPI, int INFL, int KQ, int MAXT>
__global__ void __launch_bounds__(256)
linear_xres_kernel(const T *__restrict__ x, int64_t x_stride, const T *__restrict__ w,
                   int64_t w_stride, T *__restrict__ y, int64_t y_stride, int32_t m, int32_t n,
                   int32_t k, int32_t groups, KstreamExtra<T> extra) {
  using M = SplitMma<T>;
  using vec8 = typename M::vec8;
  constexpr int KC = 64;
  constexpr int XR = 16 * MT;
  constexpr int CW = 16 * NT;
  constexpr int kSteps = KC / 32;
  constexpr int kItems = MT * 4 * 64;
  constexpr int kTiles = SWIGLU ? 2 : 1;
  const int32_t r0 = static_cast<int32_t>(blockIdx.y) * XR;
  x += static_cast<int64_t>(r0) * x_stride;
  y += static_cast<int64_t>(r0) * y_stride;
  if constexpr (EPI == kEpiResidual) extra.residual += static_cast<int64_t>(r0) * extra.residual_stride;
  m = min(m - r0, XR);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15;
  const int q4 = lane >> 4;
  constexpr int32_t kq = KQ;          // K quarter (the host checks k == 4 KQ)
  constexpr int32_t xs = kq + 8;      // padded LDS row: rows 16 B apart in the banks
  constexpr int32_t nch = kq / KC;    // chunks per tile per wavefront
  static_assert(nch % INFL == 0, "a group of INFL chunks lies in one tile");
  constexpr int XL = XR * kq / 512;   // x loads per lane
  const int32_t k0 = wave * kq;
  const int32_t ntiles = (n + CW - 1) / CW;

  extern __shared__ __attribute__((aligned(16))) unsigned char xres_smem[];
  // LDS: x quarters [4][XR][xs] | weight staging [4][WR][KC] (its space
  // holds the tile sums [4][kTiles][NT][kItems] in the epilogue) | row sums
  // of squares [4][XR] | rounded outputs [MAXT][XR][CW].
  constexpr int kStageBytes = 4 * (SWIGLU ? 2 * CW : CW) * KC * static_cast<int>(sizeof(T));
  constexpr int kTileBytes = 4 * kTiles * NT * kItems * 4;
  constexpr int kRegion = kStageBytes > kTileBytes ? kStageBytes : kTileBytes;
  T *xq = reinterpret_cast<T *>(xres_smem) + wave * XR * xs;
  unsigned char *region = xres_smem + 4 * XR * xs * sizeof(T);
  T *wl = reinterpret_cast<T *>(region) + wave * (SWIGLU ? 2 * CW : CW) * KC;
  float *tiles = reinterpret_cast<float *>(region);
  float *ssq_rows = reinterpret_cast<float *>(region + kRegion);
  T *outs = reinterpret_cast<T *>(ssq_rows + 4 * XR);

  // Weight loads of stream position i (clamped to the last): tile
  // blockIdx.x + (i / nch) groups, chunk i % nch; lane (l16, q4) of group g,
  // k-step s holds w[row][kk + 32 s + 8 q4 .. +8].
  // Weight chunks are loaded as whole 128-byte row pieces (8 lanes per row,
  // 8 rows per load) and staged in a per-wavefront LDS region before the
  // MFMA operand reads, as linear_kstream_kernel stages them.  The host
  // checks nch % INFL == 0, so a group of INFL positions lies in one tile:
  // load_w(p, s) loads position p + s of such a group (p past the stream
  // reloads its last group).
  constexpr int WR = SWIGLU ? 2 * CW : CW;
  constexpr int kLanesPerRow = KC / 8;
  constexpr int kRowsPerLoad = 64 / kLanesPerRow;
  constexpr int kLoadsW = WR / kRowsPerLoad;
  const int lrow = lane / kLanesPerRow;
  const int lpiece = lane % kLanesPerRow;
  // Row pointers of the tile being loaded: tile index lt (clamped to the
  // last one, whose chunks are reloaded past the stream), chunk lc.
  const int32_t my_tiles = (ntiles - static_cast<int32_t>(blockIdx.x) + groups - 1) / groups;
  const T *wsrc[kLoadsW];
  auto point_w = [&](int32_t lt) {
    const int32_t n0 = (static_cast<int32_t>(blockIdx.x) + min(lt, my_tiles - 1) * groups) * CW;
#pragma unroll
    for (int i = 0; i < kLoadsW; ++i) {
      const int tr = kRowsPerLoad * i + lrow;  // tile row: gate rows [0, CW), then up rows
      const int64_t row = SWIGLU ? (tr < CW ? 0 : n) + min(n0 + (tr % CW), n - 1) : min(n0 + tr, n - 1);
      wsrc[i] = w + row * w_stride + k0 + 8 * lpiece;
    }
  };
  int32_t lt = 0, lc = 0;
  point_w(0);
  // Chunk lc + s of the tile being loaded; past the stream the last tile's
  // last group again.
  auto load_w = [&](int s, vec8(&r)[kLoadsW]) {
    const int32_t c = (lt < my_tiles ? lc : nch - INFL) + s;
#pragma unroll
    for (int i = 0; i < kLoadsW; ++i) r[i] = *reinterpret_cast<const vec8 *>(wsrc[i] + c * KC);
  };
  auto next_group = [&]() {
    lc += INFL;
    if (lc == nch) {
      lc = 0;
      ++lt;
      point_w(lt);
    }
  };

  // x quarter: XR rows x kq (XL loads per lane, lane: 8 consecutive
  // elements); rows past m read row m - 1.  All of them go out before the
  // weight prefetch and are written while it is in flight.
  vec8 wr[INFL][kLoadsW];
  {
    vec8 xb[XL];
#pragma unroll
    for (int j = 0; j < XL; ++j) {
      constexpr int kPerRow = kq / 8;  // lanes' pieces per row
      const int row = (64 * j + lane) / kPerRow;
      const int col = 8 * ((64 * j + lane) % kPerRow);
      xb[j] = *reinterpret_cast<const vec8 *>(x + static_cast<int64_t>(min(row, m - 1)) * x_stride + k0 + col);
    }
#pragma unroll
    for (int s = 0; s < INFL; ++s) load_w(s, wr[s]);
    next_group();
    __asm__ volatile("" ::: "memory");  // every load above is issued before the first store
#pragma unroll
    for (int j = 0; j < XL; ++j) {
      constexpr int kPerRow = kq / 8;
      const int row = (64 * j + lane) / kPerRow;
      const int col = 8 * ((64 * j + lane) % kPerRow);
      *reinterpret_cast<vec8 *>(xq + row * xs + col) = xb[j];
    }
  }
  __asm__ volatile("" ::: "memory");  // this wavefront's x stores precede its operand reads

  f32x4 acc[MT][NT], accu[SWIGLU ? MT : 1][NT];
  float ssq[EPI == kEpiNorm ? MT : 1];
#pragma unroll
  for (int i = 0; i < (EPI == kEpiNorm ? MT : 1); ++i) ssq[i] = 0.f;
  auto zero_acc = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) {
        acc[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (SWIGLU) accu[mt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
  };
  zero_acc();
  auto compute = [&](int32_t c, const vec8(&r)[kLoadsW], bool first) {
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < kLoadsW; ++i)
      *reinterpret_cast<vec8 *>(wl + kstream_lds_offset<KC>(kRowsPerLoad * i + lrow, lpiece)) = r[i];
    __asm__ volatile("" ::: "memory");
    const T *xa = xq + l16 * xs + c * KC + 8 * q4;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const int piece = 4 * s + q4;
      vec8 b[NT], bu[NT];
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) {
        b[ct] = *reinterpret_cast<const vec8 *>(wl + kstream_lds_offset<KC>(16 * ct + l16, piece));
        if constexpr (SWIGLU)
          bu[ct] = *reinterpret_cast<const vec8 *>(wl + kstream_lds_offset<KC>(CW + 16 * ct + l16, piece));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const vec8 a = *reinterpret_cast<const vec8 *>(xa + 16 * mt * xs + 32 * s);
#pragma unroll
        for (int ct = 0; ct < NT; ++ct) {
          acc[mt][ct] = M::mma(a, b[ct], acc[mt][ct]);
          if constexpr (SWIGLU) accu[mt][ct] = M::mma(a, bu[ct], accu[mt][ct]);
        }
        if constexpr (EPI == kEpiNorm)
          if (first) ssq[mt] = dot8<T>(a, a, ssq[mt]);
      }
    }
    __asm__ volatile("" ::: "memory");
  };

  // Every workgroup has a tile (the host keeps groups <= ntiles): no path
  // skips the stream, so the prefetch above stays ahead of the x stores.
  int32_t tile = 0, c0 = 0;
  for (;;) {
    const bool first = tile == 0;
#pragma unroll
    for (int s = 0; s < INFL; ++s) {
      compute(c0 + s, wr[s], first);
      load_w(s, wr[s]);
    }
    next_group();
    c0 += INFL;
    if (c0 < nch) continue;
    // Tile done: the four wavefront tiles meet in LDS (as linear_kstream_kernel's epilogue).
    __syncthreads();  // every wavefront's operand reads are done (the sums reuse the staging)
    if constexpr (EPI == kEpiNorm) {
      if (first) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          float v = ssq[mt];
          v += __shfl_xor(v, 16, 64);
          v += __shfl_xor(v, 32, 64);
          if (q4 == 0) ssq_rows[wave * XR + 16 * mt + l16] = v;
        }
      }
    }
#pragma unroll
    for (int ct = 0; ct < NT; ++ct)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          tiles[((wave * kTiles) * NT + ct) * kItems + (mt * 4 + r) * 64 + lane] = acc[mt][ct][r];
          if constexpr (SWIGLU)
            tiles[((wave * kTiles + 1) * NT + ct) * kItems + (mt * 4 + r) * 64 + lane] = accu[mt][ct][r];
        }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NT * kItems / 256; ++j) {
      const int it = threadIdx.x + 256 * j;
      const int ct = it / kItems;
      const int item = it - ct * kItems;
      float sum = 0.f, sumu = 0.f;
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) {
        sum += tiles[((wv * kTiles) * NT + ct) * kItems + item];
        if constexpr (SWIGLU) sumu += tiles[((wv * kTiles + 1) * NT + ct) * kItems + item];
      }
      const int mt = item >> 8;
      const int r = (item >> 6) & 3;
      const int il = item & 63;
      const int32_t row = 16 * mt + 4 * (il >> 4) + r;
      if constexpr (EPI == kEpiNorm) {
        const float sq = ((ssq_rows[row] + ssq_rows[XR + row]) + ssq_rows[2 * XR + row]) +
                         ssq_rows[3 * XR + row];
        const float scale = rsqrtf(sq / static_cast<float>(k) + extra.eps);
        sum *= scale;
        sumu *= scale;
      }
      // Rounded outputs (before the residual add) wait in LDS for the stores
      // after the stream: [tile][XR][CW].
      T out;
      if constexpr (SWIGLU)
        out = from_float<T>(swiglu_act(to_float(from_float<T>(sum)), to_float(from_float<T>(sumu))));
      else
        out = from_float<T>(sum);
      outs[tile * XR * CW + row * CW + 16 * ct + (il & 15)] = out;
    }
    __syncthreads();  // the sums are read before the next tile writes them
    zero_acc();
    c0 = 0;
    if (++tile == my_tiles) break;
  }
  // Stores after the stream (a store inside it would leave the loads'
  // wait counts unknown at the loop head).
  for (int32_t e = threadIdx.x; e < my_tiles * XR * CW; e += 256) {
    const int32_t tile = e / (XR * CW);
    const int32_t rc = e - tile * XR * CW;
    const int32_t row = rc / CW;
    const int32_t col = (static_cast<int32_t>(blockIdx.x) + tile * groups) * CW + (rc - row * CW);
    if (row >= m || col >= n) continue;
    T out = outs[e];
    if constexpr (EPI == kEpiResidual)
      out = from_float<T>(to_float(out) +
                          to_float(extra.residual[static_cast<int64_t>(row) * extra.residual_stride + col]));
    y[static_cast<int64_t>(row) * y_stride + col] = out;
  }
}

template <typename T, int MT, int KC, bool SWIGLU, int NT, int EPI>
void launch_kstream(const void *x, int64_t x_stride, const void *w, int64_t w_stride, void *y,
                    int64_t y_stride, int32_t m, int32_t n, int32_t k, const KstreamExtra<T> &extra,
                    hipStream_t stream) {
  const unsigned row_blocks = static_cast<unsigned>((m + 16 * MT - 1) / (16 * MT));
  const int32_t steps = k / 32;
  const int32_t k_per_wave = ((steps + 3) / 4) * 32;
  const size_t lds =
      static_cast<size_t>(4) * (16 * MT + (SWIGLU ? 32 : 16) * NT) * KC * sizeof(T) +
      (EPI == kEpiNorm ? static_cast<size_t>(4) * 16 * MT * sizeof(float) : 0);
  if (lds > 64 * 1024) {
    // Raise the kernel's dynamic LDS limit once per device (a failure shows
    // up as a launch error).
    constexpr int kMaxDevices = 64;
    static std::atomic<bool> raised[kMaxDevices];
    int device = 0;
    if (hipGetDevice(&device) == hipSuccess && device >= 0 && device < kMaxDevices &&
        !raised[device].load(std::memory_order_acquire)) {
      if (hipFuncSetAttribute(
              reinterpret_cast<const void *>(&linear_kstream_kernel<T, MT, KC, SWIGLU, NT, EPI>),
              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) == hipSuccess)
        raised[device].store(true, std::memory_order_release);
    }
  }
  hipLaunchKernelGGL((linear_kstream_kernel<T, MT, KC, SWIGLU, NT, EPI>),
                     dim3((n + 16 * NT - 1) / (16 * NT), row_blocks), dim3(256), lds, stream,
                     static_cast<const T *>(x), x_stride, static_cast<const T *>(w), w_stride,
                     static_cast<T *>(y), y_stride, m, n, k, k_per_wave, extra);
}

// The activation-resident SwiGLU + RMSNorm launch (linear_xres_kernel):
// 32-row blocks (MT 2), one 16-column tile per step (NT 1), eight 64-k
// chunks in flight, 128 column groups per row block (one workgroup per
// compute unit at 64 rows, each holding at most kXresMaxTiles tiles' outputs
// in LDS).  Taken for 49-64 rows at K = 2048 (K quarters of 512) when the
// tiles fit: gate|up + SwiGLU of TinyLlama at 64 rows, 17.3 -> 15.9 us
// (MI355X, graph-timed, bit-identical); at 17-48 rows it is slower than
// the K-split form (32 rows 13.5 against 15.7).
constexpr int kXresMt = 2;
constexpr int kXresNt = 1;
constexpr int kXresInflight = 8;
constexpr int kXresKq = 512;
constexpr int kXresMaxTiles = 4;
constexpr int kXresGroups = 128;

size_t xres_lds_bytes(size_t elem) {
  constexpr int XR = 16 * kXresMt, CW = 16 * kXresNt;
  const size_t stage = static_cast<size_t>(4) * 2 * CW * 64 * elem;
  const size_t sums = static_cast<size_t>(4) * 2 * kXresNt * kXresMt * 256 * 4;
  return static_cast<size_t>(4) * XR * (kXresKq + 8) * elem + (stage > sums ? stage : sums) +
         static_cast<size_t>(4) * XR * 4 + static_cast<size_t>(kXresMaxTiles) * XR * CW * elem;
}

bool xres_fits(int32_t m, int32_t n, int32_t k) {
  const int32_t ntiles = (n + 16 * kXresNt - 1) / (16 * kXresNt);
  return m > 48 && m <= 64 && k == 4 * kXresKq && ntiles >= kXresGroups &&
         (ntiles + kXresGroups - 1) / kXresGroups <= kXresMaxTiles;
}

template <typename T>
void launch_xres_swiglu_norm(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                             void *y, int64_t y_stride, int32_t m, int32_t n, int32_t k,
                             const KstreamExtra<T> &extra, hipStream_t stream) {
  auto kernel = &linear_xres_kernel<T, kXresMt, kXresNt, true, kEpiNorm, kXresInflight, kXresKq,
                                    kXresMaxTiles>;
  const size_t lds = xres_lds_bytes(sizeof(T));
  // Raise the kernel's dynamic LDS limit once per device (a failure shows up
  // as a launch error).
  constexpr int kMaxDevices = 64;
  static std::atomic<bool> raised[kMaxDevices];
  int device = 0;
  if (hipGetDevice(&device) == hipSuccess && device >= 0 && device < kMaxDevices &&
      !raised[device].load(std::memory_order_acquire)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) == hipSuccess)
      raised[device].store(true, std::memory_order_release);
  }
  const unsigned row_blocks = static_cast<unsigned>((m + 16 * kXresMt - 1) / (16 * kXresMt));
  hipLaunchKernelGGL(kernel, dim3(kXresGroups, row_blocks), dim3(256), lds, stream,
                     static_cast<const T *>(x), x_stride, static_cast<const T *>(w), w_stride,
                     static_cast<T *>(y), y_stride, m, n, k, kXresGroups, extra);
}

// Chunk 64 for the SwiGLU form and above 32 rows, else 128.  A workgroup
// reads 16 (MT + NT) rows of K (x rows and weight rows; twice NT weight
// rows for SwiGLU), so fewer rows per workgroup means fewer re-reads of x;
// one workgroup per compute unit is what keeps the split even.  The plain
// form therefore takes, among workgroups of 1-4 row tiles (MT) and 1-2
// column tiles (NT) whose grid fits the 256 compute units, the one with the
// fewest rows (then the larger grid, then one column tile); a grid that
// fits with none keeps MT = ceil(m / 16), NT = 1.  On MI355X at 64 rows:
// qkv (2560 columns) MT 2, NT 2 (160 workgroups) 9.2 -> 7.9 us; 2048
// columns MT 2, NT 1 (256) 8.8 -> 6.5 us; at 33-48 rows qkv MT 1, NT 2
// (240) 7.5-7.8 -> 6.5-6.6 us.  The SwiGLU form takes MT = ceil(m / 16)
// and two column tiles from 4096 activation columns.
template <typename T, bool SWIGLU, int EPI>
void launch_kstream_mt(const void *x, int64_t x_stride, const void *w, int64_t w_stride, void *y,
                       int64_t y_stride, int32_t m, int32_t n, int32_t k,
                       const KstreamExtra<T> &extra, hipStream_t stream) {
  if constexpr (SWIGLU && EPI == kEpiNorm) {
    if (xres_fits(m, n, k)) {
      launch_xres_swiglu_norm<T>(x, x_stride, w, w_stride, y, y_stride, m, n, k, extra, stream);
      return;
    }
  }
  const int32_t row_tiles = (m + 15) / 16;
  // 64-wide chunks above 32 rows (twice the chunks per wavefront, half the
  // staging per chunk), 128 up to 32 rows; bit-identical either way (the
  // k-steps run in the same order).  On MI355X: qkv at 64 rows 9.0 -> 8.2 us,
  // o 6.7 -> 6.5, down unchanged; at 1..32 rows 64 is 0.5-1.6 us slower.
  const int kc = SWIGLU || row_tiles > 2 ? 64 : 128;
  int mt = row_tiles > 4 ? 4 : row_tiles;
  int nt = 1;
  if constexpr (SWIGLU) {
    if (n >= 4096) nt = 2;
  } else {
    int best_rows = 1 << 30;
    int64_t best_grid = 0;
    for (int cm = 1; cm <= 4 && cm <= row_tiles; ++cm) {
      for (int cn = 1; cn <= 2; ++cn) {
        const int64_t grid = static_cast<int64_t>((row_tiles + cm - 1) / cm) *
                             ((n + 16 * cn - 1) / (16 * cn));
        if (grid > 256) continue;
        if (cm + cn < best_rows || (cm + cn == best_rows && grid > best_grid) ||
            (cm + cn == best_rows && grid == best_grid && cn < nt)) {
          best_rows = cm + cn;
          best_grid = grid;
          mt = cm;
          nt = cn;
        }
      }
    }
  }
#define TF_KSTREAM_CASE(MT, NT)                                                                \
  if (mt == MT && nt == NT) {                                                                  \
    if (kc == 64)                                                                              \
      launch_kstream<T, MT, 64, SWIGLU, NT, EPI>(x, x_stride, w, w_stride, y, y_stride, m, n, k, \
                                                 extra, stream);                                  \
    else if constexpr (!SWIGLU)                                                                \
      launch_kstream<T, MT, 128, SWIGLU, NT, EPI>(x, x_stride, w, w_stride, y, y_stride, m, n, \
                                                  k, extra, stream);                              \
    return;                                                                                    \
  }
  TF_KSTREAM_CASE(1, 1)
  TF_KSTREAM_CASE(2, 1)
  TF_KSTREAM_CASE(3, 1)
  TF_KSTREAM_CASE(4, 1)
  TF_KSTREAM_CASE(1, 2)
  TF_KSTREAM_CASE(2, 2)
  TF_KSTREAM_CASE(3, 2)
  TF_KSTREAM_CASE(4, 2)
#undef TF_KSTREAM_CASE
}

template <typename T, int MT, bool SWIGLU>
void launch_stream(const void *x, int64_t x_stride, const void *w, int64_t w_stride, void *y,
                   int64_t y_stride, float *partials, int32_t m, int32_t n, int32_t k,
                   int32_t splits, int32_t k_per_split, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(16 * MT + kStreamCols) * kStreamChunk * sizeof(T);
  const int32_t cols = SWIGLU ? kStreamCols / 2 : kStreamCols;
  hipLaunchKernelGGL((linear_stream_kernel<T, MT, SWIGLU>),
                     dim3((n + cols - 1) / cols, splits), dim3(256), lds, stream,
                     static_cast<const T *>(x), x_stride, static_cast<const T *>(w), w_stride,
                     static_cast<T *>(y), y_stride, partials, m, n, k, k_per_split);
}

template <typename T, bool SWIGLU>
void launch_stream_mt(const void *x, int64_t x_stride, const void *w, int64_t w_stride, void *y,
                      int64_t y_stride, float *partials, int32_t m, int32_t n, int32_t k,
                      int32_t splits, int32_t k_per_split, hipStream_t stream) {
#define TF_STREAM_CASE(MT)                                                                   \
  launch_stream<T, MT, SWIGLU>(x, x_stride, w, w_stride, y, y_stride, partials, m, n, k,    \
                               splits, k_per_split, stream)
  switch ((m + 15) / 16) {
    case 1: TF_STREAM_CASE(1); break;
    case 2: TF_STREAM_CASE(2); break;
    case 3: TF_STREAM_CASE(3); break;
    default: TF_STREAM_CASE(4); break;
  }
#undef TF_STREAM_CASE
}

// y[m][n] = round(sum_s partials[s][m][n]), four columns per thread.
template <typename T>
__global__ void __launch_bounds__(256)
partials_sum_kernel(const float *__restrict__ partials, int32_t splits, int32_t m, int32_t n,
                    T *__restrict__ y, int64_t y_stride) {
  const int64_t quads = static_cast<int64_t>(m) * (n / 4);
  const int64_t plane = static_cast<int64_t>(m) * n;
  for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < quads;
       q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int32_t row = static_cast<int32_t>(q / (n / 4));
    const int32_t col = 4 * static_cast<int32_t>(q - static_cast<int64_t>(row) * (n / 4));
    const float *src = partials + static_cast<int64_t>(row) * n + col;
    f32x4 s = *reinterpret_cast<const f32x4 *>(src);
    for (int32_t sp = 1; sp < splits; ++sp) s += *reinterpret_cast<const f32x4 *>(src + sp * plane);
    typedef T t4 __attribute__((ext_vector_type(4)));
    const t4 v = {from_float<T>(s[0]), from_float<T>(s[1]), from_float<T>(s[2]),
                  from_float<T>(s[3])};
    *reinterpret_cast<t4 *>(y + static_cast<int64_t>(row) * y_stride + col) = v;
  }
}

template <typename T, int MT>
void launch_partials(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                     float *partials, int32_t m, int32_t n, int32_t k, int32_t splits,
                     int32_t k_per_split, hipStream_t stream) {
  const size_t lds = static_cast<size_t>(kSplitWaves) * MT * (kSplitCols / 16) * 4 * 64 *
                     sizeof(float);
  hipLaunchKernelGGL((linear_partials_kernel<T, MT>),
                     dim3((n + kSplitCols - 1) / kSplitCols, splits), dim3(kSplitWaves * 64), lds,
                     stream, static_cast<const T *>(x), x_stride, static_cast<const T *>(w),
                     w_stride, partials, m, n, k, k_per_split);
}

template <typename T>
void launch_partials_mt(const void *x, int64_t x_stride, const void *w, int64_t w_stride,
                        float *partials, int32_t m, int32_t n, int32_t k, int32_t splits,
                        int32_t k_per_split, hipStream_t stream) {
  switch ((m + 15) / 16) {
    case 1: launch_partials<T, 1>(x, x_stride, w, w_stride, partials, m, n, k, splits, k_per_split, stream); break;
    case 2: launch_partials<T, 2>(x, x_stride, w, w_stride, partials, m, n, k, splits, k_per_split, stream); break;
    case 3: launch_partials<T, 3>(x, x_stride, w, w_stride, partials, m, n, k, splits, k_per_split, stream); break;
    default: launch_partials<T, 4>(x, x_stride, w, w_stride, partials, m, n, k, splits, k_per_split, stream); break;
  }
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_linear_partials(const void *x, int64_t x_row_stride, const void *weight,
                                      int64_t weight_row_stride, float *partials, int32_t m,
                                      int32_t n, int32_t k, int32_t splits, int32_t dtype,
                                      void *stream) {
  using namespace tf;
  clear_error();
  if (dtype != TF_DTYPE_FLOAT16 && dtype != TF_DTYPE_BFLOAT16)
    return fail(TF_ERROR_UNSUPPORTED, "linear_partials supports fp16 and bf16");
  if (m < 0 || n < 0 || k < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "sizes must be non-negative");
  if (m > 64) return fail(TF_ERROR_UNSUPPORTED, "linear_partials supports at most 64 rows");
  if (k % 32 != 0 || k == 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_partials needs K to be a positive multiple of 32");
  if (splits < 1 || splits > k / 32)
    return fail(TF_ERROR_INVALID_ARGUMENT, "splits must be in [1, K / 32]");
  if (x_row_stride < k || weight_row_stride < k)
    return fail(TF_ERROR_INVALID_ARGUMENT, "row strides are shorter than the rows");
  if (n > 65535 * tf::kSplitCols || splits > 65535)
    return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  if (m == 0 || n == 0) return TF_SUCCESS;
  if (!x || !weight || !partials) return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                          static_cast<uintptr_t>(x_row_stride * 2) |
                          static_cast<uintptr_t>(weight_row_stride * 2);
  if (align % 16 != 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_partials needs 16-byte aligned x and weight rows");
  // Slices of whole k-steps; every slice is non-empty.
  const int32_t steps = k / 32;
  const int32_t k_per_split = ((steps + splits - 1) / splits) * 32;
  const int32_t used = (k + k_per_split - 1) / k_per_split;
  if (used != splits)
    return fail(TF_ERROR_INVALID_ARGUMENT, "splits must divide K / 32 into non-empty slices");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TF_DTYPE_BFLOAT16)
    launch_partials_mt<__bf16>(x, x_row_stride, weight, weight_row_stride, partials, m, n, k,
                               splits, k_per_split, s);
  else
    launch_partials_mt<_Float16>(x, x_row_stride, weight, weight_row_stride, partials, m, n, k,
                                 splits, k_per_split, s);
  return check_launch("linear_partials");
}

extern "C" int32_t tf_linear_partials_sum(const float *partials, int32_t splits, int32_t m,
                                          int32_t n, void *y, int64_t y_row_stride,
                                          int32_t dtype, void *stream) {
  using namespace tf;
  clear_error();
  if (!valid_dtype(dtype)) return fail(TF_ERROR_INVALID_ARGUMENT, "unsupported dtype code");
  if (dtype == TF_DTYPE_FLOAT32)
    return fail(TF_ERROR_UNSUPPORTED, "linear_partials_sum writes fp16 or bf16");
  if (m < 0 || n < 0 || splits < 1) return fail(TF_ERROR_INVALID_ARGUMENT, "invalid sizes");
  if (n % 4 != 0 || y_row_stride % 4 != 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_partials_sum needs N and the row stride to be multiples of 4");
  if (y_row_stride < n) return fail(TF_ERROR_INVALID_ARGUMENT, "row stride is shorter than the rows");
  if (m == 0 || n == 0) return TF_SUCCESS;
  if (!partials || !y) return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  if ((reinterpret_cast<uintptr_t>(partials) | reinterpret_cast<uintptr_t>(y)) % 16 != 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_partials_sum needs 16-byte aligned buffers");
  const int64_t quads = static_cast<int64_t>(m) * (n / 4);
  const int64_t blocks = (quads + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks < 2048 ? blocks : 2048));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TF_DTYPE_BFLOAT16)
    hipLaunchKernelGGL(partials_sum_kernel<__bf16>, grid, dim3(256), 0, s, partials, splits, m, n,
                       static_cast<__bf16 *>(y), y_row_stride);
  else
    hipLaunchKernelGGL(partials_sum_kernel<_Float16>, grid, dim3(256), 0, s, partials, splits, m,
                       n, static_cast<_Float16 *>(y), y_row_stride);
  return check_launch("linear_partials_sum");
}

namespace tf {
namespace {

int32_t linear_stream_entry(const void *x, int64_t x_row_stride, const void *weight,
                            int64_t weight_row_stride, void *y, int64_t y_row_stride,
                            float *partials, int32_t m, int32_t n, int32_t k, int32_t splits,
                            int32_t dtype, void *stream, bool swiglu, const char *name) {
  clear_error();
  if (dtype != TF_DTYPE_FLOAT16 && dtype != TF_DTYPE_BFLOAT16)
    return fail(TF_ERROR_UNSUPPORTED, "linear_stream supports fp16 and bf16");
  if (m < 0 || n < 0 || k < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "sizes must be non-negative");
  if (m > 64) return fail(TF_ERROR_UNSUPPORTED, "linear_stream supports at most 64 rows");
  if (k % 32 != 0 || k == 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_stream needs K to be a positive multiple of 32");
  if (splits < 1 || splits > k / 32)
    return fail(TF_ERROR_INVALID_ARGUMENT, "splits must be in [1, K / 32]");
  if (!partials && splits != 1)
    return fail(TF_ERROR_INVALID_ARGUMENT, "several K slices need a partials buffer");
  if (x_row_stride < k || weight_row_stride < k || (!partials && y_row_stride < n))
    return fail(TF_ERROR_INVALID_ARGUMENT, "row strides are shorter than the rows");
  if (n > 65535 * (kStreamCols / 2) || splits > 65535)
    return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  if (m == 0 || n == 0) return TF_SUCCESS;
  if (!x || !weight || (!partials && !y))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                          static_cast<uintptr_t>(x_row_stride * 2) |
                          static_cast<uintptr_t>(weight_row_stride * 2);
  if (align % 16 != 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_stream needs 16-byte aligned x and weight rows");
  const int32_t steps = k / 32;
  const int32_t k_per_split = ((steps + splits - 1) / splits) * 32;
  if ((k + k_per_split - 1) / k_per_split != splits)
    return fail(TF_ERROR_INVALID_ARGUMENT, "splits must divide K / 32 into non-empty slices");
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TF_STREAM_LAUNCH(T, G)                                                                \
  launch_stream_mt<T, G>(x, x_row_stride, weight, weight_row_stride, y, y_row_stride, partials, \
                         m, n, k, splits, k_per_split, s)
  if (dtype == TF_DTYPE_BFLOAT16) {
    if (swiglu) TF_STREAM_LAUNCH(__bf16, true); else TF_STREAM_LAUNCH(__bf16, false);
  } else {
    if (swiglu) TF_STREAM_LAUNCH(_Float16, true); else TF_STREAM_LAUNCH(_Float16, false);
  }
#undef TF_STREAM_LAUNCH
  return check_launch(name);
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_linear_stream(const void *x, int64_t x_row_stride, const void *weight,
                                    int64_t weight_row_stride, void *y, int64_t y_row_stride,
                                    float *partials, int32_t m, int32_t n, int32_t k,
                                    int32_t splits, int32_t dtype, void *stream) {
  return tf::linear_stream_entry(x, x_row_stride, weight, weight_row_stride, y, y_row_stride,
                                 partials, m, n, k, splits, dtype, stream, false,
                                 "linear_stream");
}

extern "C" int32_t tf_linear_swiglu(const void *x, int64_t x_row_stride, const void *gate_up_weight,
                                    int64_t weight_row_stride, void *y, int64_t y_row_stride,
                                    int32_t m, int32_t intermediate, int32_t k, int32_t dtype,
                                    void *stream) {
  return tf::linear_stream_entry(x, x_row_stride, gate_up_weight, weight_row_stride, y,
                                 y_row_stride, nullptr, m, intermediate, k, 1, dtype, stream,
                                 true, "linear_swiglu");
}

namespace tf {
namespace {

int32_t kstream_entry(const void *x, int64_t x_row_stride, const void *weight,
                      int64_t weight_row_stride, void *y, int64_t y_row_stride, int32_t m,
                      int32_t n, int32_t k, int32_t dtype, void *stream, bool swiglu, int epi,
                      float eps, const void *residual, int64_t residual_row_stride,
                      const char *name) {
  clear_error();
  if (dtype != TF_DTYPE_FLOAT16 && dtype != TF_DTYPE_BFLOAT16)
    return fail(TF_ERROR_UNSUPPORTED, "linear_kstream supports fp16 and bf16");
  if (m < 0 || n < 0 || k < 0) return fail(TF_ERROR_INVALID_ARGUMENT, "sizes must be non-negative");
  if (m > 64) return fail(TF_ERROR_UNSUPPORTED, "linear_kstream supports at most 64 rows");
  if (k % 32 != 0 || k == 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_kstream needs K to be a positive multiple of 32");
  if (x_row_stride < k || weight_row_stride < k || y_row_stride < n)
    return fail(TF_ERROR_INVALID_ARGUMENT, "row strides are shorter than the rows");
  if (epi == kEpiNorm && !(eps > 0.f)) return fail(TF_ERROR_INVALID_ARGUMENT, "eps must be positive");
  if (epi == kEpiResidual && residual_row_stride < n)
    return fail(TF_ERROR_INVALID_ARGUMENT, "residual row stride is shorter than the rows");
  if (n > 65535 * 16) return fail(TF_ERROR_UNSUPPORTED, "grid too large");
  if (m == 0 || n == 0) return TF_SUCCESS;
  if (!x || !weight || !y || (epi == kEpiResidual && !residual))
    return fail(TF_ERROR_INVALID_ARGUMENT, "null tensor pointer");
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                          static_cast<uintptr_t>(x_row_stride * 2) |
                          static_cast<uintptr_t>(weight_row_stride * 2);
  if (align % 16 != 0)
    return fail(TF_ERROR_UNSUPPORTED, "linear_kstream needs 16-byte aligned x and weight rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TF_KSTREAM_LAUNCH(T)                                                                  \
  do {                                                                                        \
    KstreamExtra<T> extra;                                                                    \
    extra.eps = eps;                                                                          \
    extra.residual = static_cast<const T *>(residual);                                       \
    extra.residual_stride = residual_row_stride;                                              \
    if (swiglu && epi == kEpiNorm)                                                            \
      launch_kstream_mt<T, true, kEpiNorm>(x, x_row_stride, weight, weight_row_stride, y,     \
                                           y_row_stride, m, n, k, extra, s);                  \
    else if (swiglu)                                                                          \
      launch_kstream_mt<T, true, kEpiPlain>(x, x_row_stride, weight, weight_row_stride, y,    \
                                            y_row_stride, m, n, k, extra, s);                 \
    else if (epi == kEpiNorm)                                                                 \
      launch_kstream_mt<T, false, kEpiNorm>(x, x_row_stride, weight, weight_row_stride, y,    \
                                            y_row_stride, m, n, k, extra, s);                 \
    else if (epi == kEpiResidual)                                                             \
      launch_kstream_mt<T, false, kEpiResidual>(x, x_row_stride, weight, weight_row_stride, y, \
                                                y_row_stride, m, n, k, extra, s);             \
    else                                                                                      \
      launch_kstream_mt<T, false, kEpiPlain>(x, x_row_stride, weight, weight_row_stride, y,   \
                                             y_row_stride, m, n, k, extra, s);                \
  } while (0)
  if (dtype == TF_DTYPE_BFLOAT16)
    TF_KSTREAM_LAUNCH(__bf16);
  else
    TF_KSTREAM_LAUNCH(_Float16);
#undef TF_KSTREAM_LAUNCH
  return check_launch(name);
}

}  // namespace
}  // namespace tf

extern "C" int32_t tf_linear_kstream(const void *x, int64_t x_row_stride, const void *weight,
                                     int64_t weight_row_stride, void *y, int64_t y_row_stride,
                                     int32_t m, int32_t n, int32_t k, int32_t dtype, void *stream) {
  return tf::kstream_entry(x, x_row_stride, weight, weight_row_stride, y, y_row_stride, m, n, k,
                           dtype, stream, false, tf::kEpiPlain, 0.f, nullptr, 0, "linear_kstream");
}

extern "C" int32_t tf_linear_kstream_norm(const void *x, int64_t x_row_stride,
                                          const void *weight, int64_t weight_row_stride, void *y,
                                          int64_t y_row_stride, int32_t m, int32_t n, int32_t k,
                                          float eps, int32_t dtype, void *stream) {
  return tf::kstream_entry(x, x_row_stride, weight, weight_row_stride, y, y_row_stride, m, n, k,
                           dtype, stream, false, tf::kEpiNorm, eps, nullptr, 0,
                           "linear_kstream_norm");
}

extern "C" int32_t tf_linear_kstream_residual(const void *x, int64_t x_row_stride,
                                              const void *weight, int64_t weight_row_stride,
                                              const void *residual, int64_t residual_row_stride,
                                              void *y, int64_t y_row_stride, int32_t m, int32_t n,
                                              int32_t k, int32_t dtype, void *stream) {
  return tf::kstream_entry(x, x_row_stride, weight, weight_row_stride, y, y_row_stride, m, n, k,
                           dtype, stream, false, tf::kEpiResidual, 0.f, residual,
                           residual_row_stride, "linear_kstream_residual");
}

extern "C" int32_t tf_linear_kswiglu(const void *x, int64_t x_row_stride,
                                     const void *gate_up_weight, int64_t weight_row_stride,
                                     void *y, int64_t y_row_stride, int32_t m,
                                     int32_t intermediate, int32_t k, int32_t dtype,
                                     void *stream) {
  return tf::kstream_entry(x, x_row_stride, gate_up_weight, weight_row_stride, y, y_row_stride,
                           m, intermediate, k, dtype, stream, true, tf::kEpiPlain, 0.f, nullptr, 0,
                           "linear_kswiglu");
}

extern "C" int32_t tf_linear_kswiglu_norm(const void *x, int64_t x_row_stride,
                                          const void *gate_up_weight, int64_t weight_row_stride,
                                          void *y, int64_t y_row_stride, int32_t m,
                                          int32_t intermediate, int32_t k, float eps,
                                          int32_t dtype, void *stream) {
  return tf::kstream_entry(x, x_row_stride, gate_up_weight, weight_row_stride, y, y_row_stride,
                           m, intermediate, k, dtype, stream, true, tf::kEpiNorm, eps, nullptr, 0,
                           "linear_kswiglu_norm");
}
