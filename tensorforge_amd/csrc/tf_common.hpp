// Shared device helpers and host error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdarg>

#include "../../include/tensorforge_amd.h"

namespace tf {

// ---------------------------------------------------------------------------
// Host-side status plumbing.  The message buffer is thread-local so that
// concurrent callers (one per host thread) never see each other's errors.
// ---------------------------------------------------------------------------
void set_error(const char *fmt, ...);
void clear_error();

inline int32_t fail(int32_t status, const char *what) {
  set_error("%s", what);
  return status;
}

inline int32_t check_launch(const char *kernel) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s launch failed: %s", kernel, hipGetErrorString(err));
    return TF_ERROR_LAUNCH;
  }
  return TF_SUCCESS;
}

inline bool valid_dtype(int32_t dtype) {
  return dtype == TF_DTYPE_FLOAT32 || dtype == TF_DTYPE_FLOAT16 ||
         dtype == TF_DTYPE_BFLOAT16;
}

inline int32_t dtype_size(int32_t dtype) {
  return dtype == TF_DTYPE_FLOAT32 ? 4 : 2;
}

// ---------------------------------------------------------------------------
// Element conversions.  Storage types are float, _Float16 and __bf16; the
// narrowing casts compile to the gfx950 round-to-nearest-even converts.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float to_float(T v) {
  return static_cast<float>(v);
}

template <typename T>
__device__ __forceinline__ T from_float(float v) {
  return static_cast<T>(v);
}

// fp32 -> fp16 goes through a rounded fp32 value.  Without the empty asm the
// compiler may fold a final fp32 multiply into the convert
// (v_fma_mixlo_f16: the exact product rounded once to fp16), which differs
// from rounding the fp32 product now and then and would make the scalar and
// vector forms of a kernel disagree.
template <>
__device__ __forceinline__ _Float16 from_float<_Float16>(float v) {
  asm("" : "+v"(v));
  return static_cast<_Float16>(v);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-byte global load with the nontemporal (streaming) cache policy, for
// data a kernel reads once -- the K/V pages of a decode call.  Measured on
// MI355X over config 2's page reads: 21.3 -> 19.5 us for the same loads
// with the default policy.
template <typename V>
__device__ __forceinline__ V load_stream16(const void *p) {
  static_assert(sizeof(V) == 16, "16-byte vectors only");
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return __builtin_bit_cast(V, v);
}

// ---------------------------------------------------------------------------
// Half-split rotary embedding of one pair (x1 = x[j], x2 = x[j + D/2], j < D/2):
//   out[j]       = x1 cos[j]       - x2 sin[j]         (rope_lo)
//   out[j + D/2] = x2 cos[j + D/2] + x1 sin[j + D/2]   (rope_hi)
// with the fused multiply-adds written out, so every kernel that rotates
// (the RoPE + append kernel and the attention kernel that rotates its own
// query group) rounds identically.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float rope_lo(float x1, float x2, float c, float s) {
  return __builtin_fmaf(x1, c, -(x2 * s));
}
__device__ __forceinline__ float rope_hi(float x1, float x2, float c, float s) {
  return __builtin_fmaf(x2, c, x1 * s);
}

// ---------------------------------------------------------------------------
// SwiGLU activation of one element, g * sigmoid(g) * u in fp32 (the caller
// rounds once to the storage type); one definition for every kernel that
// applies it, so they round identically.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float swiglu_act(float g, float u) {
  const float silu = g / (1.0f + expf(-g));
  return silu * u;
}

// c + a . b over 8 elements with the packed two-element dot product
// (v_dot2_f32_bf16 / v_dot2_f32_f16: fp32 products and accumulation): the
// VALU form of the attention score product, and a row's sum of squares in
// the norm-fused projections.
template <typename T>
__device__ __forceinline__ float dot8(T __attribute__((ext_vector_type(8))) a,
                                      T __attribute__((ext_vector_type(8))) b, float c);

template <>
__device__ __forceinline__ float dot8<__bf16>(__bf16 __attribute__((ext_vector_type(8))) a,
                                              __bf16 __attribute__((ext_vector_type(8))) b,
                                              float c) {
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 0, 1),
                                      __builtin_shufflevector(b, b, 0, 1), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 2, 3),
                                      __builtin_shufflevector(b, b, 2, 3), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 4, 5),
                                      __builtin_shufflevector(b, b, 4, 5), c, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(a, a, 6, 7),
                                         __builtin_shufflevector(b, b, 6, 7), c, false);
}

template <>
__device__ __forceinline__ float dot8<_Float16>(_Float16 __attribute__((ext_vector_type(8))) a,
                                                _Float16 __attribute__((ext_vector_type(8))) b,
                                                float c) {
  c = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 0, 1),
                             __builtin_shufflevector(b, b, 0, 1), c, false);
  c = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 2, 3),
                             __builtin_shufflevector(b, b, 2, 3), c, false);
  c = __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 4, 5),
                             __builtin_shufflevector(b, b, 4, 5), c, false);
  return __builtin_amdgcn_fdot2(__builtin_shufflevector(a, a, 6, 7),
                                __builtin_shufflevector(b, b, 6, 7), c, false);
}

// ---------------------------------------------------------------------------
// Wavefront (64-lane) reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
  return v;
}

}  // namespace tf
