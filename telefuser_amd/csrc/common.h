// Shared device helpers and host-side error plumbing for libqattn (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "qattn.h"

namespace qattn {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------------
// host: error reporting
// ------------------------------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

#define QATTN_REQUIRE(cond, code, ...)        \
  do {                                        \
    if (!(cond)) return ::qattn::set_error((code), __VA_ARGS__); \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------------------------------------------
// device: half <-> float
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 x;
  __builtin_memcpy(&x, &h, 2);
  return (float)x;
}

template <bool IS_FP16>
__device__ __forceinline__ float half_to_f32(uint16_t h) {
  if constexpr (IS_FP16) return f16_to_f32(h);
  else return bf16_to_f32(h);
}

// round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  _Float16 x = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  uint16_t h;
  __builtin_memcpy(&h, &x, 2);
  return h;
}

template <bool IS_FP16>
__device__ __forceinline__ uint16_t f32_to_half(float f) {
  if constexpr (IS_FP16) return f32_to_f16(f);
  else return f32_to_bf16(f);
}

// ------------------------------------------------------------------------------------------------
// device: the quantizers' rounding (shared by the quantizer kernels and the attention kernels that
// quantize Q themselves)
// ------------------------------------------------------------------------------------------------
// v_cvt_i32_f32: truncate toward zero, saturate to the int32 range, NaN -> 0 (the hardware conversion; a C
// cast leaves NaN and out-of-range values undefined)
__device__ __forceinline__ int cvt_i32_trunc_sat(float t) {
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(t));
  return r;
}

// a / b, correctly rounded, from y1 = refined_rcp(b): the fma corrections of the IEEE division sequence
// without its range scaling (div_scale / div_fixup).  Exact wherever the residuals do not underflow: the
// quantizers divide |a| <= 127 b with b >= 1e-7, where only quotients below 2^-80 (which quantize to 0
// either way) can differ.
__device__ __forceinline__ float refined_rcp(float b) {
  const float y0 = __builtin_amdgcn_rcpf(b);
  return fmaf(fmaf(-b, y0, 1.0f), y0, y0);
}
__device__ __forceinline__ float div_by(float a, float b, float y1) {
  const float q0 = a * y1;
  const float q1 = fmaf(fmaf(-b, q0, a), y1, q0);
  return fmaf(fmaf(-b, q1, a), y1, q1);
}

// Scales of the per-block / per-warp (CUDA QuantInt8Kernel: amax / 127, codes RNE(x * 127 / amax)) and
// per-thread (Triton: amax / 127 + 1e-7, codes round-half-away(x / scale)) quantizers from the |x| maximum
__device__ __forceinline__ float quant_scale_cuda(float amax) { return amax / 127.0f; }
__device__ __forceinline__ float quant_recip_cuda(float amax) { return 127.0f / amax; }
__device__ __forceinline__ float quant_scale_triton(float amax) { return amax / 127.0f + 0.0000001f; }
__device__ __forceinline__ int quant_code_cuda(float x, float recip) { return cvt_i32_trunc_sat(__builtin_rintf(x * recip)); }
__device__ __forceinline__ int quant_code_triton(float x, float scale, float rcp_scale) {
  const float t = div_by(x, scale, rcp_scale);
  return cvt_i32_trunc_sat(t + __builtin_copysignf(0.5f, t));
}

// Rows [start, start + len) of sequence b of a packed variable-length batch: cu[b] .. cu[b + 1] clamped to
// the packed tensor's `total` rows and to `maxlen`, so that a malformed sequence table cannot address
// memory outside the packed tensors (every varlen kernel and the block-offset kernel use this).
__device__ __forceinline__ void varlen_range(const int32_t* cu, int64_t b, int64_t total, int64_t maxlen,
                                             int64_t& start, int64_t& len) {
  const int64_t s0 = min(max((int64_t)cu[b], (int64_t)0), total);
  const int64_t s1 = min(max((int64_t)cu[b + 1], s0), total);
  start = s0;
  len = min(s1 - s0, maxlen);
}

// wave64 reductions (DPP / permute through the compiler's shuffle lowering)
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace qattn
