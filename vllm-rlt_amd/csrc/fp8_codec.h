// OCP e4m3fn encoding shared by the FP8 KV writers (the scatter kernel and the
// attention launch that stores its verify window): bitwise the reference's
// quantize_fp8 (vllm_rlt/core/kv_cache_manager.py:50-61), codes clamped to +-448
// with NaN kept, scales amax * float32(1/448) clamped below at FLT_MIN.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace rlt_fp8 {

constexpr float kMax = 448.f;
constexpr float kTiny = 1.17549435e-38f;  // torch.finfo(torch.float32).tiny

// NaN-propagating maximum, as torch's amax
__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __int_as_float(0x7fc00000) : (a > b ? a : b);
}

// float -> OCP e4m3fn code, round to nearest even; |x| <= 448 or NaN (the
// callers clamp first).  Normals: the 23-bit mantissa rounded to 3 bits on the
// float's bit pattern (a carry moves into the exponent); below the smallest normal
// 2^-6 the value is a multiple of 2^-9, rounded to an integer count of it.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  const uint32_t bits = __float_as_uint(x);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const float a = fabsf(x);
  if (a != a) return sign | 0x7fu;
  uint32_t code;
  if (a < 0.015625f) {                   // 2^-6
    code = (uint32_t)rintf(a * 512.f);   // 0..8 (8 is the smallest normal, 0x08)
  } else {
    const uint32_t b = __float_as_uint(a);
    const uint32_t r = b + 0x7ffffu + ((b >> 20) & 1u);  // round the low 20 bits
    code = (r >> 20) - ((127u - 7u) << 3);
  }
  return sign | code;
}

// Dynamic per-vector scale from the vector's NaN-propagating |x| maximum.
__device__ __forceinline__ float dynamic_scale(float amax) {
  const float inv_max = 1.f / kMax;  // the float32 constant 1/448 (as torch and Triton)
  const float scale = amax * inv_max;
  return scale < kTiny ? kTiny : scale;  // clamp_min(finfo.tiny); NaN stays
}

// The code of x / scale: clamp(-448, 448) with NaN kept, as torch's clamp.
__device__ __forceinline__ uint32_t encode(float x, float scale) {
  const float y = x / scale;
  const float q = y != y ? y : (y < -kMax ? -kMax : (y > kMax ? kMax : y));
  return f32_to_e4m3(q);
}

}  // namespace rlt_fp8
