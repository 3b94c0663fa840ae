// Shared definitions for the MI355X (gfx950) speculative-verification kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define RLT_WAVE 64

// Error codes returned by every extern "C" entry point.
enum rlt_status {
  RLT_OK = 0,
  RLT_ERR_ARGUMENT = 1,     // a size, stride, dtype or pointer violates the contract
  RLT_ERR_UNSUPPORTED = 2,  // a legal configuration this build does not implement
  RLT_ERR_WORKSPACE = 3,    // workspace missing or smaller than the queried size
  RLT_ERR_LAUNCH = 4,       // hipGetLastError() reported a launch failure
};

// Element type codes shared with the host wrappers.
enum rlt_dtype {
  RLT_F32 = 0,
  RLT_F16 = 1,
  RLT_BF16 = 2,
  RLT_FP8_E4M3 = 3,  // OCP e4m3fn (torch.float8_e4m3fn), saturating
};

static inline size_t rlt_align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

static inline int rlt_launch_status() {
  return hipGetLastError() == hipSuccess ? RLT_OK : RLT_ERR_LAUNCH;
}

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Two OCP e4m3 bytes (low or high half of a 32-bit word) -> two floats (exact).
template <bool kHigh>
__device__ __forceinline__ float2 fp8x2_to_f32(uint32_t word) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  f32x2 v = __builtin_amdgcn_cvt_pk_f32_fp8((int)word, kHigh);
  return make_float2(v.x, v.y);
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* base, int64_t i);

template <>
__device__ __forceinline__ float load_as_f32<RLT_F32>(const void* base, int64_t i) {
  return ((const float*)base)[i];
}
template <>
__device__ __forceinline__ float load_as_f32<RLT_BF16>(const void* base, int64_t i) {
  return bf16_bits_to_f32(((const uint16_t*)base)[i]);
}
template <>
__device__ __forceinline__ float load_as_f32<RLT_F16>(const void* base, int64_t i) {
  return f16_bits_to_f32(((const uint16_t*)base)[i]);
}
template <>
__device__ __forceinline__ float load_as_f32<RLT_FP8_E4M3>(const void* base, int64_t i) {
  uint32_t b = ((const uint8_t*)base)[i];
  return fp8x2_to_f32<false>(b).x;
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void* base, int64_t i, float v);
template <>
__device__ __forceinline__ void store_from_f32<RLT_F32>(void* base, int64_t i, float v) {
  ((float*)base)[i] = v;
}
template <>
__device__ __forceinline__ void store_from_f32<RLT_BF16>(void* base, int64_t i, float v) {
  ((uint16_t*)base)[i] = f32_to_bf16_bits(v);
}
template <>
__device__ __forceinline__ void store_from_f32<RLT_F16>(void* base, int64_t i, float v) {
  ((uint16_t*)base)[i] = f32_to_f16_bits(v);
}

// ---------------------------------------------------------------- wave helpers

__device__ __forceinline__ float wave_shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, RLT_WAVE);
}
