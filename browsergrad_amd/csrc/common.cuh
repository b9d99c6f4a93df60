// Device helpers shared by the kernel translation units.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace bgk {

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t v) {
  return __uint_as_float(uint32_t(v) << 16);
}

// Round-to-nearest-even f32 -> bf16 bits (gfx950 v_cvt_pk_bf16_f32; NaN
// stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Round-to-nearest-even f32 -> f16 bits (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// dtype codes follow include/bghip.h (0 f32, 1 f16, 2 bf16).
__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  if (dtype == 0) return static_cast<const float*>(p)[i];
  const uint16_t v = static_cast<const uint16_t*>(p)[i];
  return dtype == 1 ? f16_bits_to_f32(v) : bf16_bits_to_f32(v);
}

__device__ __forceinline__ void store_from_f32(void* p, int dtype, int64_t i, float x) {
  if (dtype == 0) {
    static_cast<float*>(p)[i] = x;
  } else {
    static_cast<uint16_t*>(p)[i] = dtype == 1 ? f32_to_f16_bits(x) : f32_to_bf16_bits(x);
  }
}

// Round an f32 value through the 16-bit dtype (1 f16, 2 bf16) and back.
__device__ __forceinline__ float round_through(float x, int dtype) {
  if (dtype == 1) return static_cast<float>(static_cast<_Float16>(x));
  if (dtype == 2) return static_cast<float>(static_cast<__bf16>(x));
  return x;
}

// The reference's tanh-approximate GELU, op for op in f32
// (_functional.py:123-134 with tanh from _functional.py:115-120):
//   0.5*x * (1 + (e^u - e^-u)/(e^u + e^-u)),  u = c*(x + ((0.044715*x)*x)*x)
__device__ __forceinline__ float gelu_tanh_ref(float x) {
  const float c = 0.7978845608028654f;  // sqrt(2/pi) rounded to f32
  float half_x = 0.5f * x;
  float cube = 0.044715f * x;
  cube = cube * x;
  cube = cube * x;
  float inner = x + cube;
  float u = c * inner;
  float ep = expf(u);
  float en = expf(-u);
  float num = ep + (-en);
  float den = ep + en;
  float th = num / den;
  float one_plus = 1.0f + th;
  return half_x * one_plus;
}

}  // namespace bgk
