// Device-side helpers shared by the kernels: number formats, rounding, vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tmh {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

// Dequantization / storage types, as the ONNX codes of the C ABI.
enum : int { DT_F32 = 1, DT_F16 = 10, DT_BF16 = 16 };

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// The f32 value of an f32 result rounded to type DT (the reference computes each operation of
// a narrow type in f32 and rounds once).
template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == DT_F16) {
    return static_cast<float>(static_cast<_Float16>(x));
  } else if constexpr (DT == DT_BF16) {
    return bf16_bits_to_f32(f32_to_bf16_bits(x));
  } else {
    return x;
  }
}

// (q - zero) * scale in type DT, each operation rounded (Packed.dequantize/3); zero and
// scale already hold DT values.
template <int DT>
__device__ __forceinline__ float dequant_value(float q, float zero, float scale) {
  float d = round_to<DT>(q - zero);
  return round_to<DT>(d * scale);
}

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i) {
  if constexpr (DT == DT_F16) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else if constexpr (DT == DT_BF16) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return static_cast<const float*>(p)[i];
  }
}

// A float element of runtime type dt (1 = f32, 10 = f16, 16 = bf16).
__device__ __forceinline__ float load_float_rt(const void* p, int dt, int64_t i) {
  if (dt == DT_F16) return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dt == DT_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_float_rt(void* p, int dt, int64_t i, float v) {
  if (dt == DT_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  } else if (dt == DT_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

template <int DT>
__device__ __forceinline__ void store_as(void* p, int64_t i, float v) {
  if constexpr (DT == DT_F16) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  } else if constexpr (DT == DT_BF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

// Value i (0 <= i < 32/BITS) of a 32-bit word of the tiled weight layout: value 2j at bits
// j*BITS, value 2j+1 at bits 16 + j*BITS (8-bit words keep their byte order).
template <int BITS>
__device__ __forceinline__ uint32_t word_value(uint32_t x, int i) {
  if constexpr (BITS == 8) {
    return (x >> (8 * i)) & 0xFFu;
  } else {
    const int pos = (i & 1) * 16 + (i >> 1) * BITS;
    return (x >> pos) & ((1u << BITS) - 1u);
  }
}

}  // namespace tmh
