// Shared helpers of the gfx950 kernels: error reporting of the C ABI, 16-bit float conversions,
// vector types of the MFMA operands.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/pyraquant_amd.h"

namespace pq {

// ---- C-ABI error reporting (thread-local text, returned status code) --------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---- vector types of the MFMA operands -----------------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// ---- 16-bit float <-> fp32 (exact widening; round-to-nearest-even narrowing) ----------------------------
template <int DT>
__device__ __forceinline__ float lo16_to_f32(uint32_t w) {
  if constexpr (DT == PQ_BF16) {
    return __uint_as_float(w << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
  }
}
template <int DT>
__device__ __forceinline__ float hi16_to_f32(uint32_t w) {
  if constexpr (DT == PQ_BF16) {
    return __uint_as_float(w & 0xffff0000u);
  } else {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
  }
}

// fp32 -> bf16 bits, round to nearest even (NaN -> quiet NaN), the rounding of torch's .to(bfloat16).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

template <int DT>
__device__ __forceinline__ uint32_t f32_to_16_bits(float f) {
  if constexpr (DT == PQ_BF16) {
    return f32_to_bf16_bits(f);
  } else {
    return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f);
  }
}

// Two fp32 values -> one dword holding two 16-bit values (lo = a, hi = b).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return f32_to_16_bits<DT>(a) | (f32_to_16_bits<DT>(b) << 16);
}

}  // namespace pq
