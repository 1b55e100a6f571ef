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
// A dispatch counts work-items in 32 bits per dimension: blocks * threads must stay below 2^32.
int check_grid(int64_t blocks, int64_t threads, const char* what);

// pq_int8_gemm_packed (pq_gemm.hip), called by the layer entries with a scheduling buffer in their staging.
int int8_gemm_packed(const int8_t* ap, const int8_t* wp, const float* s_row, const float* s_w, int64_t group,
                     const float* bias, const void* t, int64_t ldt, const void* l2t, int64_t R, int32_t lr_dtype,
                     void* c, int64_t ldc, int32_t out_dtype, const int32_t* out_row_idx, int64_t c_rows, int64_t M,
                     int64_t N, int64_t K, int32_t* sched, hipStream_t stream);

// pq_quant_rows_packed / pq_quant_rows_lowrank (pq_quant.hip) that also write zeros to zero9[0 .. 8] (when not NULL)
// in the same kernel: the layer entries clear their GEMM's scheduling buffer this way, with no memset and no extra
// launch (a captured graph clears it on every replay).
int quant_rows_packed_z(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                        const int32_t* row_idx, int8_t* qp, float* s, int32_t* zero9, hipStream_t stream);
int quant_rows_lowrank_z(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                         const int32_t* row_idx, const void* l1t, const void* l1f, int64_t R, int8_t* qp, float* s,
                         void* t, int64_t ldt, int32_t* zero9, hipStream_t stream);

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

// ---- LDS-DMA helpers ---------------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;
constexpr int kBufferWord3 = 0x00020000;   // gfx9 buffer descriptor word 3 (raw, 32-bit data format)
constexpr int kOOB = 0x40000000;           // buffer offset beyond every operand's num_records (loads nothing)

// s_waitcnt vmcnt(N) (expcnt / lgkmcnt left at their maxima). The compiler does not count LDS-DMA loads as
// LDS writes before a barrier, so every hand-over of a DMA-filled LDS stage waits for them explicitly.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// ---- packed K64 layout -----------------------------------------------------------------------------------------
// Slot of 16-byte chunk c of row r' (0..15) of a 1 KB block is c ^ k64_swz(r'): among 8 consecutive rows the
// (row parity, slot) pairs of one chunk are distinct, and among 16 consecutive rows the (row % 4, slot) pairs are,
// so the GEMM's ds_read_b128 of consecutive rows are bank-conflict free in 128- and 256-byte bank windows.
__host__ __device__ __forceinline__ int k64_swz(int r) { return ((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1); }

// Byte offset of element (m, k) of an int8 matrix in the packed K64 layout with KT = K / 64 stages.
__device__ __forceinline__ int64_t k64_offset(int64_t m, int k, int KT) {
  const int r = (int)(m & 15);
  return ((m >> 4) * KT + (k >> 6)) * 1024 + r * 64 + ((((k >> 4) & 3) ^ k64_swz(r)) << 4) + (k & 15);
}

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

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Two fp32 values -> one dword holding two 16-bit values (lo = a, hi = b), round to nearest even
// (gfx950: one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 per pair).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == PQ_BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{a, b}, v2bf));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{a, b}, v2h));
  }
}

}  // namespace pq
