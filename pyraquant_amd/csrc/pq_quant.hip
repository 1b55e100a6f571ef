// Per-token INT8 activation quantizer (with the routed row gather), the rank-R low-rank down-projection
// and the stand-alone dequant epilogue, for gfx950.
//
// Quantizer semantics (reference: deploy/int8_exec.py:78-101, torch restatement :508-509):
//   a = max(max_k |x|, 1e-8f); s = a / 127 (IEEE fp32); q = clamp(rint(x / s), -127, 127) with an IEEE
//   fp32 division and rint = round half to even.
// One wavefront owns one row. The row is loaded once with 16-byte loads and kept in registers (CH chunks
// of 8 elements per lane), so x is read from HBM exactly once. The absmax is a packed-u16 max over the
// magnitude bits (monotonic in |x| for finite 16-bit floats) and a wave reduction.
//
// Exact codes without one IEEE division per element: with c = fl(1/s) and v = x * c (exact product),
// |v - x / s| <= |x| |c - 1/s| <= 127 * 2^-24 and |x / s - fl(x / s)| <= 127 * 2^-24, so |v - fl(x / s)| < 1.6e-5:
// whenever v is farther than kTieMargin from every half-integer, rint(v) == rint(fl(x / s)). One fma gives
// m = fl(v + 1.5 * 2^23) = 1.5 * 2^23 + rint(v) (round to nearest even; |v| < 2^22), whose low byte is the int8
// code, and a second gives the residual fl(v - rint(v)), whose largest magnitude over 8 elements is tested once.
// Chunks with an element within the margin (about one element in 10^4) redo it with the correctly rounded division.
#include "pq_common.h"

#include <algorithm>
#include <type_traits>
#include <stdarg.h>
#include <stdio.h>

namespace pq {

namespace {

constexpr float kMagic = 12582912.0f;        // 1.5 * 2^23: x + kMagic rounds x to an integer (|x| < 2^22)
constexpr float kTieMargin = 6.0e-5f;        // > 1.6e-5 error bound of v, see the header comment
constexpr float kNearHalf = 0.5f - kTieMargin;

// Code of one element: returns kMagic + q as fp32 (its low byte is the int8 code q).
__device__ __forceinline__ float code_exact(float x, float s) {
  float q = rintf(__fdiv_rn(x, s));
  q = fminf(fmaxf(q, -127.0f), 127.0f);
  return q + kMagic;
}

// Low bytes of four fp32 bit patterns packed into one dword (three byte permutes).
__device__ __forceinline__ uint32_t low_bytes4(float m0, float m1, float m2, float m3) {
  const uint32_t a = __builtin_amdgcn_perm(__float_as_uint(m1), __float_as_uint(m0), 0x0c0c0400u);   // m0.b0 m1.b0
  const uint32_t b = __builtin_amdgcn_perm(__float_as_uint(m3), __float_as_uint(m2), 0x0c0c0400u);   // m2.b0 m3.b0
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}

// Quantize 8 elements held in one 16-byte chunk; returns 8 int8 codes packed in a uint2.
template <int DT>
__device__ __forceinline__ v2u quant_chunk(v4u v, float s, float rc) {
  float f[8];
  f[0] = lo16_to_f32<DT>(v.x); f[1] = hi16_to_f32<DT>(v.x);
  f[2] = lo16_to_f32<DT>(v.y); f[3] = hi16_to_f32<DT>(v.y);
  f[4] = lo16_to_f32<DT>(v.z); f[5] = hi16_to_f32<DT>(v.z);
  f[6] = lo16_to_f32<DT>(v.w); f[7] = hi16_to_f32<DT>(v.w);
  float m[8];
  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m[i] = __builtin_fmaf(f[i], rc, kMagic);
    d = fmaxf(d, fabsf(__builtin_fmaf(f[i], rc, -(m[i] - kMagic))));
  }
  if (__builtin_expect(d > kNearHalf, 0)) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (fabsf(__builtin_fmaf(f[i], rc, -(m[i] - kMagic))) > kNearHalf) m[i] = code_exact(f[i], s);
  }
  return v2u{low_bytes4(m[0], m[1], m[2], m[3]), low_bytes4(m[4], m[5], m[6], m[7])};
}

// Maximum over the 64 lanes of a wave, for values below 2^31, in DPP row operations (no LDS round trip): quad_perm
// [1,0,3,2] and [2,3,0,1] within groups of 4 lanes, the half-row and row mirrors within 8 and 16, then row_bcast:15
// (lane 15 of rows 0 and 2 into rows 1 and 3) and row_bcast:31 (lane 31 into rows 2 and 3), after which lane 63
// holds the maximum of all 64; readlane makes it wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  int x = (int)v;
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0xb1, 0xf, 0xf, false));    // quad_perm [1,0,3,2]
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x4e, 0xf, 0xf, false));    // quad_perm [2,3,0,1]
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x141, 0xf, 0xf, false));   // row_half_mirror
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x140, 0xf, 0xf, false));   // row_mirror
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x142, 0xa, 0xf, false));   // row_bcast:15 -> rows 1, 3
  x = max(x, __builtin_amdgcn_update_dpp(x, x, 0x143, 0xc, 0xf, false));   // row_bcast:31 -> rows 2, 3
  return (uint32_t)__builtin_amdgcn_readlane(x, 63);
}

// Magnitude bits of a 16-bit float pair -> fp32 of the larger magnitude.
template <int DT>
__device__ __forceinline__ float absmax_from_bits(uint32_t mag16) {
  return lo16_to_f32<DT>(mag16);
}

// Vectorised quantizer: one wave per row, CH 16-byte chunks per lane, 4 rows per 256-thread block.
// PACKED: codes go to the packed K64 layout (8-byte stores at k64_offset), and the waves of the padding rows
// M .. 16 * ceil(M / 16) - 1 write zeros there. A gathered source row outside [0, x_rows) reads as zeros.
template <int DT, int CH, bool PACKED>
__global__ __launch_bounds__(256) void quant_rows_vec_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int K, int64_t M, const int32_t* __restrict__ row_idx,
    int8_t* __restrict__ q, float* __restrict__ s, int64_t x_rows, int32_t* __restrict__ zero9) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nvec = K >> 3;
  if (zero9 && blockIdx.x == 0 && threadIdx.x < 9) zero9[threadIdx.x] = 0;
  if constexpr (PACKED) {
    if (m >= M) {
      if (m < ((M + 15) & ~15LL)) {
        for (int idx = lane; idx < nvec; idx += 64)
          *reinterpret_cast<v2u*>(q + k64_offset(m, idx * 8, K >> 6)) = v2u{0u, 0u};
      }
      return;
    }
  }
  if (m >= M) return;
  const int64_t src = row_idx ? (int64_t)row_idx[m] : m;
  const bool live = src >= 0 && src < x_rows;
  const v4u* __restrict__ xr = reinterpret_cast<const v4u*>(x + (live ? src : 0) * ldx);
  v4u v[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = c * 64 + lane;
    v[c] = live && idx < nvec ? __builtin_nontemporal_load(xr + idx) : v4u{0u, 0u, 0u, 0u};
  }
  us2 mx2 = {0, 0};
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[c].x & 0x7fff7fffu));
    mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[c].y & 0x7fff7fffu));
    mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[c].z & 0x7fff7fffu));
    mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[c].w & 0x7fff7fffu));
  }
  uint32_t mx = mx2.x > mx2.y ? mx2.x : mx2.y;
  mx = wave_max_u32(mx);
  const float a = fmaxf(absmax_from_bits<DT>(mx), 1e-8f);
  const float sc = __fdiv_rn(a, 127.0f);
  const float rc = __fdiv_rn(1.0f, sc);
  v2u* __restrict__ qr = reinterpret_cast<v2u*>(q + m * (int64_t)K);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = c * 64 + lane;
    if (idx < nvec) {
      const v2u codes = quant_chunk<DT>(v[c], sc, rc);
      if constexpr (PACKED) {
        *reinterpret_cast<v2u*>(q + k64_offset(m, idx * 8, K >> 6)) = codes;
      } else {
        qr[idx] = codes;
      }
    }
  }
  if (lane == 0) s[m] = sc;
}

// Per-element quantizer for unaligned rows or odd K: one wave per row, two sweeps over the row (a gathered source row
// outside [0, x_rows) reads as zeros).
template <int DT, bool PACKED>
__global__ __launch_bounds__(256) void quant_rows_scalar_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int K, int64_t M, const int32_t* __restrict__ row_idx,
    int8_t* __restrict__ q, float* __restrict__ s, int64_t x_rows, int32_t* __restrict__ zero9) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (zero9 && blockIdx.x == 0 && threadIdx.x < 9) zero9[threadIdx.x] = 0;
  if constexpr (PACKED) {
    if (m >= M) {
      if (m < ((M + 15) & ~15LL)) {
        for (int k = lane; k < K; k += 64) q[k64_offset(m, k, K >> 6)] = 0;
      }
      return;
    }
  }
  if (m >= M) return;
  const int64_t src = row_idx ? (int64_t)row_idx[m] : m;
  const bool live = src >= 0 && src < x_rows;
  const uint16_t* __restrict__ xr = x + (live ? src : 0) * ldx;
  uint32_t mx = 0;
  for (int k = lane; k < K; k += 64) {
    const uint32_t b = live ? xr[k] & 0x7fffu : 0u;
    mx = b > mx ? b : mx;
  }
  mx = wave_max_u32(mx);
  const float a = fmaxf(absmax_from_bits<DT>(mx), 1e-8f);
  const float sc = __fdiv_rn(a, 127.0f);
  int8_t* __restrict__ qr = q + m * (int64_t)K;
  for (int k = lane; k < K; k += 64) {
    const float f = live ? lo16_to_f32<DT>(xr[k]) : 0.0f;
    const int8_t code = (int8_t)(__float_as_uint(code_exact(f, sc)) & 0xffu);
    if constexpr (PACKED) {
      q[k64_offset(m, k, K >> 6)] = code;
    } else {
      qr[k] = code;
    }
  }
  if (lane == 0) s[m] = sc;
}

template <int DT, bool PACKED>
int launch_quant(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t x_rows, const int32_t* row_idx, int8_t* q,
                 float* s, int32_t* zero9, hipStream_t stream) {
  const dim3 block(256);
  const int64_t rows = PACKED ? ((M + 15) & ~15LL) : M;
  if (const int st = check_grid((rows + 3) / 4, 256, "quant_rows")) return st;
  const dim3 grid((unsigned)((rows + 3) / 4));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const bool vec = ((uintptr_t)x % 16 == 0) && (ldx % 8 == 0) && (K % 8 == 0) && ((uintptr_t)q % 8 == 0);
  const int need = (int)((K / 8 + 63) / 64);
  if (vec && need <= 32) {
#define PQ_QCASE(C)                                                                                       \
  if (need <= C) {                                                                                        \
    hipLaunchKernelGGL((quant_rows_vec_kernel<DT, C, PACKED>), grid, block, 0, stream, xp, ldx, (int)K, M, \
                       row_idx, q, s, x_rows, zero9);                                                     \
    return check_launch("quant_rows_vec");                                                                \
  }
    PQ_QCASE(1) PQ_QCASE(2) PQ_QCASE(3) PQ_QCASE(4) PQ_QCASE(5) PQ_QCASE(6) PQ_QCASE(8) PQ_QCASE(10)
    PQ_QCASE(12) PQ_QCASE(16) PQ_QCASE(20) PQ_QCASE(24) PQ_QCASE(32)
#undef PQ_QCASE
  }
  hipLaunchKernelGGL((quant_rows_scalar_kernel<DT, PACKED>), grid, block, 0, stream, xp, ldx, (int)K, M, row_idx,
                     q, s, x_rows, zero9);
  return check_launch("quant_rows_scalar");
}

// ---- low-rank down-projection t = x[rows] @ L1 (x: [*, ldx], l1t = L1^T: [R, K]) --------------------
// One wave owns 32 rows and all R output columns; bf16/fp16 MFMA 32x32x16 with fp32 accumulation.
// Lane l feeds row (l % 32) and the 8-element K slice (l / 32) * 8 of every 16-wide step, for both
// operands, so the MFMA sums exactly the products x[row, k] * L1[k, col].
template <int DT, int RB>
__global__ __launch_bounds__(256) void lowrank_down_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int K, int64_t M, const int32_t* __restrict__ row_idx,
    const uint16_t* __restrict__ l1t, uint16_t* __restrict__ t, int64_t ldt, int64_t x_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 32;
  if (r0 >= M) return;
  int64_t mrow = r0 + (lane & 31);
  const int64_t mcl = mrow < M ? mrow : M - 1;
  const int64_t src = row_idx ? (int64_t)row_idx[mcl] : mcl;
  const bool live = src >= 0 && src < x_rows;   // a gathered row outside x reads as zeros
  const uint16_t* __restrict__ xr = x + (live ? src : 0) * ldx + (lane >> 5) * 8;
  const uint16_t* __restrict__ lr = l1t + (int64_t)(lane & 31) * K + (lane >> 5) * 8;
  v16f acc[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) acc[b] = v16f{};
  const int koff = (lane >> 5) * 8;
  for (int k0 = 0; k0 < K; k0 += 16) {
    const bool in = (k0 + koff) < K;
    const v4u xa = in && live ? *reinterpret_cast<const v4u*>(xr + k0) : v4u{0u, 0u, 0u, 0u};
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const v4u lb = in ? *reinterpret_cast<const v4u*>(lr + (int64_t)b * 32 * K + k0) : v4u{0u, 0u, 0u, 0u};
      if constexpr (DT == PQ_BF16) {
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, xa),
                                                         __builtin_bit_cast(v8bf, lb), acc[b], 0, 0, 0);
      } else {
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, xa),
                                                        __builtin_bit_cast(v8h, lb), acc[b], 0, 0, 0);
      }
    }
  }
  // D[i][j]: i = x row block index 8*(r/4) + 4*(lane/32) + r%4, j = output column (lane % 32).
#pragma unroll
  for (int b = 0; b < RB; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = r0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (row < M) t[row * ldt + b * 32 + (lane & 31)] = (uint16_t)f32_to_16_bits<DT>(acc[b][r]);
    }
  }
}

// ---- weight RTN (one-off at conversion) -----------------------------------------------------------------------
// Per output channel (group == 0, deploy/int8_exec.py:355-357) or per group of `group` consecutive K elements
// (pyraquant/quantizers_weight.py:96-109): s = max(absmax, 1e-8) / 127 and q = clamp(rint(w / s), -127, 127),
// both IEEE fp32 divisions. One wave per (row, group) segment; s is [N, K / group] ([N] per channel).
__global__ __launch_bounds__(256) void quant_weight_kernel(const float* __restrict__ w, int64_t ldw, int N, int K,
                                                           int group, int8_t* __restrict__ q, float* __restrict__ s) {
  const int lane = threadIdx.x & 63;
  const int G = K / group;
  const int64_t seg = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (seg >= (int64_t)N * G) return;
  const int64_t n = seg / G;
  const int g = (int)(seg - n * G);
  const float* __restrict__ wr = w + n * ldw + (int64_t)g * group;
  float a = 0.0f;
  for (int k = lane; k < group; k += 64) a = fmaxf(a, fabsf(wr[k]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 64));
  a = fmaxf(a, 1e-8f);
  const float sc = __fdiv_rn(a, 127.0f);
  int8_t* __restrict__ qr = q + n * (int64_t)K + (int64_t)g * group;
  for (int k = lane; k < group; k += 64) qr[k] = (int8_t)(__float_as_uint(code_exact(wr[k], sc)) & 0xffu);
  if (lane == 0) s[seg] = sc;
}

// ---- row-major int8 -> packed K64 layout (one-off, weights) --------------------------------------------------
// One thread per 16-byte slot of the destination: slot (r', p) of block (rb, kt) receives chunk p ^ swz(r') of
// row 16 rb + r' (zeros past the last row).
__global__ __launch_bounds__(256) void pack_k64_kernel(const int8_t* __restrict__ src, int64_t R, int KT, int64_t lds,
                                                       int8_t* __restrict__ dst, int64_t nslots) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= nslots) return;
  const int64_t blk = t >> 6;
  const int within = (int)(t & 63);
  const int rr = within >> 2, slot = within & 3;
  const int64_t rb = blk / KT;
  const int kt = (int)(blk - rb * KT);
  const int64_t r = rb * 16 + rr;
  v4i v = {0, 0, 0, 0};
  if (r < R) v = *reinterpret_cast<const v4i*>(src + r * lds + kt * 64 + ((slot ^ k64_swz(rr)) << 4));
  *reinterpret_cast<v4i*>(dst + t * 16) = v;
}

// ---- low-rank down-projection over an LDS-DMA ring (K % 64 == 0) ------------------------------------------------
// t[m, :] = x[src(m), :] @ L1 with src(m) = row_idx ? row_idx[m] : m. A workgroup (4 waves) owns 128 output rows,
// 32 per wave; K streams in 64-element (128-byte) stages through a 4-stage LDS ring filled by LDS-DMA: 128 rows of
// x plus the R rows of l1t (= L1^T) for the stage. One DMA instruction fills 8 LDS rows of 128 bytes (each lane the
// 16-byte chunk the swizzle puts at its slot), so every request is a whole row segment and x is read exactly once.
// Per 16-wide K step a wave does R / 32 bf16/fp16 MFMA 32x32x16 with D[r][m] = sum_k l1t[r, k] x[m, k] (fp32), then
// rounds to the 16-bit type (round to nearest even).
constexpr int kLrRows = 128;
constexpr int kLrNS = 4;

template <int DT, int RB>
__global__ __launch_bounds__(256) void lowrank_down_dma_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t x_rows, int K, int64_t M, const int32_t* __restrict__ row_idx,
    const uint16_t* __restrict__ l1t, uint16_t* __restrict__ t, int64_t ldt) {
  constexpr int XB = kLrRows * 128, LB = RB * 32 * 128, STAGE = XB + LB;
  constexpr int DPW = 4 + RB;   // DMA instructions per wave and stage: 4 for x, RB for l1t
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLrNS * STAGE];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t m0 = (int64_t)blockIdx.x * kLrRows;
  const int KT = K / 64;

  const __amdgpu_buffer_rsrc_t rs_x = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, (int)(x_rows * ldx * 2), kBufferWord3);
  const __amdgpu_buffer_rsrc_t rs_l = __builtin_amdgcn_make_buffer_rsrc((void*)l1t, (short)0, RB * 32 * K * 2, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rs_none = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, 0, kBufferWord3);

  // x: instruction i fills rows (4 wave + i) * 8 + lane / 8 of the block; row % 8 = lane / 8 and row / 8 % 2 = i % 2
  int vx[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = min(m0 + (wave * 4 + i) * 8 + (lane >> 3), M - 1);
    const int64_t src = row_idx ? (int64_t)row_idx[m] : m;
    // a gathered row outside x: offset kOOB, the DMA loads zeros
    vx[i] = src >= 0 && src < x_rows ? (int)(src * ldx * 2) + (((lane & 7) ^ (lane >> 3) ^ (i & 1)) << 4) : kOOB;
  }
  // l1t: instruction j fills rows 32 j + 8 wave + lane / 8; row % 8 = lane / 8 and row / 8 % 2 = wave % 2
  const int vl = ((wave * 8 + (lane >> 3)) * K) * 2 + (((lane & 7) ^ (lane >> 3) ^ (wave & 1)) << 4);

  auto dma = [&](int buf, int kt) {
    uint8_t* sb = smem + buf * STAGE;
    const bool live = kt < KT;   // past the end of K: a zero-size descriptor, the loads read nothing
    const __amdgpu_buffer_rsrc_t rx = live ? rs_x : rs_none;
    const __amdgpu_buffer_rsrc_t rl = live ? rs_l : rs_none;
    const int ko = live ? kt * 128 : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(sb + (wave * 4 + i) * 1024), 16, vx[i] + ko, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < RB; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (lds_void_t*)(sb + XB + (j * 4 + wave) * 1024), 16,
                                               vl + j * 32 * K * 2 + ko, 0, 0, 0);
  };

  const int sw = (lane & 7) ^ ((lane >> 3) & 1);
  const int kh = lane >> 5;
  const int xo = (wave * 32 + (lane & 31)) * 128;
  const int lo = XB + (lane & 31) * 128;
  v16f acc[RB];
#pragma unroll
  for (int j = 0; j < RB; ++j) acc[j] = v16f{};

#pragma unroll
  for (int st = 0; st < kLrNS; ++st) dma(st, st);
  wait_vmcnt<(kLrNS - 1) * DPW>();
  __syncthreads();
  int b = 0;
  for (int kt = 0; kt < KT; ++kt) {
    const uint8_t* sb = smem + b * STAGE;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = ((2 * s + kh) ^ sw) << 4;
      const v4i xf = *reinterpret_cast<const v4i*>(sb + xo + c);
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const v4i lf = *reinterpret_cast<const v4i*>(sb + lo + j * 32 * 128 + c);
        if constexpr (DT == PQ_BF16) {
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, lf), __builtin_bit_cast(v8bf, xf), acc[j], 0, 0, 0);
        } else {
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, lf), __builtin_bit_cast(v8h, xf), acc[j], 0, 0, 0);
        }
      }
    }
    wait_vmcnt<(kLrNS - 2) * DPW>();   // this wave's DMA of stage kt + 1 has landed
    __syncthreads();                    // every wave's has, and every wave is done reading buffer b
    dma(b, kt + kLrNS);
    b = b + 1 == kLrNS ? 0 : b + 1;
  }
  wait_vmcnt<0>();
  // D[r][m]: lane holds row m = wave * 32 + lane % 32 and r = 32 j + 8 q + 4 (lane / 32) + (0..3)
  const int64_t m = m0 + wave * 32 + (lane & 31);
  if (m < M) {
    uint16_t* trow = t + m * ldt + 4 * kh;
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<v2u*>(trow + j * 32 + 8 * q) =
            v2u{pack2<DT>(acc[j][4 * q + 0], acc[j][4 * q + 1]), pack2<DT>(acc[j][4 * q + 2], acc[j][4 * q + 3])};
  }
}

// Byte offset of output row m's source row in x (x_rows * ldx * 2 < 2^30), or kOOB (a DMA that loads zeros) past M
// and for a gathered row outside [0, x_rows).
__device__ __forceinline__ int row_byte_offset(int64_t m, int64_t M, const int32_t* __restrict__ row_idx, int64_t ldx,
                                               int64_t x_rows) {
  if (m >= M) return kOOB;
  const int64_t src = row_idx ? (int64_t)row_idx[m] : m;
  return src >= 0 && src < x_rows ? (int)(src * ldx * 2) : kOOB;
}

// ---- fused quantizer + low-rank down-projection (one read of x) ----------------------------------------------
// pq_quant_rows_packed and pq_lowrank_down (R = 32) in one pass: deploy/int8_exec.py:390-391 computes
// t = x @ lr_A and quant_rows(x) from the same x, and both need every element of a row.
// One workgroup of W waves per CU, persistent over batches of 16 rows. A batch is brought into LDS by LDS-DMA in
// 1 KB row-contiguous pieces (the DRAM-friendly pattern of the row-per-wave quantizer), then every wave reads its
// K slice [w K / W, (w + 1) K / W) of the 16 rows into registers (lane: row l % 16, K group l / 16), the DMA of the
// next batch is issued into the freed buffer, and the wave works from registers:
//   absmax over the slice -> LDS -> the row scale (the same IEEE steps as quant_rows_vec_kernel); codes from the
//   registers (quant_chunk), each wave storing whole 16-row x 64-byte packed K64 blocks;
//   t partial = the slice of x . l1t by v_mfma_f32_16x16x32, whose l1t slice stays in registers for the whole
//   kernel -> LDS -> t = (..((p0 + p1) + p2) ..) + p(W-1) in fp32, rounded to the 16-bit type.
// The l1t slice comes from l1f when given: the same matrix in fragment order (pack_lowrank_l1t_kernel), where each
// of the wave's 4 NC register loads is one contiguous 1 KB piece. From row-major l1t each load touches 16 rows at
// half a cache line apiece; with one batch per workgroup (c0: M = 4096, 256 batches) the whole 192 KB slice set is
// on the critical path, and the fragment order takes the pass from 15.8 to 12.8 us.
// W = 16 where K allows it (K % 1024 == 0), else 8, else 4: the batch's work is spread over more waves while the
// single LDS batch buffer (the memory pipeline) stays the same (c1: 143 -> 130 us from W = 4 to 16).
// K assignment inside the 64-wide K block c of a slice (MFMA steps 2c and 2c + 1): lane group g covers
// K [64 c + 16 g, +16), 8 values per step. Both MFMA operands use it, so each step contracts 32 distinct K; the
// 16 codes a lane produces per block are chunk g of its row's 64-byte segment.
template <int DT, int NC, int W>   // W waves, NC: 64-wide K blocks per wave, K = 64 W NC
__global__ __launch_bounds__(64 * W, 1) void quant_lowrank_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t x_rows, int64_t M, const int32_t* __restrict__ row_idx,
    const uint16_t* __restrict__ l1t, const uint16_t* __restrict__ l1f, int8_t* __restrict__ qp,
    float* __restrict__ s, uint16_t* __restrict__ t, int64_t ldt, int nbatch, int32_t* __restrict__ zero9) {
  constexpr int K = 64 * W * NC, R = 32, NS = 2 * NC;
  // (an older vector store than every DMA the ring counts: the vmcnt waits below only wait for it as well)
  if (zero9 && blockIdx.x == 0 && threadIdx.x < 9) zero9[threadIdx.x] = 0;
  constexpr int CHUNKS = (2 * K + 1023) / 1024;      // 1 KB DMA pieces per row
  constexpr int PITCH = CHUNKS * 1024 + 64;          // LDS row pitch (+64 bytes: rows start 16 banks apart)
  __shared__ __attribute__((aligned(1024))) uint8_t xs[16 * PITCH];
  __shared__ uint32_t amax_l[W][16];
  __shared__ __attribute__((aligned(16))) float red[W][16][R];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int k0 = wave * (K / W);
  const int G = gridDim.x;
  const __amdgpu_buffer_rsrc_t rs_x =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, (int)(x_rows * ldx * 2), kBufferWord3);

  // DMA of batch b: wave w copies rows (16 / W) w .. + 16 / W - 1, CHUNKS pieces each (rows past M: out of range,
  // zeros).
  // Source rows come from uniform (scalar) reads of the gather list, so no vector load joins the vmcnt queue.
  // xoff[j]: byte offset of this wave's row j of the batch whose DMA is issued next (kOOB past M). The gather index
  // is read one batch ahead of its DMA, so the scalar load completes under the previous batch's work instead of
  // delaying the DMA issue.
  int xoff[16 / W];
  auto row_off = [&](int bb, int j) {
    return row_byte_offset((int64_t)bb * 16 + wave * (16 / W) + j, M, row_idx, ldx, x_rows);
  };
  auto dma = [&]() {
#pragma unroll
    for (int j = 0; j < 16 / W; ++j) {
      // (a local copy: with the captured array element as the builtin's operand, hipcc emitted no host stub)
      const int off = xoff[j];
#pragma unroll
      for (int c = 0; c < CHUNKS; ++c)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_x, (lds_void_t*)(xs + (wave * (16 / W) + j) * PITCH + c * 1024), 16,
                                                 off + c * 1024 + lane * 16, 0, 0, 0);
    }
  };

  v4u xv[NS];
  const uint8_t* xrow = xs + r * PITCH + 2 * (k0 + 16 * g);
  // l1t fragments of this wave's slice: lf[h][2 c + e] = l1t[16 h + r][k0 + 64 c + 16 g + 8 e .. + 8]
  // (in l1f: 16-byte piece ((wave * 2 + h) * NS + 2 c + e) * 64 + lane)
  v4u lf[2][NS];
  if (l1f) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < NS; ++i)
        lf[h][i] = *reinterpret_cast<const v4u*>(l1f + ((int64_t)((wave * 2 + h) * NS + i) * 64 + lane) * 8);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < NS; ++i)
        lf[h][i] = *reinterpret_cast<const v4u*>(l1t + (int64_t)(16 * h + r) * K + k0 + 64 * (i >> 1) + 16 * g +
                                                 8 * (i & 1));
  }
  // The l1t loads go out before the first batch's DMA: at small M every workgroup runs a single batch, whose x
  // arrives from HBM later than l1t from L2, so the slice is in registers by the time the batch is (measured at
  // M = 4096, K = 3072: 13.0 -> 11.7 us against issuing the DMA first).
  __builtin_amdgcn_sched_barrier(0);
  int b = blockIdx.x;
#pragma unroll
  for (int j = 0; j < 16 / W; ++j) xoff[j] = row_off(b, j);
  dma();
#pragma unroll
  for (int j = 0; j < 16 / W; ++j) xoff[j] = row_off(b + G, j);
  // One batch. Its DMA was the last memory operation this wave issued before the batch (after the l1t loads, or
  // after the previous batch's stores), so the wait is for everything. The first batch is peeled off the loop (the
  // `first` tag only makes it a separate copy of the code): with every batch in one loop the compiler runs out of
  // the 128 VGPRs of a 16-wave workgroup by one, spills it, and its reload inside the loop waits with vmcnt(0), i.e.
  // also for the next batch's DMA in flight, which takes the c1 pass from 118 to 132 us.
  auto batch = [&](int b, auto first) {
    (void)first;
    wait_vmcnt<0>();
    __syncthreads();   // every wave's DMA of batch b has landed
#pragma unroll
    for (int i = 0; i < NS; ++i) xv[i] = *reinterpret_cast<const v4u*>(xrow + 128 * (i >> 1) + 16 * (i & 1));
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS reads are done
    __syncthreads();                      // every wave's are: the buffer takes the next batch
    dma();   // batch b + G
#pragma unroll
    for (int j = 0; j < 16 / W; ++j) xoff[j] = row_off(b + 2 * G, j);

    const int64_t m = (int64_t)b * 16 + r;
    // absmax: magnitude bits, packed u16 max, then the 4 lanes of the row, then the W slices
    us2 mx2 = {0, 0};
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, xv[i].x & 0x7fff7fffu));
      mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, xv[i].y & 0x7fff7fffu));
      mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, xv[i].z & 0x7fff7fffu));
      mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, xv[i].w & 0x7fff7fffu));
    }
    uint32_t mx = mx2.x > mx2.y ? mx2.x : mx2.y;
#pragma unroll
    for (int off = 16; off <= 32; off <<= 1) {
      const uint32_t o = (uint32_t)__shfl_xor((int)mx, off, 64);
      mx = mx > o ? mx : o;
    }
    if (g == 0) amax_l[wave][r] = mx;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();   // amax_l complete (LDS only: the DMA of the next batch stays in flight)
    __builtin_amdgcn_sched_barrier(0);
    uint32_t am = amax_l[0][r];
#pragma unroll
    for (int w = 1; w < W; ++w) am = am > amax_l[w][r] ? am : amax_l[w][r];
    const float a = fmaxf(lo16_to_f32<DT>(am), 1e-8f);
    const float sc = __fdiv_rn(a, 127.0f);
    const float rc = __fdiv_rn(1.0f, sc);
    // codes: block c of the slice, chunk g of row m (padding rows past M quantize zeros to zero codes)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const v2u lo = quant_chunk<DT>(xv[2 * c], sc, rc);
      const v2u hi = quant_chunk<DT>(xv[2 * c + 1], sc, rc);
      *reinterpret_cast<v4u*>(qp + k64_offset(m, k0 + 64 * c + 16 * g, K / 64)) = v4u{lo.x, lo.y, hi.x, hi.y};
    }
    if (wave == 0 && g == 0 && m < M) s[m] = sc;
    // low rank: partial t over the slice
    v4f acc[2] = {v4f{}, v4f{}};
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (DT == PQ_BF16)
          acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, lf[h][i]),
                                                          __builtin_bit_cast(v8bf, xv[i]), acc[h], 0, 0, 0);
        else
          acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, lf[h][i]),
                                                         __builtin_bit_cast(v8h, xv[i]), acc[h], 0, 0, 0);
      }
    // D[rr][m]: lane holds m = r and rr = 16 h + 4 g + (0..3)
#pragma unroll
    for (int h = 0; h < 2; ++h) *reinterpret_cast<v4f*>(&red[wave][r][16 * h + 4 * g]) = acc[h];
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();   // red complete
    __builtin_amdgcn_sched_barrier(0);
    if (tid < 256) {
      const int mr = tid >> 4, rr = (tid & 15) * 2;
      const int64_t mo = (int64_t)b * 16 + mr;
      float v0 = red[0][mr][rr], v1 = red[0][mr][rr + 1];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        v0 = v0 + red[w][mr][rr];
        v1 = v1 + red[w][mr][rr + 1];
      }
      if (mo < M) *reinterpret_cast<uint32_t*>(t + mo * ldt + rr) = pack2<DT>(v0, v1);
    }
  };
  if (b < nbatch) batch(b, std::true_type{});
  for (b += G; b < nbatch; b += G) batch(b, std::false_type{});
}

// Waves per workgroup of quant_lowrank_kernel for rank R and row length K, or 0 where it does not apply: R == 32
// and K / 256 in {4, 5, 8, 10, 12}; W = 16 when K % 1024 == 0, 8 when K % 512 == 0, else 4.
inline int lowrank_fused_waves(int64_t R, int64_t K) {
  if (R != 32 || K % 256 != 0) return 0;
  const int64_t nc = K / 256;
  if (nc != 4 && nc != 5 && nc != 8 && nc != 10 && nc != 12) return 0;
  return nc % 4 == 0 ? 16 : nc % 2 == 0 ? 8 : 4;
}

// l1t [32, K] -> the fragment order quant_lowrank_kernel loads from l1f (W waves, NS = K / (32 W) loads of 16 bytes
// per lane and half): piece p = ((w * 2 + h) * NS + i) * 64 + l holds l1t[16 h + l % 16][w K / W + 64 (i / 2) +
// 16 (l / 16) + 8 (i % 2) .. + 8]. One thread per 16-byte piece (4 K of them).
__global__ __launch_bounds__(256) void pack_lowrank_l1t_kernel(const v4u* __restrict__ src, int K, int W,
                                                               v4u* __restrict__ dst) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= 4 * K) return;
  const int NS = K / (32 * W);
  const int l = p & 63, rest = p >> 6;
  const int i = rest % NS, wh = rest / NS;
  const int h = wh & 1, w = wh >> 1;
  const int row = 16 * h + (l & 15);
  const int col = w * (K / W) + 64 * (i >> 1) + 16 * (l >> 4) + 8 * (i & 1);
  dst[p] = src[(row * K + col) / 8];
}

// ---- fused quantizer + low-rank down-projection for wide rows (K = 4096 .. 12288, and 15360) ----------------------
// The same results as quant_lowrank_kernel (codes and scales of pq_quant_rows_packed, t = x @ L1 rounded to 16 bits)
// for rows too wide for its LDS staging (c2a: K = 12288, a 16-row batch is 384 KB). x is read from HBM once: a
// re-read of a batch runs at HBM speed even when the memory-side cache holds it, so reading twice costs twice.
// One workgroup of 8 waves per CU, persistent over batches of 8 RPW rows; wave w holds rows RPW w .. RPW w + RPW - 1
// of the batch whole in registers (NCH 16-byte chunks per lane per row, the row-per-wave load pattern of
// quant_rows_vec_kernel). RPW = 2 up to K = 12288 (192 registers of row data per lane); RPW = 1 for K = 15360 (FLUX's
// single-block proj_out, 3072 + 12288: two rows would need 240), whose 8-row batches fill half of the MFMA's 16
// columns (the other half, zeros, is computed and discarded) and half of a 16-row packed block each.
// Per batch: the absmax and scale of each row from the registers (a wave reduction; the IEEE steps of
// quant_rows_vec_kernel); then for each 512-wide K slab e:
//   a. the wave writes its two rows' chunk e into the x slab buffer (16 rows, double buffered);
//   c. quantizes chunk e and stores its codes (packed K64);
//   -- barrier (the x slab is complete, and the L1^T slab e, DMA'd one slab ahead, has landed) --
//   b. issues the LDS-DMA of the L1^T slab e + 1 (32 rows of 1 KB, double buffered);
//   d. reads its 64-wide share of slab e for all 16 rows and the matching L1^T fragments (LDS) and runs
//      v_mfma_f32_16x16x32 into its t partial.
// The 8 waves' t partials are summed in LDS in wave order, (..(p0 + p1) ..) + p7, and rounded to 16 bits.
// Batches are software-pipelined through the registers: after chunk e of batch b is in LDS and quantized, the wave
// loads chunk e of its next batch into the same registers, so the next rows stream in under this batch's work.
// Ordering: the L1^T DMA of slab e + 1 is issued after barrier e, when every wave has read that buffer's previous slab
// (e - 1); it must land before barrier e + 1, and the only vector-memory instructions issued after it are slab e + 1's
// RPW code stores and RPW next-batch loads, hence vmcnt(2 RPW) there (vector-memory instructions retire in issue
// order).
// Past the last batch the next-batch loads read this batch's rows again (discarded), which keeps that count exact.
constexpr int kWideWaves = 8;                 // waves per workgroup, two rows each: batches of 16 rows
constexpr int kWideSlab = 512;                // K elements per slab
constexpr int kWidePitch = 2 * kWideSlab + 16;   // LDS row pitch: consecutive rows 16 bytes apart in the bank window
constexpr int kWideRedPitch = 36;             // floats per row of the partial-sum buffer

template <int DT, int NCH, int RPW>   // NCH = K / 512: 16-byte chunks per lane per row, and slabs; RPW rows per wave
__global__ __launch_bounds__(64 * kWideWaves, 1) void quant_lowrank_wide_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t x_rows, int64_t M, const int32_t* __restrict__ row_idx,
    const uint16_t* __restrict__ l1t, int8_t* __restrict__ qp, float* __restrict__ s, uint16_t* __restrict__ t,
    int64_t ldt, int nbatch, int32_t* __restrict__ zero9) {
  constexpr int K = 512 * NCH;
  // (an older vector store than every load the slab loop counts: the vmcnt waits below only wait for it as well)
  if (zero9 && blockIdx.x == 0 && threadIdx.x < 9) zero9[threadIdx.x] = 0;
  constexpr int KW = kWideSlab / kWideWaves;   // 64: each wave's share of a slab, two MFMA K steps
  constexpr int BR = kWideWaves * RPW;         // rows per batch (16 or 8)
  static_assert(RPW == 1 || RPW == 2, "rows per wave");
  // double buffers as separate arrays, so that the compiler can tell an LDS read of one buffer from a pending
  // LDS-DMA into the other (it waits for every DMA that may alias a read)
  __shared__ __attribute__((aligned(1024))) uint8_t lbuf0[32 * kWidePitch], lbuf1[32 * kWidePitch];   // L1^T slabs
  __shared__ __attribute__((aligned(16))) uint8_t xbuf0[16 * kWidePitch], xbuf1[16 * kWidePitch];     // x slabs
  __shared__ __attribute__((aligned(16))) float red[kWideWaves][16][kWideRedPitch];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // MFMA 16x16x32 operands: lane l feeds A row (L1^T row) and B column (batch row) l % 16, K group l / 16
  const int nr = lane & 15, kg = lane >> 4;
  if constexpr (BR < 16) {
    // x slab rows BR .. 15 feed MFMA columns whose results are discarded: zeros, never written again
    for (int i = tid; i < (16 - BR) * kWidePitch / 16; i += 64 * kWideWaves) {
      reinterpret_cast<v4u*>(xbuf0 + BR * kWidePitch)[i] = v4u{0u, 0u, 0u, 0u};
      reinterpret_cast<v4u*>(xbuf1 + BR * kWidePitch)[i] = v4u{0u, 0u, 0u, 0u};
    }
  }
  const __amdgpu_buffer_rsrc_t rs_l =
      __builtin_amdgcn_make_buffer_rsrc((void*)l1t, (short)0, 32 * K * 2, kBufferWord3);
  // L1^T slab e -> lbuf[e & 1]: wave w copies rows 4 w .. 4 w + 3, one 1 KB LDS-DMA each; the slab's offset rides
  // the scalar offset operand, so the per-lane offsets stay four registers
  const int voff_l = 4 * wave * K * 2 + lane * 16;
  auto dma_l = [&](int e) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_l, (lds_void_t*)((e & 1 ? lbuf1 : lbuf0) + (4 * wave + i) * kWidePitch), 16,
                                               voff_l + i * K * 2, e * kWideSlab * 2, 0, 0);
  };

  // Row rho of this wave in batch bb: its source row in x, or -1 for a padding row past M and a gathered row outside
  // [0, x_rows) (both read as zeros: row 0 is loaded, harmlessly, and the data cleared before use). Wave-uniform:
  // the row bases stay in scalar registers and each lane adds its own 16-byte offset.
  auto src_of = [&](int bb, int rho) -> int64_t {
    const int64_t m = (int64_t)bb * BR + RPW * wave + rho;
    const int64_t src = m >= M ? -1 : (row_idx ? (int64_t)row_idx[m] : m);
    return src >= 0 && src < x_rows ? src : -1;
  };
  auto src_row = [&](int bb, int rho) -> const v4u* {
    const int64_t src = src_of(bb, rho);
    return reinterpret_cast<const v4u*>(x + (src < 0 ? 0 : src) * ldx);
  };
  // this lane's byte offset inside a row's packed K64 codes, for row r' (0 .. 15) of its 16-row block
  auto qlane_of = [&](int rb) {
    return (lane >> 3) * 1024 + ((((lane >> 1) & 3) ^ k64_swz(rb)) << 4) + (lane & 1) * 8;
  };
  v4u v[RPW][NCH];
  // live[rho]: row rho of the batch in hand has a source row (decided when its loads were issued, one batch ahead:
  // recomputing it per batch cost the K = 12288 kernel a spilled register)
  bool live[RPW];
#pragma unroll
  for (int rho = 0; rho < RPW; ++rho) live[rho] = false;
  if ((int)blockIdx.x < nbatch) {
#pragma unroll
    for (int rho = 0; rho < RPW; ++rho) {
      live[rho] = src_of(blockIdx.x, rho) >= 0;
      const v4u* xr = src_row(blockIdx.x, rho);
#pragma unroll
      for (int c = 0; c < NCH; ++c) v[rho][c] = __builtin_nontemporal_load(xr + c * 64 + lane);
    }
  }
  for (int b = blockIdx.x; b < nbatch; b += gridDim.x) {
    const int bn = b + gridDim.x;   // the next batch (past the end: this batch's rows again, loaded and discarded)
    int64_t mrow[RPW];
    const v4u* xn[RPW];
#pragma unroll
    for (int rho = 0; rho < RPW; ++rho) {
      mrow[rho] = (int64_t)b * BR + RPW * wave + rho;
      xn[rho] = src_row(bn < nbatch ? bn : b, rho);
      if (!live[rho]) {   // a padding row or a gathered row outside x: it quantizes as zeros
#pragma unroll
        for (int c = 0; c < NCH; ++c) v[rho][c] = v4u{0u, 0u, 0u, 0u};
      }
      live[rho] = src_of(bn < nbatch ? bn : b, rho) >= 0;   // the batch whose loads xn starts
    }
    dma_l(0);   // lands before slab 0's barrier: only that slab's code stores and next-batch loads come after it
    float sc[RPW], rc[RPW];
#pragma unroll
    for (int rho = 0; rho < RPW; ++rho) {
      us2 mx2 = {0, 0};
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[rho][c].x & 0x7fff7fffu));
        mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[rho][c].y & 0x7fff7fffu));
        mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[rho][c].z & 0x7fff7fffu));
        mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(us2, v[rho][c].w & 0x7fff7fffu));
      }
      const uint32_t mx = wave_max_u32(mx2.x > mx2.y ? mx2.x : mx2.y);
      const float a = fmaxf(absmax_from_bits<DT>(mx), 1e-8f);
      sc[rho] = __fdiv_rn(a, 127.0f);
      rc[rho] = __fdiv_rn(1.0f, sc[rho]);
    }
    // packed K64 rows of the batch: rows b BR .. b BR + BR - 1 are rows (b BR) % 16 .. of block row b BR / 16, this
    // wave's first row is row rb0 = (b BR) % 16 + RPW w of its block (k64_offset, split into the wave-uniform part
    // and qlane)
    const int rb0 = (b * BR) % 16 + RPW * wave;
    int8_t* const qbatch = qp + (int64_t)b * BR / 16 * (K / 64) * 1024 + rb0 * 64;
    int qlane[RPW];
#pragma unroll
    for (int rho = 0; rho < RPW; ++rho) qlane[rho] = qlane_of(rb0 + rho);
    v4f acc[2] = {v4f{}, v4f{}};   // t partial of this wave's K shares: D[r = 16 h + 4 kg + i][batch row nr]
#pragma unroll
    for (int e = 0; e < NCH; ++e) {
      uint8_t* const xs = e & 1 ? xbuf1 : xbuf0;
      const uint8_t* const ls = e & 1 ? lbuf1 : lbuf0;
#pragma unroll
      for (int rho = 0; rho < RPW; ++rho)
        *reinterpret_cast<v4u*>(xs + (RPW * wave + rho) * kWidePitch + lane * 16) = v[rho][e];
      // codes of chunk e (padding rows past M hold zeros and quantize to zero codes): K elements 512 e + 8 lane ..
      // sit 8 packed blocks (8 KB) after those of chunk e - 1
#pragma unroll
      for (int rho = 0; rho < RPW; ++rho)
        *reinterpret_cast<v2u*>(qbatch + rho * 64 + e * 8192 + qlane[rho]) = quant_chunk<DT>(v[rho][e], sc[rho], rc[rho]);
      // chunk e of the next batch into the registers just freed
#pragma unroll
      for (int rho = 0; rho < RPW; ++rho) v[rho][e] = __builtin_nontemporal_load(xn[rho] + e * 64 + lane);
      wait_vmcnt<2 * RPW>();   // this wave's DMA of L1^T slab e has landed (RPW stores, RPW loads after it)
      __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's x slab writes are done
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();         // both slabs complete; every wave is done with slab e - 1
      __builtin_amdgcn_sched_barrier(0);
      if (e + 1 < NCH) dma_l(e + 1);
#pragma unroll
      for (int ks = 0; ks < KW / 32; ++ks) {
        const int kk = wave * KW + ks * 32 + kg * 8;   // K offset inside the slab
        const v4u bf = *reinterpret_cast<const v4u*>(xs + nr * kWidePitch + kk * 2);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const v4u af = *reinterpret_cast<const v4u*>(ls + (16 * h + nr) * kWidePitch + kk * 2);
          if constexpr (DT == PQ_BF16)
            acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, af), __builtin_bit_cast(v8bf, bf),
                                                            acc[h], 0, 0, 0);
          else
            acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, af), __builtin_bit_cast(v8h, bf),
                                                           acc[h], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) *reinterpret_cast<v4f*>(&red[wave][nr][16 * h + 4 * kg]) = acc[h];
    if (lane == 0) {
#pragma unroll
      for (int rho = 0; rho < RPW; ++rho)
        if (mrow[rho] < M) s[mrow[rho]] = sc[rho];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();   // every wave's partials are in red (and every wave is done with the last slabs)
    __builtin_amdgcn_sched_barrier(0);
    if (tid < 16 * BR) {
      const int n = tid >> 4, rr = (tid & 15) * 2;
      const int64_t mo = (int64_t)b * BR + n;
      float v0 = red[0][n][rr], v1 = red[0][n][rr + 1];
#pragma unroll
      for (int w = 1; w < kWideWaves; ++w) {
        v0 = v0 + red[w][n][rr];
        v1 = v1 + red[w][n][rr + 1];
      }
      if (mo < M) *reinterpret_cast<uint32_t*>(t + mo * ldt + rr) = pack2<DT>(v0, v1);
    }
  }
}

// ---- dequant epilogue over a materialised int32 accumulator ----------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void dequant_epilogue_kernel(
    const int32_t* __restrict__ acc, const float* __restrict__ s_row, const float* __restrict__ s_col,
    const float* __restrict__ bias, uint16_t* __restrict__ c, int64_t ldc, int64_t M, int N) {
  const int64_t q4 = (int64_t)blockIdx.x * 256 + threadIdx.x;   // index of a 4-column group
  const int n4 = N >> 2;
  const int64_t m = q4 / n4;
  if (m >= M) return;
  const int n = (int)(q4 - m * n4) * 4;
  const v4i a = *reinterpret_cast<const v4i*>(acc + m * (int64_t)N + n);
  const float sr = s_row[m];
  const v4f sc = *reinterpret_cast<const v4f*>(s_col + n);
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = (float)a[e] * (sr * sc[e]);
  if (bias) {
    const v4f b = *reinterpret_cast<const v4f*>(bias + n);
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = y[e] + b[e];
  }
  *reinterpret_cast<v2u*>(c + m * ldc + n) = v2u{pack2<DT>(y[0], y[1]), pack2<DT>(y[2], y[3])};
}

}  // namespace

// ---- error reporting ---------------------------------------------------------------------------------------
static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_grid(int64_t blocks, int64_t threads, const char* what) {
  if (blocks * threads > 0xffffffffLL)
    return set_error(PQ_ESHAPE, "%s: %lld blocks of %lld threads exceed the 32-bit dispatch size", what,
                     (long long)blocks, (long long)threads);
  return PQ_OK;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(PQ_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PQ_OK;
}

}  // namespace pq

using namespace pq;

extern "C" int pq_abi_version(void) { return PQ_ABI_VERSION; }

extern "C" const char* pq_last_error(void) { return pq::g_err; }

extern "C" int pq_quant_rows(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                             const int32_t* row_idx, int8_t* q, float* s, hipStream_t stream) {
  if (M < 0 || K < 1) return set_error(PQ_ESHAPE, "pq_quant_rows: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  if (M == 0) return PQ_OK;
  if (!x || !q || !s) return set_error(PQ_EINVAL, "pq_quant_rows: null pointer");
  if (ldx < K) return set_error(PQ_ESHAPE, "pq_quant_rows: ldx=%lld < K=%lld", (long long)ldx, (long long)K);
  if (K > (1LL << 30) || M > (1LL << 40)) return set_error(PQ_ESHAPE, "pq_quant_rows: shape too large");
  if (x_rows < 1 || (!row_idx && x_rows < M))
    return set_error(PQ_ESHAPE, "pq_quant_rows: x_rows=%lld must cover the rows read", (long long)x_rows);
  if (x_dtype == PQ_BF16) return launch_quant<PQ_BF16, false>(x, M, K, ldx, x_rows, row_idx, q, s, nullptr, stream);
  if (x_dtype == PQ_F16) return launch_quant<PQ_F16, false>(x, M, K, ldx, x_rows, row_idx, q, s, nullptr, stream);
  return set_error(PQ_EDTYPE, "pq_quant_rows: unsupported dtype code %d", (int)x_dtype);
}

extern "C" int pq_quant_rows_packed(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                                    const int32_t* row_idx, int8_t* qp, float* s, hipStream_t stream) {
  return pq::quant_rows_packed_z(x, x_dtype, M, K, ldx, x_rows, row_idx, qp, s, nullptr, stream);
}

int pq::quant_rows_packed_z(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                            const int32_t* row_idx, int8_t* qp, float* s, int32_t* zero9, hipStream_t stream) {
  if (M < 0 || K < 1) return set_error(PQ_ESHAPE, "pq_quant_rows_packed: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  if (K % 64 != 0) return set_error(PQ_ESHAPE, "pq_quant_rows_packed: K=%lld must be a multiple of 64", (long long)K);
  if (M == 0) return PQ_OK;
  if (!x || !qp || !s) return set_error(PQ_EINVAL, "pq_quant_rows_packed: null pointer");
  if ((uintptr_t)qp % 16) return set_error(PQ_EALIGN, "pq_quant_rows_packed: qp must be 16-byte aligned");
  if (ldx < K) return set_error(PQ_ESHAPE, "pq_quant_rows_packed: ldx=%lld < K=%lld", (long long)ldx, (long long)K);
  if (K > (1LL << 30) || M > (1LL << 40)) return set_error(PQ_ESHAPE, "pq_quant_rows_packed: shape too large");
  if (x_rows < 1 || (!row_idx && x_rows < M))
    return set_error(PQ_ESHAPE, "pq_quant_rows_packed: x_rows=%lld must cover the rows read", (long long)x_rows);
  if (x_dtype == PQ_BF16) return launch_quant<PQ_BF16, true>(x, M, K, ldx, x_rows, row_idx, qp, s, zero9, stream);
  if (x_dtype == PQ_F16) return launch_quant<PQ_F16, true>(x, M, K, ldx, x_rows, row_idx, qp, s, zero9, stream);
  return set_error(PQ_EDTYPE, "pq_quant_rows_packed: unsupported dtype code %d", (int)x_dtype);
}

extern "C" int pq_lowrank_down(const void* x, int32_t dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                               const int32_t* row_idx, const void* l1t, int64_t R, void* t, int64_t ldt,
                               hipStream_t stream) {
  if (M < 0 || K < 1) return set_error(PQ_ESHAPE, "pq_lowrank_down: bad shape");
  if (M == 0) return PQ_OK;
  if (!x || !l1t || !t) return set_error(PQ_EINVAL, "pq_lowrank_down: null pointer");
  if (R < 32 || R > 128 || R % 32 != 0)
    return set_error(PQ_ESHAPE, "pq_lowrank_down: rank R=%lld must be 32, 64, 96 or 128", (long long)R);
  if (K % 8 != 0 || ldx < K || ldx % 8 != 0 || ldt < R || ldt % 8 != 0)
    return set_error(PQ_ESHAPE, "pq_lowrank_down: need K %% 8 == 0, ldx %% 8 == 0, ldt %% 8 == 0");
  if (x_rows < 1 || (!row_idx && x_rows < M))
    return set_error(PQ_ESHAPE, "pq_lowrank_down: x_rows=%lld must cover the rows read", (long long)x_rows);
  if ((uintptr_t)x % 16 || (uintptr_t)l1t % 16 || (uintptr_t)t % 16)
    return set_error(PQ_EALIGN, "pq_lowrank_down: x, l1t, t must be 16-byte aligned");
  if (dtype != PQ_BF16 && dtype != PQ_F16) return set_error(PQ_EDTYPE, "pq_lowrank_down: bad dtype %d", (int)dtype);
  if (const int st = check_grid((M + 127) / 128, 256, "pq_lowrank_down")) return st;
  const dim3 block(256), grid((unsigned)((M + 127) / 128));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* lp = static_cast<const uint16_t*>(l1t);
  uint16_t* tp = static_cast<uint16_t*>(t);
  // LDS-DMA kernel when K streams in whole 64-element stages and every byte offset fits the 32-bit buffer range
  if (K % 64 == 0 && x_rows * ldx * 2 + 128 <= 0x7fffffffLL && R * K * 2 <= 0x7fffffffLL) {
#define PQ_LRDMA(D, RB)                                                                                     \
    if (dtype == D && R == RB * 32) {                                                                       \
      hipLaunchKernelGGL((lowrank_down_dma_kernel<D, RB>), grid, block, 0, stream, xp, ldx, x_rows, (int)K, \
                         M, row_idx, lp, tp, ldt);                                                          \
      return check_launch("lowrank_down");                                                                  \
    }
    PQ_LRDMA(PQ_BF16, 1) PQ_LRDMA(PQ_BF16, 2) PQ_LRDMA(PQ_F16, 1) PQ_LRDMA(PQ_F16, 2)
#undef PQ_LRDMA
  }
#define PQ_LRCASE(D, RB)                                                                                    \
  if (dtype == D && R == RB * 32) {                                                                         \
    hipLaunchKernelGGL((lowrank_down_kernel<D, RB>), grid, block, 0, stream, xp, ldx, (int)K, M, row_idx,  \
                       lp, tp, ldt, x_rows);                                                                \
    return check_launch("lowrank_down");                                                                    \
  }
  PQ_LRCASE(PQ_BF16, 1) PQ_LRCASE(PQ_BF16, 2) PQ_LRCASE(PQ_BF16, 3) PQ_LRCASE(PQ_BF16, 4)
  PQ_LRCASE(PQ_F16, 1) PQ_LRCASE(PQ_F16, 2) PQ_LRCASE(PQ_F16, 3) PQ_LRCASE(PQ_F16, 4)
#undef PQ_LRCASE
  return set_error(PQ_ESHAPE, "pq_lowrank_down: unsupported rank");
}

// Fused per-token quantizer (packed K64 codes) + rank-32 low-rank down-projection: the results of
// pq_quant_rows_packed and pq_lowrank_down on the same x, with x read once where a fused kernel applies (R == 32,
// 16-byte aligned rows, and K in {1024, 1280, 2048, 2560, 3072} with 32-bit x offsets, or K in {4096, 6144, 8192,
// 10240, 12288, 15360}); otherwise the two.
extern "C" int pq_quant_rows_lowrank(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx,
                                     int64_t x_rows, const int32_t* row_idx, const void* l1t, const void* l1f,
                                     int64_t R, int8_t* qp, float* s, void* t, int64_t ldt, hipStream_t stream) {
  return pq::quant_rows_lowrank_z(x, x_dtype, M, K, ldx, x_rows, row_idx, l1t, l1f, R, qp, s, t, ldt, nullptr, stream);
}

int pq::quant_rows_lowrank_z(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                             const int32_t* row_idx, const void* l1t, const void* l1f, int64_t R, int8_t* qp, float* s,
                             void* t, int64_t ldt, int32_t* zero9, hipStream_t stream) {
  if (M < 0 || K < 1) return set_error(PQ_ESHAPE, "pq_quant_rows_lowrank: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  if (M == 0) return PQ_OK;
  if (!x || !qp || !s || !l1t || !t) return set_error(PQ_EINVAL, "pq_quant_rows_lowrank: null pointer");
  if (l1f && (uintptr_t)l1f % 16) return set_error(PQ_EINVAL, "pq_quant_rows_lowrank: l1f must be 16-byte aligned");
  const int nc = (int)(K / 256);
  const bool fused = lowrank_fused_waves(R, K) != 0 && ldx >= K && ldx % 8 == 0 && ldt >= R && ldt % 2 == 0 && x_rows >= 1 &&
                     (row_idx || x_rows >= M) && x_rows * ldx * 2 + 2 * K <= 0x3fffffffLL &&
                     (uintptr_t)x % 16 == 0 && (uintptr_t)l1t % 16 == 0 && (uintptr_t)t % 4 == 0 &&
                     (uintptr_t)qp % 16 == 0 && (x_dtype == PQ_BF16 || x_dtype == PQ_F16);
  // wide rows: one read of x through registers (quant_lowrank_wide_kernel), two rows per wave up to K = 12288, one at
  // K = 15360
  const bool wide = !fused && R == 32 && ((K % 2048 == 0 && K >= 4096 && K <= 12288) || K == 15360) && ldx >= K && ldx % 8 == 0 &&
                    ldt >= R && ldt % 2 == 0 && x_rows >= 1 && (row_idx || x_rows >= M) && (uintptr_t)x % 16 == 0 &&
                    (uintptr_t)l1t % 16 == 0 && (uintptr_t)t % 4 == 0 && (uintptr_t)qp % 16 == 0 &&
                    (x_dtype == PQ_BF16 || x_dtype == PQ_F16);
  if (wide) {
    // batches of 16 rows (two per wave) or 8 (one per wave), covering the packed padding rows up to a multiple of 16
    const int rpw = K <= 12288 ? 2 : 1;
    const int nbatch = (int)((M + 15) / 16) * (2 / rpw);
    const dim3 grid((unsigned)std::min(nbatch, 256));
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const uint16_t* lp = static_cast<const uint16_t*>(l1t);
    uint16_t* tp = static_cast<uint16_t*>(t);
#define PQ_QWCASE(D, NCH, RPW)                                                                                 \
    if (x_dtype == D && K == 512 * NCH) {                                                                      \
      hipLaunchKernelGGL((quant_lowrank_wide_kernel<D, NCH, RPW>), grid, dim3(64 * kWideWaves), 0, stream, xp,    \
                         ldx, x_rows, M, row_idx, lp, qp, s, tp, ldt, nbatch, zero9);                          \
      return check_launch("quant_rows_lowrank");                                                               \
    }
    PQ_QWCASE(PQ_BF16, 8, 2) PQ_QWCASE(PQ_BF16, 12, 2) PQ_QWCASE(PQ_BF16, 16, 2) PQ_QWCASE(PQ_BF16, 20, 2)
    PQ_QWCASE(PQ_BF16, 24, 2) PQ_QWCASE(PQ_BF16, 30, 1)
    PQ_QWCASE(PQ_F16, 8, 2) PQ_QWCASE(PQ_F16, 12, 2) PQ_QWCASE(PQ_F16, 16, 2) PQ_QWCASE(PQ_F16, 20, 2)
    PQ_QWCASE(PQ_F16, 24, 2) PQ_QWCASE(PQ_F16, 30, 1)
#undef PQ_QWCASE
  }
  if (!fused) {
    const int st = pq::quant_rows_packed_z(x, x_dtype, M, K, ldx, x_rows, row_idx, qp, s, zero9, stream);
    if (st != PQ_OK) return st;
    return pq_lowrank_down(x, x_dtype, M, K, ldx, x_rows, row_idx, l1t, R, t, ldt, stream);
  }
  const int nbatch = (int)((M + 15) / 16);
  const dim3 grid((unsigned)std::min(nbatch, 256));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* lp = static_cast<const uint16_t*>(l1t);
  const uint16_t* fp = static_cast<const uint16_t*>(l1f);
  uint16_t* tp = static_cast<uint16_t*>(t);
  // nc = K / 256; W = 16 waves when nc % 4 == 0, 8 when nc % 2 == 0, else 4 (lowrank_fused_waves)
#define PQ_QLCASE(D, NC, W)                                                                                  \
  if (x_dtype == D && nc == NC) {                                                                           \
    hipLaunchKernelGGL((quant_lowrank_kernel<D, NC * 4 / W, W>), grid, dim3(64 * W), 0, stream, xp, ldx, x_rows, \
                       M, row_idx, lp, fp, qp, s, tp, ldt, nbatch, zero9);                                  \
    return check_launch("quant_rows_lowrank");                                                              \
  }
  PQ_QLCASE(PQ_BF16, 4, 16) PQ_QLCASE(PQ_BF16, 5, 4) PQ_QLCASE(PQ_BF16, 8, 16) PQ_QLCASE(PQ_BF16, 10, 8)
  PQ_QLCASE(PQ_BF16, 12, 16)
  PQ_QLCASE(PQ_F16, 4, 16) PQ_QLCASE(PQ_F16, 5, 4) PQ_QLCASE(PQ_F16, 8, 16) PQ_QLCASE(PQ_F16, 10, 8)
  PQ_QLCASE(PQ_F16, 12, 16)
#undef PQ_QLCASE
  return set_error(PQ_ESHAPE, "pq_quant_rows_lowrank: unsupported shape");
}

extern "C" int pq_pack_lowrank_l1t(const void* l1t, int32_t dtype, int64_t R, int64_t K, void* l1f, hipStream_t stream) {
  if (!l1t || !l1f) return set_error(PQ_EINVAL, "pq_pack_lowrank_l1t: null pointer");
  if (dtype != PQ_BF16 && dtype != PQ_F16) return set_error(PQ_EDTYPE, "pq_pack_lowrank_l1t: dtype must be bf16 or fp16");
  const int W = lowrank_fused_waves(R, K);
  if (W == 0)
    return set_error(PQ_ESHAPE, "pq_pack_lowrank_l1t: the fragment order exists for R == 32 and K in {1024, 1280, "
                                "2048, 2560, 3072} only (got R=%lld K=%lld)", (long long)R, (long long)K);
  if ((uintptr_t)l1t % 16 || (uintptr_t)l1f % 16) return set_error(PQ_EINVAL, "pq_pack_lowrank_l1t: 16-byte alignment");
  hipLaunchKernelGGL(pack_lowrank_l1t_kernel, dim3((unsigned)((4 * K + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const v4u*>(l1t), (int)K, W, static_cast<v4u*>(l1f));
  return check_launch("pack_lowrank_l1t");
}

extern "C" int pq_dequant_epilogue(const int32_t* acc, const float* s_row, const float* s_col,
                                   const float* bias, void* c, int64_t ldc, int32_t out_dtype, int64_t M,
                                   int64_t N, hipStream_t stream) {
  if (M < 0 || N < 1) return set_error(PQ_ESHAPE, "pq_dequant_epilogue: bad shape");
  if (M == 0) return PQ_OK;
  if (!acc || !s_row || !s_col || !c) return set_error(PQ_EINVAL, "pq_dequant_epilogue: null pointer");
  if (N % 4 != 0 || ldc < N || ldc % 4 != 0)
    return set_error(PQ_ESHAPE, "pq_dequant_epilogue: need N %% 4 == 0 and ldc %% 4 == 0");
  if ((uintptr_t)acc % 16 || (uintptr_t)s_col % 16 || (uintptr_t)c % 8 || (bias && (uintptr_t)bias % 16))
    return set_error(PQ_EALIGN, "pq_dequant_epilogue: misaligned operand");
  const int64_t groups = M * (N / 4);
  if (const int st = check_grid((groups + 255) / 256, 256, "pq_dequant_epilogue")) return st;
  const dim3 block(256), grid((unsigned)((groups + 255) / 256));
  if (out_dtype == PQ_BF16) {
    hipLaunchKernelGGL((dequant_epilogue_kernel<PQ_BF16>), grid, block, 0, stream, acc, s_row, s_col, bias,
                       static_cast<uint16_t*>(c), ldc, M, (int)N);
  } else if (out_dtype == PQ_F16) {
    hipLaunchKernelGGL((dequant_epilogue_kernel<PQ_F16>), grid, block, 0, stream, acc, s_row, s_col, bias,
                       static_cast<uint16_t*>(c), ldc, M, (int)N);
  } else {
    return set_error(PQ_EDTYPE, "pq_dequant_epilogue: bad dtype %d", (int)out_dtype);
  }
  return check_launch("dequant_epilogue");
}

extern "C" int pq_quant_weight(const float* w, int64_t N, int64_t K, int64_t ldw, int64_t group, int8_t* q, float* s,
                               hipStream_t stream) {
  if (N < 0 || K < 1) return set_error(PQ_ESHAPE, "pq_quant_weight: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  if (N == 0) return PQ_OK;
  if (!w || !q || !s) return set_error(PQ_EINVAL, "pq_quant_weight: null pointer");
  if (ldw < K) return set_error(PQ_ESHAPE, "pq_quant_weight: ldw < K");
  if (group < 0 || (group > 0 && K % group != 0))
    return set_error(PQ_ESHAPE, "pq_quant_weight: group %lld must divide K=%lld", (long long)group, (long long)K);
  if (K > (1LL << 30) || N > (1LL << 30)) return set_error(PQ_ESHAPE, "pq_quant_weight: shape too large");
  const int g = group ? (int)group : (int)K;
  const int64_t segs = N * (K / g);
  if (const int st = check_grid((segs + 3) / 4, 256, "pq_quant_weight")) return st;
  hipLaunchKernelGGL(quant_weight_kernel, dim3((unsigned)((segs + 3) / 4)), dim3(256), 0, stream, w, ldw, (int)N,
                     (int)K, g, q, s);
  return check_launch("quant_weight");
}

extern "C" int pq_pack_k64(const int8_t* src, int64_t R, int64_t K, int64_t lds, int8_t* dst, hipStream_t stream) {
  if (R < 0 || K < 1 || K % 64 != 0) return set_error(PQ_ESHAPE, "pq_pack_k64: need R >= 0 and K %% 64 == 0 (K=%lld)", (long long)K);
  if (R == 0) return PQ_OK;
  if (!src || !dst) return set_error(PQ_EINVAL, "pq_pack_k64: null pointer");
  if (lds < K || lds % 16 || (uintptr_t)src % 16 || (uintptr_t)dst % 16)
    return set_error(PQ_EALIGN, "pq_pack_k64: src / dst 16-byte aligned, lds %% 16 == 0 and lds >= K required");
  const int64_t nslots = ((R + 15) / 16) * (K / 64) * 64;
  if (const int st = check_grid((nslots + 255) / 256, 256, "pq_pack_k64")) return st;
  hipLaunchKernelGGL(pack_k64_kernel, dim3((unsigned)((nslots + 255) / 256)), dim3(256), 0, stream, src, R,
                     (int)(K / 64), lds, dst, nslots);
  return check_launch("pack_k64");
}
