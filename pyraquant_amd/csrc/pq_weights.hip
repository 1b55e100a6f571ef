// Weight-side conversion of an SVDQuant package on the device, for gfx950: the smoothing / shift fold of
// `_fold_one` (deploy/run_flux_latency.py:210-250), one pass over the 16-bit weight.
//
// For a Linear y = QDQ((x + shift) / smooth) @ W^T + b, the package stores W, smooth and shift; the fold is
//   Wf      = float(W) / smooth               (IEEE fp32 division; smooth is one scalar or one value per input)
//   add[n]  = sum_k Wf[n, k] * shift[k]        (per-input shift; fp32)   or   (sum_k Wf[n, k]) * shift (scalar)
//   W      <- Wf rounded to W's 16-bit type     (lin.weight.data.copy_(Wf.to(dt)))
//   b      <- b + add, both rounded to the bias' 16-bit type first (lin.bias.data.add_(add.to(b.dtype))), or
//             b = add rounded when the Linear has no bias.
// The INT8 codes are then derived from the folded 16-bit weight as for any Linear (pq_quant_weight).
// One workgroup per output row: every thread walks a strided slice of the row, writes the folded values in place or
// to a second buffer, and the fp32 partial sums of the shift term are reduced across the workgroup.
#include "pq_common.h"

namespace pq {
namespace {

template <int DT>
__device__ __forceinline__ float load16(const uint16_t* p) {
  return lo16_to_f32<DT>((uint32_t)*p);
}

template <int DT>
__device__ __forceinline__ float round16f(float v) {
  return lo16_to_f32<DT>(f32_to_16_bits<DT>(v));
}

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void fold_weight_kernel(const uint16_t* __restrict__ w, int64_t ldw, int K,
                                                          const float* __restrict__ smooth, int n_smooth,
                                                          const float* __restrict__ shift, int n_shift,
                                                          const uint16_t* __restrict__ bias_in,
                                                          uint16_t* __restrict__ w_out, int64_t ldo,
                                                          uint16_t* __restrict__ bias_out) {
  __shared__ float red[4];
  const int64_t n = blockIdx.x;
  const uint16_t* __restrict__ wr = w + n * ldw;
  uint16_t* __restrict__ orow = w_out + n * ldo;
  const float s0 = smooth && n_smooth == 1 ? smooth[0] : 1.0f;
  float part = 0.0f;
  if constexpr (VEC) {   // 8 elements per thread and step: 16-byte weight loads / stores, 32-byte smooth / shift
    const float h0 = shift && n_shift == 1 ? 1.0f : 0.0f;
    for (int c = threadIdx.x; c < K / 8; c += blockDim.x) {
      const v4u v = *reinterpret_cast<const v4u*>(wr + 8 * c);
      const uint32_t in[4] = {v.x, v.y, v.z, v.w};
      float sm[8], sh[8];
      if (smooth && n_smooth != 1) {
        const v4f a = *reinterpret_cast<const v4f*>(smooth + 8 * c), b = *reinterpret_cast<const v4f*>(smooth + 8 * c + 4);
        sm[0] = a.x; sm[1] = a.y; sm[2] = a.z; sm[3] = a.w; sm[4] = b.x; sm[5] = b.y; sm[6] = b.z; sm[7] = b.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) sm[e] = s0;
      }
      if (shift && n_shift != 1) {
        const v4f a = *reinterpret_cast<const v4f*>(shift + 8 * c), b = *reinterpret_cast<const v4f*>(shift + 8 * c + 4);
        sh[0] = a.x; sh[1] = a.y; sh[2] = a.z; sh[3] = a.w; sh[4] = b.x; sh[5] = b.y; sh[6] = b.z; sh[7] = b.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) sh[e] = h0;
      }
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float w0 = lo16_to_f32<DT>(in[e]), w1 = hi16_to_f32<DT>(in[e]);
        if (smooth) {
          w0 = w0 / sm[2 * e];
          w1 = w1 / sm[2 * e + 1];
        }
        o[e] = f32_to_16_bits<DT>(w0) | (f32_to_16_bits<DT>(w1) << 16);
        if (shift) {
          part += n_shift == 1 ? w0 : w0 * sh[2 * e];
          part += n_shift == 1 ? w1 : w1 * sh[2 * e + 1];
        }
      }
      *reinterpret_cast<v4u*>(orow + 8 * c) = v4u{o[0], o[1], o[2], o[3]};
    }
  } else {
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
      float wf = load16<DT>(wr + k);
      if (smooth) wf = wf / (n_smooth == 1 ? s0 : smooth[k]);
      orow[k] = (uint16_t)f32_to_16_bits<DT>(wf);
      if (shift) part += n_shift == 1 ? wf : wf * shift[k];
    }
  }
  if (!shift && !bias_out) return;
  // workgroup sum of the partials (fp32; the order differs from torch's matmul, so the sum agrees to rounding)
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = part;
  __syncthreads();
  if (threadIdx.x == 0 && bias_out) {
    float add = 0.0f;
    if (shift) {
      add = ((red[0] + red[1]) + red[2]) + red[3];
      if (n_shift == 1) add = add * shift[0];
    }
    const float add16 = round16f<DT>(add);
    const float b = bias_in ? round16f<DT>(load16<DT>(bias_in + n) + add16) : add16;
    bias_out[n] = (uint16_t)f32_to_16_bits<DT>(b);
  }
}

}  // namespace
}  // namespace pq

using namespace pq;

extern "C" int pq_fold_weight(const void* w, int32_t dtype, int64_t N, int64_t K, int64_t ldw, const float* smooth,
                              int64_t n_smooth, const float* shift, int64_t n_shift, const void* bias_in,
                              void* w_out, int64_t ldo, void* bias_out, hipStream_t stream) {
  if (N < 0 || K < 1 || ldw < K || ldo < K || N > 0x7fffffff || K > 0x7fffffff)
    return set_error(PQ_ESHAPE, "pq_fold_weight: bad shape N=%lld K=%lld ldw=%lld ldo=%lld", (long long)N,
                     (long long)K, (long long)ldw, (long long)ldo);
  if (N == 0) return PQ_OK;
  if (!w || !w_out) return set_error(PQ_EINVAL, "pq_fold_weight: null weight pointer");
  if (smooth && n_smooth != 1 && n_smooth != K)
    return set_error(PQ_ESHAPE, "pq_fold_weight: smooth length %lld is neither 1 nor in_features %lld",
                     (long long)n_smooth, (long long)K);
  if (shift && n_shift != 1 && n_shift != K)
    return set_error(PQ_ESHAPE, "pq_fold_weight: shift length %lld is neither 1 nor in_features %lld",
                     (long long)n_shift, (long long)K);
  if (shift && !bias_out) return set_error(PQ_EINVAL, "pq_fold_weight: a shift needs bias_out");
  if ((uintptr_t)w % 2 || (uintptr_t)w_out % 2 || (bias_in && (uintptr_t)bias_in % 2) ||
      (bias_out && (uintptr_t)bias_out % 2) || (smooth && (uintptr_t)smooth % 4) || (shift && (uintptr_t)shift % 4))
    return set_error(PQ_EALIGN, "pq_fold_weight: misaligned operand");
  if (dtype != PQ_BF16 && dtype != PQ_F16) return set_error(PQ_EDTYPE, "pq_fold_weight: dtype %d", dtype);
  if (const int st = check_grid(N, 256, "pq_fold_weight")) return st;
  const dim3 grid((unsigned)N), block(256);
  const bool vec = K % 8 == 0 && ldw % 8 == 0 && ldo % 8 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)w_out % 16 == 0 &&
                   (!smooth || n_smooth == 1 || (uintptr_t)smooth % 16 == 0) &&
                   (!shift || n_shift == 1 || (uintptr_t)shift % 16 == 0);
#define PQ_FOLD(D, V)                                                                                                \
  hipLaunchKernelGGL((fold_weight_kernel<D, V>), grid, block, 0, stream, (const uint16_t*)w, ldw, (int)K, smooth,   \
                     (int)n_smooth, shift, (int)n_shift, (const uint16_t*)bias_in, (uint16_t*)w_out, ldo,            \
                     (uint16_t*)bias_out)
  if (dtype == PQ_BF16) {
    if (vec) PQ_FOLD(PQ_BF16, true); else PQ_FOLD(PQ_BF16, false);
  } else {
    if (vec) PQ_FOLD(PQ_F16, true); else PQ_FOLD(PQ_F16, false);
  }
#undef PQ_FOLD
  return check_launch("fold_weight");
}
