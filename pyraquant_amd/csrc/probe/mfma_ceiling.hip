// Register-only MFMA throughput probe for gfx950 (measurement only; not part of libpqint8.so's ABI).
//
// Each wave holds 8 A and 8 B operand fragments in VGPRs and issues MFMAs back to back over 4 independent
// accumulators, cycling through the fragments so that consecutive instructions see different operands (as the
// GEMM's do, each fragment being a fresh LDS read there). No memory traffic inside the loop. The operand bytes come
// from a host-filled buffer, so the same kernel measures random operands against constant or zero ones: the MFMA's
// power, and so the clock the chip sustains, depends on how many operand bits toggle.
//
//   kind 0: v_mfma_i32_32x32x32_i8   (65536 int8 ops per instruction)
//   kind 1: v_mfma_f32_32x32x16_f16  (32768 flops per instruction; operands are the fp16 images of int8 codes)
//   kind 2: kind 0 in workgroups of 8 waves (two per SIMD), all at the default issue priority
//   kind 3: kind 2 with waves 0-3 raised to issue priority 1 (s_setprio) for the whole kernel: on each SIMD the
//           high-priority wave issues its MFMAs back to back and the other wave issues only when it stalls
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

template <int KIND>
__global__ __launch_bounds__(512) void mfma_ceiling_kernel(const v4i* __restrict__ src, int iters,
                                                           int* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  if constexpr (KIND == 3) {
    if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < 4) __builtin_amdgcn_s_setprio(1);
  }
  v4i a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = src[i * 64 + lane];
    b[i] = src[(8 + i) * 64 + lane];
  }
  if constexpr (KIND != 1) {
    v16i acc[4] = {v16i{}, v16i{}, v16i{}, v16i{}};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[(5 * i + 3) & 7], acc[i & 3], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s ^= acc[j][r];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
  } else {
    v16f acc[4] = {v16f{}, v16f{}, v16f{}, v16f{}};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[i]),
                                                            __builtin_bit_cast(v8h, b[(5 * i + 3) & 7]), acc[i & 3], 0,
                                                            0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[j][r];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = __float_as_int(s);
  }
}

}  // namespace

// Runs the probe once: `blocks` workgroups of 4 waves (8 for kinds 2 and 3), `iters` x 8 MFMAs per wave, operands from `src` (16 x 64
// fragments of 16 bytes). Returns 0 or a HIP error code; the kernel time is left to the caller's events.
extern "C" int pq_probe_mfma(int kind, const void* src, int blocks, int iters, int* sink, hipStream_t stream) {
  if (blocks < 1 || iters < 1 || !src || !sink) return -1;
  if (kind == 0) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<0>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 1) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<1>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 2) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<2>, dim3(blocks), dim3(512), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 3) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<3>, dim3(blocks), dim3(512), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else {
    return -1;
  }
  return (int)hipGetLastError();
}
