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
//   kind 4: the group-32 inner loop on int8 MFMAs: per 32-wide K group and 32 x 32 tile, one
//           v_mfma_i32_32x32x32_i8 from zero, then acc = fma(scale, (float)partial, acc) on the 16 values per lane
//   kind 5: the same group on fp16 MFMAs: two v_mfma_f32_32x32x16_f16 (the partial arrives in fp32, exact for
//           int8 codes), then the 16 fmas; kinds 4 and 5 count 65536 int8-equivalent ops per group and tile
//   kinds 6, 7: kinds 4, 5 in workgroups of 8 waves with waves 0-3 at issue priority 1, as kind 3
//   kinds 8, 9: kinds 5, 4 software-pipelined: the partial of the tile two steps ahead is computed into its own
//           register set while the fmas consume the current one, and fences fix the order (one MFMA, then a share
//           of the fmas), so the wave's VALU work can run under its own MFMAs
//   kind 10: kind 9 with the convert replaced by an exact float subtraction: the MFMA starts from the integer
//           0x4B400000 (the bits of 1.5 * 2^23), so for a partial |p| < 2^22 the result reinterpreted as a float is
//           1.5 * 2^23 + p exactly, and subtracting 1.5 * 2^23 gives (float)p bit for bit
//   kind 11: kind 9 without the convert (the fma takes the partial's bits as a float): the fma-only cost, a timing
//           reference whose sums mean nothing
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

template <int KIND>
__global__ __launch_bounds__(512) void mfma_ceiling_kernel(const v4i* __restrict__ src, int iters,
                                                           int* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  if constexpr (KIND == 3 || KIND == 6 || KIND == 7) {
    if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) < 4) __builtin_amdgcn_s_setprio(1);
  }
  v4i a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = src[i * 64 + lane];
    b[i] = src[(8 + i) * 64 + lane];
  }
  if constexpr (KIND >= 8) {
    constexpr bool I8 = KIND != 8;
    // kind 10: the partial's accumulator starts at the bits of 1.5 * 2^23 (see the kind list)
    const v16i c0 = KIND == 10 ? v16i{} + 0x4B400000 : v16i{};
    using part_t = typename std::conditional<I8, v16i, v16f>::type;
    float sc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) sc[i] = 1.0f + 1e-3f * (float)((lane + i) & 7);
    v16f acc[4] = {v16f{}, v16f{}, v16f{}, v16f{}};
    // Step j handles tile-group idx = j (idx = 4 g + t: K group g of 2, tile t of 2 x 2). Four partial buffers:
    // step j issues the MFMA(s) of step j + 2 and runs the fmas of step j, whose partial was issued two steps
    // earlier, so the fmas never wait on the MFMA in flight. Hard scheduling fences fix the order MFMA, half the
    // fmas, [second fp16 MFMA, other half].
    auto first = [&](int idx) -> part_t {
      const int g = idx >> 2, t = idx & 3;
      if constexpr (I8) return __builtin_amdgcn_mfma_i32_32x32x32_i8(a[2 * g + (t >> 1)], b[4 * g + (t & 1)], c0, 0, 0, 0);
      else return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[4 * g + (t >> 1)]),
                                                         __builtin_bit_cast(v8h, b[4 * g + (t & 1)]), v16f{}, 0, 0, 0);
    };
    auto second = [&](int idx, part_t p) -> part_t {
      const int g = idx >> 2, t = idx & 3;
      if constexpr (I8) return p;
      else return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[4 * g + 2 + (t >> 1)]),
                                                         __builtin_bit_cast(v8h, b[4 * g + 2 + (t & 1)]), p, 0, 0, 0);
    };
    part_t p[4];
    p[0] = second(0, first(0));
    p[1] = second(1, first(1));
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int idx = j, ahead = (j + 2) & 7;
        const float sg = sc[idx];
        v16f& ac = acc[idx & 3];
        part_t& cur = p[j & 3];
        part_t& nxt = p[(j + 2) & 3];
        nxt = first(ahead);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (KIND == 10) {
#pragma unroll
          for (int r = 0; r < 16; ++r) ac[r] = __builtin_fmaf(sg, __int_as_float(cur[r]) - 12582912.0f, ac[r]);
          __builtin_amdgcn_sched_barrier(0);
        } else if constexpr (KIND == 11) {
#pragma unroll
          for (int r = 0; r < 16; ++r) ac[r] = __builtin_fmaf(sg, __int_as_float(cur[r]), ac[r]);
          __builtin_amdgcn_sched_barrier(0);
        } else if constexpr (I8) {
#pragma unroll
          for (int r = 0; r < 16; ++r) ac[r] = __builtin_fmaf(sg, (float)cur[r], ac[r]);
          __builtin_amdgcn_sched_barrier(0);
        } else {
#pragma unroll
          for (int r = 0; r < 8; ++r) ac[r] = __builtin_fmaf(sg, cur[r], ac[r]);
          __builtin_amdgcn_sched_barrier(0);
          nxt = second(ahead, nxt);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int r = 8; r < 16; ++r) ac[r] = __builtin_fmaf(sg, cur[r], ac[r]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    part_t cur = p[0] + p[1];
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += (float)cur[r];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[j][r];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = __float_as_int(s);
  } else if constexpr (KIND == 4 || KIND == 5 || KIND == 6 || KIND == 7) {
    constexpr bool I8 = KIND == 4 || KIND == 6;
    // 2 x 2 tiles of fp32 accumulators; the group scales rotate through 8 registers per lane
    float sc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) sc[i] = 1.0f + 1e-3f * (float)((lane + i) & 7);
    v16f acc[4] = {v16f{}, v16f{}, v16f{}, v16f{}};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float sg = sc[(4 * g + t) & 7];
          if constexpr (I8) {
            const v16i part = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[2 * g + (t >> 1)], b[4 * g + (t & 1)], v16i{}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(sg, (float)part[r], acc[t][r]);
          } else {
            v16f part = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[4 * g + (t >> 1)]),
                                                               __builtin_bit_cast(v8h, b[4 * g + (t & 1)]), v16f{}, 0, 0, 0);
            part = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a[4 * g + 2 + (t >> 1)]),
                                                          __builtin_bit_cast(v8h, b[4 * g + 2 + (t & 1)]), part, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(sg, part[r], acc[t][r]);
          }
        }
      }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += acc[j][r];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = __float_as_int(s);
  } else if constexpr (KIND != 1) {
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

// Streaming read of `n16` 16-byte chunks, grid-stride, plain (NT = 0) or non-temporal (NT = 1) loads; the XOR of
// everything read goes to sink so the loads stay.
template <int NT>
__global__ __launch_bounds__(256) void read_probe_kernel(const v4i* __restrict__ src, int64_t n16,
                                                         int* __restrict__ sink) {
  v4i x = v4i{0, 0, 0, 0};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += 4 * stride) {
    v4i v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = i + u * stride;
      if (j < n16) v[u] = NT ? __builtin_nontemporal_load(src + j) : src[j];
      else v[u] = v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) x ^= v[u];
  }
  sink[blockIdx.x * blockDim.x + threadIdx.x] = x.x ^ x.y ^ x.z ^ x.w;
}

}  // namespace

// Streaming read of `bytes` (a multiple of 16) from src over `blocks` workgroups of 256 threads (sink: blocks * 256
// ints), plain or non-temporal loads: how fast a buffer of a given size is read back, HBM or memory-side cache.
extern "C" int pq_probe_read(const void* src, int64_t bytes, int nt, int blocks, int* sink, hipStream_t stream) {
  if (!src || !sink || bytes < 16 || bytes % 16 || blocks < 1) return -1;
  if (nt) hipLaunchKernelGGL(read_probe_kernel<1>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                             bytes / 16, sink);
  else hipLaunchKernelGGL(read_probe_kernel<0>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                          bytes / 16, sink);
  return (int)hipGetLastError();
}

// Runs the probe once: `blocks` workgroups of 4 waves (8 for kinds 2, 3, 6 and 7), `iters` x 8 MFMAs per wave, operands from `src` (16 x 64
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
  } else if (kind == 4) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<4>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 5) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<5>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 6) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<6>, dim3(blocks), dim3(512), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 7) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<7>, dim3(blocks), dim3(512), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 8) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<8>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 9) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<9>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 10) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<10>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else if (kind == 11) {
    hipLaunchKernelGGL(mfma_ceiling_kernel<11>, dim3(blocks), dim3(256), 0, stream, static_cast<const v4i*>(src),
                       iters, sink);
  } else {
    return -1;
  }
  return (int)hipGetLastError();
}
