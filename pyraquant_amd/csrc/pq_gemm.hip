// Fused INT8 GEMM + dequant / low-rank / bias epilogue (+ routed row scatter) for gfx950.
//
// Math (reference: deploy/int8_exec.py:144-183 and :272-314, epilogue order :303-309):
//   per-channel: y[m,n] = (float)(sum_k a[m,k] w[n,k]) * (s_row[m] * s_w[n])
//   group-32   : y[m,n] = s_row[m] * sum_g s_w[g,n] * (float)(sum_{k in g} a[m,k] w[n,k])   (fma over g)
//   then y += sum_r t[m,r] l2t[n,r] (low-rank up-projection), y += bias[n], rounded to bf16/fp16.
//
// Kernel structure. The MFMA computes D = W_tile * A_tile^T: its row operand ("i") is a weight row n and
// its column operand ("j") an activation row m, so each lane ends up holding 4 consecutive n of one
// output row m (8-byte bf16 stores) and one s_row value per tile. A workgroup owns a BN x BM output block
// (n x m), split over a WN x WM grid of wavefronts; each wave holds TI x TJ MFMA tiles of
// v_mfma_i32_32x32x32_i8 (int32 accumulators, kept in AGPRs). K advances in steps of 64 bytes through an
// LDS double buffer fed from registers; the 16-byte chunks of every 64-byte LDS row are XOR-swizzled
// with row bits 1..2 so that the ds_read_b128 of 8 consecutive rows hit 8 different bank groups.
// Workgroup ids are remapped so that each XCD (ids are dealt round-robin over the 8 XCDs) walks a
// contiguous run of tiles, rasterised in groups of GROUP_M m-tiles for L2 reuse.
#include "pq_common.h"

#include <type_traits>

namespace pq {
namespace {

constexpr int kBK = 64;        // K bytes per pipeline stage
constexpr int kGroupM = 8;     // m-tiles per raster group
constexpr int kBufferWord3 = 0x00020000;   // gfx9 buffer descriptor word 3 (raw, 32-bit data format)

struct GemmArgs {
  const int8_t* a;
  const int8_t* w;
  const float* s_row;
  const float* s_w;
  const float* bias;
  const uint16_t* t;
  const uint16_t* l2t;
  void* c;
  const int32_t* out_row_idx;
  int64_t lda, ldw, ldt, ldc;
  int M, N, K, R;
  int tiles_m, tiles_n;
};

enum { kModeI32 = 0, kModeChannel = 1, kModeGroup32 = 2 };

// Map the linear workgroup id to (tile_m, tile_n): XCD-contiguous, then GROUP_M raster.
__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per = nblocks >> 3, rem = nblocks & 7;
  const int xcd = bid & 7, local = bid >> 3;
  const int logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
  const int in_group = kGroupM * tiles_n;
  const int group = logical / in_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int r = logical - group * in_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

template <int LRDT>
__device__ __forceinline__ v16f lr_mfma(v4i a, v4i b, v16f c) {
  if constexpr (LRDT == PQ_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  }
}

// Byte offset of 16-byte chunk `chunk` of LDS row `row` (rows of 64 bytes, swizzled).
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ ((row >> 1) & 3)) << 4); }

template <int WN, int WM, int TI, int TJ, int MODE, bool HAS_LR, int LRDT, int ODT>
__global__ __attribute__((amdgpu_flat_work_group_size(WN * WM * 64, WN * WM * 64)))
void gemm_kernel(const GemmArgs p) {
  constexpr int NT = WN * WM * 64;
  constexpr int BN = WN * TI * 32;
  constexpr int BM = WM * TJ * 32;
  constexpr int CW = BN * kBK / 16 / NT;   // 16-byte chunks of W per thread per stage
  constexpr int CA = BM * kBK / 16 / NT;   // 16-byte chunks of A per thread per stage
  static_assert(CW * NT * 16 == BN * kBK && CA * NT * 16 == BM * kBK, "tile / thread mismatch");
  constexpr int ROWS_PER_PASS = NT / 4;    // 4 chunks per 64-byte row

  __shared__ __attribute__((aligned(16))) uint8_t smem[2][(BN + BM) * kBK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave % WN;
  const int wm = wave / WN;

  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;

  // ---- global -> register loaders. Buffer resources based at the block's first row: rows past M / N
  //      are outside num_records and load as zeros. Thread owns chunk (tid % 4) of rows
  //      tid / 4 + ROWS_PER_PASS * i; the per-i and per-stage offsets are wave-uniform (SGPR).
  const int lrow = tid >> 2;
  const int lchunk = tid & 3;
  const int rows_w = min(BN, p.N - n0), rows_a = min(BM, p.M - m0);
  const __amdgpu_buffer_rsrc_t rs_w = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.w + (int64_t)n0 * p.ldw), (short)0, (int)(rows_w * p.ldw), kBufferWord3);
  const __amdgpu_buffer_rsrc_t rs_a = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.a + (int64_t)m0 * p.lda), (short)0, (int)(rows_a * p.lda), kBufferWord3);
  const int vo_w = lrow * (int)p.ldw + lchunk * 16;
  const int vo_a = lrow * (int)p.lda + lchunk * 16;
  const int pass_w = ROWS_PER_PASS * (int)p.ldw;
  const int pass_a = ROWS_PER_PASS * (int)p.lda;
  const int st_off = lds_off(lrow, lchunk);   // + i * ROWS_PER_PASS * kBK (row bits 1..2 unchanged)
  static_assert((ROWS_PER_PASS & 7) == 0, "rows per pass must keep the swizzle bits");

  // ---- MFMA operand offsets in LDS
  const int rsub = lane & 31;
  const int khalf = lane >> 5;

  using acc_t = typename std::conditional<MODE == kModeGroup32, v16f, v16i>::type;
  acc_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = acc_t{};

  v4i rw[CW], ra[CA];
#pragma unroll
  for (int i = 0; i < CW; ++i) rw[i] = __builtin_amdgcn_raw_buffer_load_b128(rs_w, vo_w, i * pass_w, 0);
#pragma unroll
  for (int i = 0; i < CA; ++i) ra[i] = __builtin_amdgcn_raw_buffer_load_b128(rs_a, vo_a, i * pass_a, 0);
  {
    uint8_t* sw = smem[0];
    uint8_t* sa = smem[0] + BN * kBK;
#pragma unroll
    for (int i = 0; i < CW; ++i) *reinterpret_cast<v4i*>(sw + st_off + i * ROWS_PER_PASS * kBK) = rw[i];
#pragma unroll
    for (int i = 0; i < CA; ++i) *reinterpret_cast<v4i*>(sa + st_off + i * ROWS_PER_PASS * kBK) = ra[i];
  }
  __syncthreads();

  const int KT = p.K / kBK;
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      const int ko = (kt + 1) * kBK;
#pragma unroll
      for (int i = 0; i < CW; ++i) rw[i] = __builtin_amdgcn_raw_buffer_load_b128(rs_w, vo_w, ko + i * pass_w, 0);
#pragma unroll
      for (int i = 0; i < CA; ++i) ra[i] = __builtin_amdgcn_raw_buffer_load_b128(rs_a, vo_a, ko + i * pass_a, 0);
    }
    const uint8_t* sw = smem[buf];
    const uint8_t* sa = smem[buf] + BN * kBK;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      v4i fw[TI], fa[TJ];
      const int chunk = kk * 2 + khalf;
#pragma unroll
      for (int i = 0; i < TI; ++i)
        fw[i] = *reinterpret_cast<const v4i*>(sw + lds_off(wn * TI * 32 + i * 32 + rsub, chunk));
#pragma unroll
      for (int j = 0; j < TJ; ++j)
        fa[j] = *reinterpret_cast<const v4i*>(sa + lds_off(wm * TJ * 32 + j * 32 + rsub, chunk));
      if constexpr (MODE == kModeGroup32) {
        // one 32-wide K group per MFMA: int32 partial -> fp32, fma with the group scale of each row n
        const int g = kt * 2 + kk;
        const float* sg = p.s_w + (int64_t)g * p.N;
#pragma unroll
        for (int i = 0; i < TI; ++i) {
          const int nb = n0 + wn * TI * 32 + i * 32 + 4 * khalf;
          v4f s4[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n = min(nb + 8 * q, p.N - 4);
            s4[q] = *reinterpret_cast<const v4f*>(sg + n);
          }
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            const v16i part = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[i], fa[j], v16i{}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float sc = s4[r >> 2][r & 3];
              acc[i][j][r] = __builtin_fmaf(sc, (float)part[r], acc[i][j][r]);
            }
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[i], fa[j], acc[i][j], 0, 0, 0);
      }
    }
    if (more) {
      uint8_t* nw = smem[buf ^ 1];
      uint8_t* na = smem[buf ^ 1] + BN * kBK;
#pragma unroll
      for (int i = 0; i < CW; ++i) *reinterpret_cast<v4i*>(nw + st_off + i * ROWS_PER_PASS * kBK) = rw[i];
#pragma unroll
      for (int i = 0; i < CA; ++i) *reinterpret_cast<v4i*>(na + st_off + i * ROWS_PER_PASS * kBK) = ra[i];
    }
    __syncthreads();
  }

  // ---- epilogue. Lane holds, for tile (i, j) and register r: m = j-tile row (lane % 32),
  //      n = 8 * (r / 4) + 4 * (lane / 32) + r % 4 within the 32-row weight tile.
  //      Loop order: weight tile outer (its scales / bias / low-rank rows loaded once), rows inner.
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    const int ntile = n0 + wn * TI * 32 + i * 32;
    if (ntile >= p.N) continue;   // N % 32 == 0: a weight tile is entirely in or out of range
    const int nb = ntile + 4 * khalf;
    v4f sc[4], bi[4];
    v4i lb[HAS_LR ? 4 : 1];
    if constexpr (MODE != kModeI32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sc[q] = MODE == kModeChannel ? *reinterpret_cast<const v4f*>(p.s_w + nb + 8 * q) : v4f{};
        bi[q] = p.bias ? *reinterpret_cast<const v4f*>(p.bias + nb + 8 * q) : v4f{};
      }
      if constexpr (HAS_LR) {
        const uint16_t* lrow = p.l2t + (int64_t)(ntile + rsub) * p.R + khalf * 8;
#pragma unroll
        for (int rs = 0; rs < 4; ++rs) lb[rs] = rs * 16 < p.R ? *reinterpret_cast<const v4i*>(lrow + rs * 16) : v4i{};
      }
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int m = m0 + wm * TJ * 32 + j * 32 + rsub;
      const int mc = min(m, p.M - 1);
      const bool mvalid = m < p.M;
      if constexpr (MODE == kModeI32) {
        if (mvalid) {
          int32_t* crow = static_cast<int32_t*>(p.c) + (int64_t)m * p.ldc;
          const v16i& v = acc[i][j];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<v4i*>(crow + nb + 8 * q) = v4i{v[4 * q + 0], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
        }
      } else {
        const float sr = p.s_row[mc];
        float y[16];
        if constexpr (MODE == kModeChannel) {
#pragma unroll
          for (int r = 0; r < 16; ++r) y[r] = (float)acc[i][j][r] * (sr * sc[r >> 2][r & 3]);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) y[r] = acc[i][j][r] * sr;
        }
        if constexpr (HAS_LR) {
          const uint16_t* trow = p.t + (int64_t)mc * p.ldt + khalf * 8;
          v16f lr = v16f{};
#pragma unroll
          for (int rs = 0; rs < 4; ++rs) {
            if (rs * 16 < p.R) lr = lr_mfma<LRDT>(lb[rs], *reinterpret_cast<const v4i*>(trow + rs * 16), lr);
          }
#pragma unroll
          for (int r = 0; r < 16; ++r) y[r] = y[r] + lr[r];
        }
        if (p.bias) {
#pragma unroll
          for (int r = 0; r < 16; ++r) y[r] = y[r] + bi[r >> 2][r & 3];
        }
        if (mvalid) {
          const int64_t orow = p.out_row_idx ? (int64_t)p.out_row_idx[m] : (int64_t)m;
          uint16_t* crow = static_cast<uint16_t*>(p.c) + orow * p.ldc;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<v2u*>(crow + nb + 8 * q) =
                v2u{pack2<ODT>(y[4 * q + 0], y[4 * q + 1]), pack2<ODT>(y[4 * q + 2], y[4 * q + 3])};
        }
      }
      __builtin_amdgcn_sched_barrier(0);   // keep one tile's epilogue live at a time (no AGPR mass copy)
    }
  }
}

template <int WN, int WM, int TI, int TJ, int MODE, bool HAS_LR, int LRDT, int ODT>
int launch(GemmArgs& a, hipStream_t stream) {
  constexpr int BN = WN * TI * 32, BM = WM * TJ * 32;
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  const int64_t nblocks = (int64_t)a.tiles_m * a.tiles_n;
  if (nblocks > 0x7fffffff) return set_error(PQ_ESHAPE, "pq_int8_gemm: too many tiles");
  hipLaunchKernelGGL((gemm_kernel<WN, WM, TI, TJ, MODE, HAS_LR, LRDT, ODT>), dim3((unsigned)nblocks),
                     dim3(WN * WM * 64), 0, stream, a);
  return check_launch("int8_gemm");
}

template <int MODE, bool HAS_LR, int LRDT, int ODT>
int dispatch_tiles(GemmArgs& a, hipStream_t stream) {
  if constexpr (MODE == kModeGroup32) {
    // fp32 accumulators live in VGPRs (the VALU rescales them every group): 2 x 2 waves of 64 x 64
    return launch<2, 2, 2, 2, MODE, HAS_LR, LRDT, ODT>(a, stream);
  } else {
    return launch<2, 2, 4, 4, MODE, HAS_LR, LRDT, ODT>(a, stream);
  }
}

template <int MODE>
int dispatch_dtypes(GemmArgs& a, bool has_lr, int lr_dtype, int out_dtype, hipStream_t stream) {
  if (out_dtype == PQ_BF16) {
    if (!has_lr) return dispatch_tiles<MODE, false, PQ_BF16, PQ_BF16>(a, stream);
    if (lr_dtype == PQ_BF16) return dispatch_tiles<MODE, true, PQ_BF16, PQ_BF16>(a, stream);
    if (lr_dtype == PQ_F16) return dispatch_tiles<MODE, true, PQ_F16, PQ_BF16>(a, stream);
  } else if (out_dtype == PQ_F16) {
    if (!has_lr) return dispatch_tiles<MODE, false, PQ_F16, PQ_F16>(a, stream);
    if (lr_dtype == PQ_BF16) return dispatch_tiles<MODE, true, PQ_BF16, PQ_F16>(a, stream);
    if (lr_dtype == PQ_F16) return dispatch_tiles<MODE, true, PQ_F16, PQ_F16>(a, stream);
  }
  return set_error(PQ_EDTYPE, "pq_int8_gemm: unsupported dtype (out %d, low-rank %d)", out_dtype, lr_dtype);
}

int check_common(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                 const char* who) {
  if (M < 0 || N < 1 || K < 1) return set_error(PQ_ESHAPE, "%s: bad shape M=%lld N=%lld K=%lld", who, (long long)M, (long long)N, (long long)K);
  if (K % 64 != 0 || N % 64 != 0)
    return set_error(PQ_ESHAPE, "%s: need K %% 64 == 0 and N %% 64 == 0 (K=%lld, N=%lld)", who, (long long)K, (long long)N);
  if (M > 0x7fffffffLL - 512 || N > (1 << 30) || K > (1 << 30)) return set_error(PQ_ESHAPE, "%s: shape too large", who);
  if (!a || !w) return set_error(PQ_EINVAL, "%s: null operand", who);
  if (lda < K || ldw < K) return set_error(PQ_ESHAPE, "%s: lda/ldw < K", who);
  if ((uintptr_t)a % 16 || (uintptr_t)w % 16 || lda % 16 || ldw % 16)
    return set_error(PQ_EALIGN, "%s: a / w must be 16-byte aligned with lda, ldw %% 16 == 0", who);
  if (256 * lda > 0x7fffffffLL || 256 * ldw > 0x7fffffffLL)   // 32-bit buffer range of one 256-row tile
    return set_error(PQ_ESHAPE, "%s: row stride too large", who);
  return PQ_OK;
}

}  // namespace
}  // namespace pq

using namespace pq;

extern "C" int pq_int8_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, const float* s_row,
                            const float* s_w, int64_t group, const float* bias, const void* t, int64_t ldt,
                            const void* l2t, int64_t R, int32_t lr_dtype, void* c, int64_t ldc,
                            int32_t out_dtype, const int32_t* out_row_idx, int64_t M, int64_t N, int64_t K,
                            hipStream_t stream) {
  int st = check_common(a, lda, w, ldw, M, N, K, "pq_int8_gemm");
  if (st != PQ_OK) return st;
  if (M == 0) return PQ_OK;
  if (!s_row || !s_w || !c) return set_error(PQ_EINVAL, "pq_int8_gemm: null s_row / s_w / c");
  if (group != 0 && group != 32) return set_error(PQ_ESHAPE, "pq_int8_gemm: group must be 0 or 32, got %lld", (long long)group);
  if (ldc < N || ldc % 4 != 0 || (uintptr_t)c % 8)
    return set_error(PQ_EALIGN, "pq_int8_gemm: c must be 8-byte aligned with ldc >= N, ldc %% 4 == 0");
  if ((uintptr_t)s_w % 16 || (bias && (uintptr_t)bias % 16))
    return set_error(PQ_EALIGN, "pq_int8_gemm: s_w and bias must be 16-byte aligned");
  const bool has_lr = (t != nullptr) || (l2t != nullptr);
  if (has_lr) {
    if (!t || !l2t) return set_error(PQ_EINVAL, "pq_int8_gemm: low-rank needs both t and l2t");
    if (R < 16 || R > 64 || R % 16 != 0)
      return set_error(PQ_ESHAPE, "pq_int8_gemm: low-rank rank R=%lld must be 16, 32, 48 or 64", (long long)R);
    if (ldt < R || ldt % 8 != 0 || (uintptr_t)t % 16 || (uintptr_t)l2t % 16)
      return set_error(PQ_EALIGN, "pq_int8_gemm: t, l2t must be 16-byte aligned with ldt %% 8 == 0");
  }
  GemmArgs args{};
  args.a = a; args.w = w; args.s_row = s_row; args.s_w = s_w; args.bias = bias;
  args.t = static_cast<const uint16_t*>(t); args.l2t = static_cast<const uint16_t*>(l2t);
  args.c = c; args.out_row_idx = out_row_idx;
  args.lda = lda; args.ldw = ldw; args.ldt = ldt; args.ldc = ldc;
  args.M = (int)M; args.N = (int)N; args.K = (int)K; args.R = (int)R;
  if (group == 32) return dispatch_dtypes<kModeGroup32>(args, has_lr, lr_dtype, out_dtype, stream);
  return dispatch_dtypes<kModeChannel>(args, has_lr, lr_dtype, out_dtype, stream);
}

extern "C" int pq_int8_gemm_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c,
                                int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  int st = check_common(a, lda, w, ldw, M, N, K, "pq_int8_gemm_i32");
  if (st != PQ_OK) return st;
  if (M == 0) return PQ_OK;
  if (!c) return set_error(PQ_EINVAL, "pq_int8_gemm_i32: null c");
  if (ldc < N || ldc % 4 != 0 || (uintptr_t)c % 16)
    return set_error(PQ_EALIGN, "pq_int8_gemm_i32: c must be 16-byte aligned with ldc %% 4 == 0");
  GemmArgs args{};
  args.a = a; args.w = w; args.c = c;
  args.lda = lda; args.ldw = ldw; args.ldc = ldc;
  args.M = (int)M; args.N = (int)N; args.K = (int)K;
  return launch<2, 2, 4, 4, kModeI32, false, PQ_BF16, PQ_BF16>(args, stream);
}
