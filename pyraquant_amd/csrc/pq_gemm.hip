// Fused INT8 GEMM + dequant / low-rank / bias epilogue (+ routed row scatter) for gfx950.
//
// Math (reference: deploy/int8_exec.py:144-183 and :272-314, epilogue order :303-309):
//   per-channel: y[m,n] = (float)(sum_k a[m,k] w[n,k]) * (s_row[m] * s_w[n])
//   group-32   : y[m,n] = s_row[m] * sum_g s_w[g,n] * (float)(sum_{k in g} a[m,k] w[n,k])   (fma over g)
//   then y += sum_r t[m,r] l2t[n,r] (low-rank up-projection), y += bias[n], rounded to bf16/fp16.
//
// Operand roles. The MFMA computes D = W_tile * A_tile^T: its row operand ("i") is a weight row n and its
// column operand ("j") an activation row m, so each lane ends up holding 4 consecutive n of one output
// row m (8-byte 16-bit stores) and needs one s_row value per 32 x 32 tile. Group-32 without a low-rank term swaps
// the two (each lane holds one column n and needs one group scale per tile; see the main loop).
//
// The kernel (gemm_dma_kernel). 2 x WMW wavefronts (WMW = 2 or 4 along m). A workgroup owns a BN x BM (n x m)
// block, each wave a (BN/2) x (BM/WMW) part held as TI x TJ v_mfma_i32_32x32x32_i8 tiles (int32 accumulators in
// VGPRs: the kernels name no AGPR, so the compiler selects the MFMA form whose C / D operands are VGPRs, and the
// epilogue reads the accumulators in place, with no v_accvgpr_read copies). Large problems, and those whose 256 x 256
// blocks all fit on the CUs at once while their 128 x 128 blocks would not, run 256 x 256 blocks of 8 waves at one
// workgroup per CU (128 accumulators per wave, two waves per SIMD); smaller ones 128 x 128 blocks of 4 waves at two
// workgroups per CU, or 128 x 64 when the 128 x 128 blocks are too few to fill the chip.
// K advances in stages of 64 bytes through a ring of NS LDS stages (5 x 32 KB for the 256 x 256 block) filled by
// LDS-DMA buffer loads (buffer_load_dwordx4 ... lds): no VGPR staging, no ds_write, and NS - 1 stages of
// prefetch in flight to cover L2 / MALL latency. One DMA instruction fills 1 KB = 16 LDS rows of 64 bytes;
// each lane fetches the 16-byte chunk that the XOR swizzle places at its LDS slot, so the MFMA operand reads
// (ds_read_b128, one tile row per lane) are bank-conflict free. In the 8-wave 256 x 256 blocks the two wave groups
// ping-pong: per SIMD, one wave issues a stage's MFMAs back to back while the other reads the next stage's fragments
// and issues its DMA, swapping at each of two workgroup barriers per stage. In the 4-wave blocks the two 32-byte K
// substeps of a stage are software-pipelined instead: the fragments of the next substep are read from LDS while the
// MFMAs of the current one run, and the DMA of a new stage is interleaved with the MFMAs; one barrier per stage.
//
// Group-32 runs on the same kernel (MODE kModeGroup32): every 32-wide K substep is one K group, whose int32 partial
// (one MFMA from zero) the VALU converts and fma's with s_w[g, n] into an fp32 accumulator held in VGPRs, groups in
// order. The scales of each stage ride the DMA ring (dword LDS-DMA, a ring of NS + 1 slots of their own). That is
// 16 converts + 16 FMAs per lane per MFMA (128 VALU cycles of a wave64 against 32 of the MFMA), so group-32 is
// VALU-bound at a quarter of the INT8 MFMA rate; blocks are 128 x 128 at two workgroups per CU (128 x 64 for small
// problems and with a low-rank term).
//
// Workgroup ids are remapped so that each XCD (ids are dealt round-robin over the 8 XCDs) walks a contiguous
// run of tiles, rasterised in groups of group_m() m-tiles for L2 reuse. Large 256 x 256 products run one persistent
// workgroup per CU, which claims its XCD's tiles (then the other XCDs') through a scheduling buffer the caller owns
// (or, without one, takes a fixed share of them).
#include "pq_common.h"

#include <atomic>
#include <type_traits>

namespace pq {
namespace {

// m-tiles per raster group: about the square root of the tiles an XCD runs at once (32 CUs x workgroups per CU),
// so that the concurrent tiles cover a near-square block and re-read the fewest A and W rows beyond its L2
// (measured in the layer step: 6 for the 256 x 256 block at one per CU beat 4 by 0.7 % and 8 by 3 %).
template <int OCC>
constexpr int group_m() { return OCC == 1 ? 6 : 8; }

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
  int64_t c_rows;   // rows of c a scattered row may name: a row index outside [0, c_rows) is not written
  int64_t lda, ldw, ldt, ldc;
  int M, N, K, R;
  int tiles_m, tiles_n;
  int* sched;         // persistent blocks: 9 ints of claim counters, zero at launch and left zero (or NULL)
};

enum { kModeI32 = 0, kModeChannel = 1, kModeGroup32 = 2 };

// Map the linear workgroup id to (tile_m, tile_n): XCD-contiguous, then a raster of kGroupM m-tiles.
template <int kGroupM>
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

// c + y for 8 16-bit values (16 bytes): each sum in fp32, rounded to the 16-bit type (to nearest even), as torch adds
// two 16-bit tensors. The accumulate mode's last step: the addend already holds a rounded output, y the new one.
template <int DT>
__device__ __forceinline__ v4u add_16x8(v4u c, v4u y) {
  v4u r;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    r[q] = pack2<DT>(lo16_to_f32<DT>(c[q]) + lo16_to_f32<DT>(y[q]), hi16_to_f32<DT>(c[q]) + hi16_to_f32<DT>(y[q]));
  return r;
}

template <int LRDT>
__device__ __forceinline__ v16f lr_mfma(v4i a, v4i b, v16f c) {
  if constexpr (LRDT == PQ_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
  }
}

// ---- epilogue ---------------------------------------------------------------------------------------
// The wave's accumulators cover weight rows nbase + 32 i + [0, 32) and activation rows mbase + 32 j + [0, 32).
// Lane holds, for tile (i, j) and register r: m = mbase + 32 j + lane % 32,
// n = nbase + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4. The fp32 operations run in the reference's order
// (deploy/int8_exec.py:303-309). Operands are fetched ahead of use so that no tile waits on its own global load:
// the per-row operands (s_row, the scatter row, the low-rank row t[m, :]) are issued by prefetch_rows() while the
// last MFMAs run, and the per-column operands (s_w, bias, low-rank rows l2t[n, :]) of weight tile i + 1 are
// issued before the tiles of weight tile i are computed. LRS = number of 16-wide low-rank slices held (0: none).
// NTS: output stores carry the non-temporal hint (streamed past the L2). The large blocks' outputs (c1: 1.6 GB per
// launch) are never re-read by the kernel, and keeping them out of the L2 leaves it to the operand tiles (measured
// 0.5-1.3 % faster at c1 / c2b in the layer step).
template <int TI, int TJ, int MODE, int LRS, int LRDT, int ODT, int CB = 2, bool NTS = false, bool ACC = false>
struct Epilogue {
  // CB = 2: the column operands of weight tile i + 1 load while tile i is computed (one workgroup per CU);
  // CB = 1: loaded right before use (two workgroups per CU hide the latency and the register budget is halved).
  static constexpr bool HAS_LR = LRS > 0;
  static constexpr int RS = HAS_LR ? LRS : 1;   // 16-wide slices of the low rank: R == 16 * LRS exactly
  float sr[TJ];
  int orow[TJ];
  v4i tv[TJ][RS];
  v4f sc[CB][4], bi[CB][4];
  v4i lb[CB][RS];

  __device__ __forceinline__ void load_cols(const GemmArgs& p, int slot, int ntile, int lane) {
    if constexpr (MODE != kModeI32) {
      if (ntile >= p.N) return;
      const int nb = ntile + 4 * (lane >> 5);
      if constexpr (MODE == kModeChannel) {
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[slot][q] = *reinterpret_cast<const v4f*>(p.s_w + nb + 8 * q);
      }
      if (p.bias) {
#pragma unroll
        for (int q = 0; q < 4; ++q) bi[slot][q] = *reinterpret_cast<const v4f*>(p.bias + nb + 8 * q);
      }
      if constexpr (HAS_LR) {
        const uint16_t* lrow = p.l2t + (int64_t)(ntile + (lane & 31)) * p.R + (lane >> 5) * 8;
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) lb[slot][rs] = *reinterpret_cast<const v4i*>(lrow + rs * 16);
      }
    }
  }

  // per-row operands (issued under the last stage's MFMAs)
  __device__ __forceinline__ void prefetch_rows(const GemmArgs& p, int mbase, int lane) {
    if constexpr (MODE != kModeI32) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int m = mbase + j * 32 + (lane & 31);
        const int mc = min(m, p.M - 1);
        sr[j] = p.s_row[mc];
        if constexpr (HAS_LR) {
          const uint16_t* trow = p.t + (int64_t)mc * p.ldt + (lane >> 5) * 8;
#pragma unroll
          for (int rs = 0; rs < RS; ++rs) tv[j][rs] = *reinterpret_cast<const v4i*>(trow + rs * 16);
        }
      }
      if (p.out_row_idx) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) orow[j] = p.out_row_idx[min(mbase + j * 32 + (lane & 31), p.M - 1)];
      } else {
#pragma unroll
        for (int j = 0; j < TJ; ++j) orow[j] = mbase + j * 32 + (lane & 31);
      }
    }
  }

  // ---- operands in LDS (run_lds) ----
  // The first two ring stages past the end of K carry the epilogue operands instead of operand tiles (1 KB slots):
  //   row buffer:    [s_row[m0 ..]] [out_row_idx[m0 ..]] [t rows m0 .., R 16-bit values each]
  //   column buffer: [s_w[n0 ..]]   [bias[n0 ..]]        [l2t rows n0 .., R 16-bit values each]
  // The t / l2t rows are packed back to back and cut into 64-byte lines that are swizzled like the operand tiles
  // (16-byte chunk c of line L at slot c ^ swz(L % 16)), so the low-rank fragment reads are conflict free.
  static constexpr int kR = 16 * RS;
  __device__ __forceinline__ static int lr_off(int row, int rs, int kh) {
    const int b = row * kR * 2 + rs * 32 + kh * 16;
    const int line = b >> 6, ch = (b >> 4) & 3;
    return 2048 + line * 64 + ((ch ^ k64_swz(line & 15)) << 4);
  }
  // Output staging of run_lds: 32 rows x 64 outputs (two weight tiles) per pass, rows padded by 16 bytes.
  static constexpr int kPitchL = 128 + 16;
  static constexpr int kStageBytesL = 32 * kPitchL;

  // nloc / mloc: the wave's first column / row inside the workgroup block; nbase / mbase: the same, global.
  template <typename AccT>
  __device__ __forceinline__ void run_lds(const GemmArgs& p, AccT (&acc)[TI][TJ], int nloc, int mloc, int nbase,
                                          int mbase, int lane, uint8_t* stage, const uint8_t* cbuf,
                                          const uint8_t* rbuf) {
    static_assert(MODE != kModeI32 && TI % 2 == 0, "run_lds: dequant modes, pairs of weight tiles");
    const int khalf = lane >> 5;
    const bool has_bias = p.bias != nullptr;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int ml = mloc + j * 32 + (lane & 31);
      sr[j] = reinterpret_cast<const float*>(rbuf)[ml];
      if constexpr (HAS_LR) {
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) tv[j][rs] = *reinterpret_cast<const v4i*>(rbuf + lr_off(ml, rs, khalf));
      }
    }
    const int* orows = reinterpret_cast<const int*>(rbuf + 1024);
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      v4f srt[4];   // transposed tiles: s_row of this lane's 16 rows of tile j
      if constexpr (kT) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          srt[q] = *reinterpret_cast<const v4f*>(rbuf + (mloc + j * 32 + 8 * q + 4 * khalf) * 4);
      }
#pragma unroll
      for (int ih = 0; ih < TI / 2; ++ih) {
        // staging -> global: 8 lanes x 16 bytes per 128-byte row piece, 8 rows per store instruction
        // row addresses: one 32 x 32 -> 64-bit product per scattered row (ldc < 2^31), or the lane's first row plus a
        // wave-uniform offset
        const int lr_ = lane >> 3, lc = lane & 7;
        const int n = nbase + ih * 64 + lc * 8;
        const bool nvalid = n < p.N;
        const int ldc = (int)p.ldc;
        uint16_t* const cn = static_cast<uint16_t*>(p.c) + n;
        uint16_t* const cm = cn + (int64_t)(mbase + lr_) * ldc;
        auto valid = [&](int s0) {
          return nvalid && mbase + j * 32 + s0 + lr_ < p.M &&
                 (!p.out_row_idx || (uint64_t)(int64_t)orows[mloc + j * 32 + s0 + lr_] < (uint64_t)p.c_rows);
        };
        auto dst_of = [&](int s0) {
          return p.out_row_idx ? cn + (int64_t)orows[mloc + j * 32 + s0 + lr_] * ldc : cm + (int64_t)(j * 32 + s0) * ldc;
        };
        v4u prev[4];
        if constexpr (ACC) {
          // accumulate into c: its current contents are fetched before the tiles are computed, hiding the latency
#pragma unroll
          for (int s0 = 0; s0 < 32; s0 += 8)
            prev[s0 >> 3] = valid(s0) ? *reinterpret_cast<const v4u*>(dst_of(s0)) : v4u{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
          const int i = 2 * ih + ii;
          const int nl = nloc + 32 * i;
          if constexpr (kT) {
            const float bn = has_bias ? reinterpret_cast<const float*>(cbuf + 1024)[nl + (lane & 31)] : 0.0f;
            tile_t(acc[i][j], srt, bn, has_bias, stage + 4 * khalf * kPitchL + (ii * 32 + (lane & 31)) * 2, kPitchL);
            continue;
          }
          if constexpr (MODE == kModeChannel) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              sc[0][q] = *reinterpret_cast<const v4f*>(cbuf + (nl + 4 * khalf + 8 * q) * 4);
          }
          if (has_bias) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              bi[0][q] = *reinterpret_cast<const v4f*>(cbuf + 1024 + (nl + 4 * khalf + 8 * q) * 4);
          }
          if constexpr (HAS_LR) {
#pragma unroll
            for (int rs = 0; rs < RS; ++rs)
              lb[0][rs] = *reinterpret_cast<const v4i*>(cbuf + lr_off(nl + (lane & 31), rs, khalf));
          }
          tile(acc[i][j], j, 0, has_bias, stage + (lane & 31) * kPitchL + (ii * 32 + 4 * khalf) * 2);
        }
#pragma unroll
        for (int s0 = 0; s0 < 32; s0 += 8) {
          v4u v = *reinterpret_cast<const v4u*>(stage + (s0 + lr_) * kPitchL + lc * 16);
          if (valid(s0)) {
            uint16_t* const dst = dst_of(s0);
            if constexpr (ACC) v = add_16x8<ODT>(prev[s0 >> 3], v);
            if constexpr (NTS) {
              __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(dst));
            } else {
              *reinterpret_cast<v4u*>(dst) = v;
            }
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // One 32 x 32 tile: dequant (+ low rank, + bias) in the reference's order, rounded to 16 bits and written to
  // `dst` (this lane's row in the staging area, at its first output column): outputs 8 q + 4 (lane / 32) .. + 3.
  template <typename AccV>
  __device__ __forceinline__ void tile(const AccV& a, int j, int c, bool has_bias, uint8_t* dst) {
    v16f y;
    if constexpr (MODE == kModeChannel) {
#pragma unroll
      for (int r = 0; r < 16; ++r) y[r] = (float)a[r] * (sr[j] * sc[c][r >> 2][r & 3]);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) y[r] = a[r] * sr[j];
    }
    if constexpr (HAS_LR) {
      // y += t[m, :] . l2t[n, :] (fp32 accumulation of the 16-bit operands, deploy/int8_exec.py:304-307)
      v16f lr = v16f{};
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) lr = lr_mfma<LRDT>(lb[c][rs], tv[j][rs], lr);
#pragma unroll
      for (int r = 0; r < 16; ++r) y[r] = y[r] + lr[r];
    }
    if (has_bias) {
#pragma unroll
      for (int r = 0; r < 16; ++r) y[r] = y[r] + bi[c][r >> 2][r & 3];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<v2u*>(dst + 16 * q) =
          v2u{pack2<ODT>(y[4 * q + 0], y[4 * q + 1]), pack2<ODT>(y[4 * q + 2], y[4 * q + 3])};
  }

  // Group-32 without a low-rank term keeps its tiles transposed (see the main loop): lane l holds output column
  // n = l % 32 and rows 8 (r / 4) + 4 (l / 32) + r % 4. Same per-element dequant as tile() (y = acc * s_row[m],
  // + bias[n]); srt holds the s_row of the lane's 16 rows, bn its column's bias. Each converted pair (rows m, m + 1)
  // goes to the row-major staging area as two 16-bit writes: `col` is this lane's column in row 4 (l / 32).
  static constexpr bool kT = MODE == kModeGroup32 && LRS == 0;
  __device__ __forceinline__ void tile_t(const v16f& a, const v4f (&srt)[4], float bn, bool has_bias, uint8_t* col,
                                         int pitch) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        float y0 = a[4 * q + e] * srt[q][e], y1 = a[4 * q + e + 1] * srt[q][e + 1];
        if (has_bias) {
          y0 = y0 + bn;
          y1 = y1 + bn;
        }
        const uint32_t v = pack2<ODT>(y0, y1);
        *reinterpret_cast<uint16_t*>(col + (8 * q + e) * pitch) = (uint16_t)(v & 0xffffu);
        *reinterpret_cast<uint16_t*>(col + (8 * q + e + 1) * pitch) = (uint16_t)(v >> 16);
      }
  }

  // Rows of the wave's output sub-tile (32 TJ rows of 32 TI outputs) staged in LDS by run(): 16-bit outputs,
  // rows padded by 16 bytes so that the column-wise fragment writes spread over the banks.
  static constexpr int kRowBytes = 64 * TI;
  static constexpr int kPitch = kRowBytes + 16;
  static constexpr int kStageBytes = 32 * TJ * kPitch + 32 * TJ * 4;   // + the rows' scatter targets
  static constexpr int kPitch32 = 64 * 4 + 16;   // int32 mode: a staged row of two weight tiles' outputs, padded

  // Epilogue. int32 mode: the accumulators go through the wave's LDS staging area two weight tiles at a time and
  // out as whole rows. Dequant modes: each fragment is
  // dequantized (+ low rank, + bias) and rounded in registers, written to the wave's LDS staging area in row-major
  // order, and the wave then stores whole rows: lane l writes 16 bytes, 4 TI lanes cover a row's 64 TI bytes, so
  // every store instruction writes complete 128-byte lines (the fragment layout alone would write 16-byte pieces
  // of 32 rows per instruction). `stage` is this wave's kStageBytes of LDS, free once the main loop has ended.
  template <typename AccT>
  __device__ __forceinline__ void run(const GemmArgs& p, AccT (&acc)[TI][TJ], int nbase, int mbase, int lane,
                                      uint8_t* stage) {
    const int khalf = lane >> 5;
    const bool has_bias = p.bias != nullptr;
    if constexpr (MODE == kModeI32) {
      // Two weight tiles (32 rows x 64 int32 outputs) per pass through the staging area, then whole rows out: 16
      // lanes cover a row's 256 bytes, so each store instruction writes 4 rows of two complete 128-byte lines (the
      // fragments alone would write 32 rows x 32 bytes per instruction).
      static_assert(TI % 2 == 0 && 32 * kPitch32 <= kStageBytes, "int32 staging: pairs of weight tiles");
      const int lr4 = lane >> 4, lc16 = lane & 15;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
#pragma unroll
        for (int ih = 0; ih < TI / 2; ++ih) {
#pragma unroll
          for (int ii = 0; ii < 2; ++ii) {
            const v16i& v = acc[2 * ih + ii][j];
            // fragment -> staging row lane % 32, outputs 32 ii + 8 q + 4 (lane / 32) .. + 3
            uint8_t* const dst = stage + (lane & 31) * kPitch32 + (ii * 32 + 4 * khalf) * 4;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              *reinterpret_cast<v4i*>(dst + 32 * q) = v4i{v[4 * q + 0], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
          }
          const int n = nbase + ih * 64 + lc16 * 4;
#pragma unroll
          for (int s0 = 0; s0 < 32; s0 += 4) {
            const v4i v = *reinterpret_cast<const v4i*>(stage + (s0 + lr4) * kPitch32 + lc16 * 16);
            const int m = mbase + j * 32 + s0 + lr4;
            if (m < p.M && n < p.N)
              *reinterpret_cast<v4i*>(static_cast<int32_t*>(p.c) + (int64_t)m * p.ldc + n) = v;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      return;
    } else {
      int* srow = reinterpret_cast<int*>(stage + 32 * TJ * kPitch);
      if (khalf == 0) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) srow[j * 32 + (lane & 31)] = orow[j];
      }
      if constexpr (CB == 2) load_cols(p, 0, nbase, lane);
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        if constexpr (CB == 2) {
          if (i + 1 < TI) load_cols(p, (i + 1) & 1, nbase + (i + 1) * 32, lane);
        } else {
          load_cols(p, 0, nbase + i * 32, lane);
        }
        __builtin_amdgcn_sched_barrier(0);
        const int c = CB == 2 ? (i & 1) : 0;
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          if constexpr (kT) {
            // transposed tile: the lane's column n and its 16 rows (s_row clamped at the last row: rows past M are
            // computed but not stored)
            const int m0 = mbase + j * 32 + 4 * khalf;
            v4f srt[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int e = 0; e < 4; ++e) srt[q][e] = p.s_row[min(m0 + 8 * q + e, p.M - 1)];
            const int n = nbase + i * 32 + (lane & 31);
            const float bn = has_bias && n < p.N ? p.bias[n] : 0.0f;
            tile_t(acc[i][j], srt, bn, has_bias, stage + (j * 32 + 4 * khalf) * kPitch + (i * 32 + (lane & 31)) * 2,
                   kPitch);
          } else {
            // fragment -> staging rows: row (32 j + lane % 32), outputs 32 i + 8 q + 4 (lane / 32) .. + 3
            tile(acc[i][j], j, c, has_bias, stage + (j * 32 + (lane & 31)) * kPitch + (i * 32 + 4 * khalf) * 2);
          }
          __builtin_amdgcn_sched_barrier(0);   // keep one tile's epilogue live at a time
        }
      }
      // staging rows -> global: instruction s stores rows 16 s / TI + lane / (4 TI), 16 bytes per lane
      constexpr int LPR = 4 * TI;          // lanes per row
      constexpr int RPI = 64 / LPR;        // rows per store instruction
      static_assert(64 % LPR == 0 && (32 * TJ) % RPI == 0, "whole rows per store instruction");
      const int lr_ = lane / LPR, lc = lane % LPR;
      const int n = nbase + lc * 8;
      const bool nvalid = n < p.N;
      const int ldc = (int)p.ldc;
      uint16_t* const cn = static_cast<uint16_t*>(p.c) + n;
      uint16_t* const cm = cn + (int64_t)(mbase + lr_) * ldc;
#pragma unroll 4
      for (int s0 = 0; s0 < 32 * TJ; s0 += RPI) {
        const int row = s0 + lr_;
        const int m = mbase + row;
        v4u v = *reinterpret_cast<const v4u*>(stage + row * kPitch + lc * 16);
        if (nvalid && m < p.M && (!p.out_row_idx || (uint64_t)(int64_t)srow[row] < (uint64_t)p.c_rows)) {
          uint16_t* const dst = p.out_row_idx ? cn + (int64_t)srow[row] * ldc : cm + (int64_t)s0 * ldc;
          if constexpr (ACC) v = add_16x8<ODT>(*reinterpret_cast<const v4u*>(dst), v);   // accumulate into c
          if constexpr (NTS) {
            __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(dst));
          } else {
            *reinterpret_cast<v4u*>(dst) = v;
          }
        }
      }
    }
  }
};

// ---- the GEMM kernel: LDS-DMA ring of NS stages, 64-byte K stages ---------------------------------
constexpr int kBKd = 64;   // K bytes per stage (two 32-byte MFMA substeps)

// LDS row r (64 bytes, one tile row) stores its 16-byte chunk c at slot c ^ swz(r). Among 8 consecutive rows the
// (row parity, slot) pairs of one chunk are distinct, and among 16 consecutive rows the (row % 4, slot) pairs are,
// so the ds_read_b128 of 8 (or 16) lanes reading consecutive rows touch distinct banks in a 128-byte (or
// 256-byte) bank window.
__device__ __forceinline__ int swz(int r) { return k64_swz(r); }

template <int N>
__device__ __forceinline__ void wait_dma() { wait_vmcnt<N>(); }

// The ring's workgroup barrier. A fenced barrier (__syncthreads(), or a fence limited to LDS) makes the compiler
// wait for every LDS-DMA this wave has in flight (vmcnt(0)), which would drain the ring each stage. Here the
// ordering is explicit: the caller's vmcnt wait covers the DMA the next stage needs, lgkmcnt(0) completes this
// wave's LDS reads of the buffer that is about to be refilled, and sched_barrier keeps the scheduler from moving
// LDS accesses or DMA across the s_barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0), vmcnt and expcnt unconstrained
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Whether the block's epilogue takes its operands through the ring (run_lds): the row and column slots must fit one
// stage each and the operand DMA slots of one stage, and the output staging the remaining NS - 2 buffers.
template <int TI, int TJ, int WMW, int NS, int OCC, int MODE, int LRS, int LRDT, int ODT, bool ACC>
constexpr bool epilogue_in_ring() {
  using Epi = Epilogue<TI, TJ, MODE, LRS, LRDT, ODT, OCC * WMW == 2 ? 2 : 1, OCC == 1, ACC>;
  constexpr int NW = 2 * WMW, BN = 64 * TI, BM = 32 * TJ * WMW;
  constexpr int stage = (BN + BM) * kBKd, dma = (BN + BM) / 16;   // bytes and 1 KB DMA slots of a stage
  constexpr int lr = LRS * 16 * 2;                                // one low-rank row
  constexpr int rows = 2 + BM * lr / 1024, cols = 2 + BN * lr / 1024;
  return MODE != kModeI32 && TI % 2 == 0 && NS >= 3 && BN <= 256 && BM <= 256 && rows * 1024 <= stage &&
         cols * 1024 <= stage && rows <= dma && cols <= dma && (NS - 2) * (stage / Epi::kStageBytesL) >= NW;
}

// Persistent blocks (see the kernel): the 256 x 256 tile at one workgroup per CU with its epilogue operands in the
// ring and no accumulate (the other variants keep one tile per workgroup: in a loop they spill registers).
template <int TI, int TJ, int WMW, int NS, int OCC, int MODE, int LRS, int LRDT, int ODT, bool ACC>
constexpr bool persistent_block() {
  return OCC == 1 && TI == 4 && WMW == 4 && !ACC && epilogue_in_ring<TI, TJ, WMW, NS, OCC, MODE, LRS, LRDT, ODT, ACC>();
}

// WMW waves along m (2 or 4) times 2 along n; OCC workgroups per CU.
template <int TI, int TJ, int WMW, int NS, int OCC, bool PACKED, int MODE, int LRS, int LRDT, int ODT, bool ACC = false>
__global__ __attribute__((amdgpu_flat_work_group_size(128 * WMW, 128 * WMW),
                          amdgpu_waves_per_eu(OCC * WMW / 2, OCC * WMW / 2)))
void gemm_dma_kernel(const GemmArgs p) {
  constexpr bool G32 = MODE == kModeGroup32;
  constexpr int NW = 2 * WMW;                 // waves per workgroup
  constexpr int BN = 64 * TI, BM = 32 * TJ * WMW;
  constexpr int WB = BN * kBKd, AB = BM * kBKd;
  constexpr int SB = G32 ? 2 * BN * 4 : 0;    // group-32: the stage's two scale rows s_w[g, n0 .. n0 + BN)
  constexpr int STAGE = WB + AB;
  // Group-32 scales have a ring of their own, one slot longer than the operand ring: stage s in slot s % (NS + 1).
  // The DMA issued in iteration kt (stage kt + NS) then refills the slot of stage kt - 1, which every wave has
  // finished reading before the barrier of iteration kt, so the MFMA substeps read their scales straight from LDS.
  constexpr int SLOTS = NS + 1;
  constexpr int DW = BN / 16 / NW, DA = BM / 16 / NW;   // 1 KB DMA instructions per wave and stage (W, A)
  constexpr int DS = SB / 256 / NW;           // 256-byte (dword) DMA instructions per wave and stage (scales)
  static_assert(DW * 16 * NW == BN && DA * 16 * NW == BM && DS * 256 * NW == SB, "DMA split over the waves");
  constexpr int DPW = DW + DA + DS;
  // Epilogue operands through the ring (run_lds): see epilogue_in_ring.
  using Epi = Epilogue<TI, TJ, MODE, LRS, LRDT, ODT, OCC * WMW == 2 ? 2 : 1, OCC == 1, ACC>;
  constexpr int kLrBytes = LRS * 16 * 2;                       // one low-rank row
  constexpr int kRowSlots = 2 + BM * kLrBytes / 1024, kColSlots = 2 + BN * kLrBytes / 1024;
  constexpr bool ELDS = epilogue_in_ring<TI, TJ, WMW, NS, OCC, MODE, LRS, LRDT, ODT, ACC>();
  constexpr int NF = TI + TJ;                 // fragments per substep
  constexpr int kRest = TI * TJ - NF;         // MFMAs of a substep beyond the NF that carry a fragment read
  constexpr int kVPer = kRest > 0 ? (DPW + kRest - 1) / (kRest > 0 ? kRest : 1) : 0;   // DMA per such MFMA
  static_assert(NS >= 3 && (NS * STAGE + SLOTS * SB) * OCC <= 160 * 1024, "LDS ring");
  // LDS: the group-32 scale slots first, then the operand ring. With the scales at the start their LDS reads fit the
  // 16-bit immediate offset of ds_read (past a 64 KB ring they cost a v_add each); SLOTS * SB is a multiple of 1 KB.
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE + SLOTS * SB];
  uint8_t* const sscale = smem;
  uint8_t* const ring = smem + SLOTS * SB;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1;
  const int wm = wave >> 1;

  // Persistent blocks (the 256 x 256 tile with its epilogue operands in the ring, no accumulate): one workgroup per
  // CU loops over tiles, which takes the relaunch gap out of every tile after the first. Virtual block vb is the id
  // the launch-per-tile grid would have given the tile (tile_coords: XCD vb % 8, its local index vb / 8), so a
  // workgroup stays on its XCD's tiles and the raster is unchanged. The first tile of workgroup b is vb = b. After
  // that, with a scheduling buffer (p.sched: 8 per-XCD claim counters and an exit count, zero at launch), a
  // workgroup claims the next local index of its own XCD's tiles, and once those are gone it claims from the other
  // XCDs' lists. The XCDs of one chip run the loop at different speeds (up to 5 % apart), so fixed shares finish
  // up to 165 us apart at c1. Without the buffer it steps vb by the grid size (a fixed share per workgroup).
  constexpr bool PERSIST = persistent_block<TI, TJ, WMW, NS, OCC, MODE, LRS, LRDT, ODT, ACC>();
  // Ping-pong main loop for the 8-wave 256 x 256 blocks (see below); the 4-wave blocks interleave instead.
  constexpr bool PP = NW == 8 && OCC == 1 && !G32;
  const int nbt = p.tiles_m * p.tiles_n;
  // Claims (lane 0 of wave 0). XCD x's list holds cnt(x) tiles, of which first(x) went out as first tiles.
  const int x0 = blockIdx.x & 7;
  auto xcd_cnt = [&](int x) { return (nbt >> 3) + (x < (nbt & 7) ? 1 : 0); };
  auto xcd_first = [&](int x) { return ((int)gridDim.x - x + 7) >> 3; };
  // Part 1, issued before the epilogue so that the atomic's round trip overlaps it: the next local index of the own
  // XCD's list (or cnt(x0) if the first tiles took them all).
  auto claim_own = [&]() -> int {
    if (xcd_first(x0) >= xcd_cnt(x0)) return xcd_cnt(x0);
    return atomicAdd(p.sched + x0, 1) + xcd_first(x0);
  };
  // Part 2, after the epilogue: the own index if the list still had one, else the other 7 lists in a rotated order,
  // so that stealers spread over the victims. Without a scheduling buffer, the fixed share: vb + grid.
  auto claim_rest = [&](int vb, int own) -> int {
    if (!p.sched) return vb + (int)gridDim.x;
    if (own < xcd_cnt(x0)) return (own << 3) | x0;
    const int rot = blockIdx.x >> 3;
    for (int k = 1; k < 8; ++k) {
      const int x = (x0 + 1 + (k - 1 + rot) % 7) & 7;
      const int cnt = xcd_cnt(x), first = xcd_first(x);
      if (first >= cnt) continue;
      const int li = atomicAdd(p.sched + x, 1) + first;
      if (li < cnt) return (li << 3) | x;
    }
    return nbt;
  };
  for (int vb = blockIdx.x; vb < nbt;) {
  int tm, tn;
  tile_coords<group_m<OCC>()>(vb, nbt, p.tiles_m, p.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  // Persistent blocks: alternate rounds of an XCD's tiles (round = local index / workgroups per XCD) sweep K in
  // opposite directions. The raster's consecutive rounds share their m-tiles' A rows, so a reversed round starts on
  // the K range the previous round read last, which is still in the L2: 15 % fewer bytes fetched beyond the L2 at
  // c1 (3.79 -> 3.23 GB), the same time. The int32 sums do not depend on the order; group-32's fp32 sum over the
  // groups does (and its scale DMA follows kt), so it always sweeps forward.
  const bool rev = PERSIST && !G32 && (((vb >> 3) / max(1, (int)(gridDim.x >> 3))) & 1);

  // Buffer resources based at the block's first row. Rows past M / N, and the DMA of a stage past the end of K
  // (offset kOOB), lie outside num_records: those loads read no memory.
  //
  // Row-major operands: DMA instruction i of this wave fills LDS bytes [(wave * D + i) * 1024, +1024) of its
  // operand tile: rows (wave * D + i) * 16 + lane / 4, slot lane % 4. The chunk stored at that slot is
  // (lane % 4) ^ swz(row), and row % 16 == lane / 4, so it depends on the lane only.
  // Packed operands (packed K64 layout, see pq_pack_k64): the same 1 KB is the contiguous block (row block, kt)
  // at ((row block) * KT + kt) * 1024, already swizzled: lane l copies bytes [16 l, 16 l + 16).
  const int KT = p.K / kBKd;
  const int rows_w = min(BN, p.N - n0), rows_a = min(BM, p.M - m0);
  const int l4 = lane >> 2;
  int vw, va, stw, sta;
  __amdgpu_buffer_rsrc_t rs_w, rs_a;
  if constexpr (PACKED) {
    const int blk_w = (rows_w + 15) / 16, blk_a = (rows_a + 15) / 16;
    rs_w = __builtin_amdgcn_make_buffer_rsrc((void*)(p.w + (int64_t)(n0 / 16) * KT * 1024), (short)0,
                                             blk_w * KT * 1024, kBufferWord3);
    rs_a = __builtin_amdgcn_make_buffer_rsrc((void*)(p.a + (int64_t)(m0 / 16) * KT * 1024), (short)0,
                                             blk_a * KT * 1024, kBufferWord3);
    vw = wave * DW * KT * 1024 + lane * 16;
    va = wave * DA * KT * 1024 + lane * 16;
    stw = KT * 1024;
    sta = KT * 1024;
  } else {
    rs_w = __builtin_amdgcn_make_buffer_rsrc((void*)(p.w + (int64_t)n0 * p.ldw), (short)0, (int)(rows_w * p.ldw),
                                             kBufferWord3);
    rs_a = __builtin_amdgcn_make_buffer_rsrc((void*)(p.a + (int64_t)m0 * p.lda), (short)0, (int)(rows_a * p.lda),
                                             kBufferWord3);
    const int cdma = ((lane & 3) ^ swz(l4)) << 4;
    vw = (wave * DW * 16 + l4) * (int)p.ldw + cdma;
    va = (wave * DA * 16 + l4) * (int)p.lda + cdma;
    stw = 16 * (int)p.ldw;
    sta = 16 * (int)p.lda;
  }
  constexpr int kStageStep = PACKED ? 1024 : kBKd;   // buffer offset of one K stage
  // group-32 scales ([K/32, N] fp32): instruction i of this wave copies 64 scales of group 2 kt + d / (BN / 64),
  // d = DS * wave + i, starting at n0 + 64 (d % (BN / 64))
  __amdgpu_buffer_rsrc_t rs_s;
  int vs = 0;
  if constexpr (G32) {
    rs_s = __builtin_amdgcn_make_buffer_rsrc((void*)p.s_w, (short)0, (p.K / 32) * p.N * 4, kBufferWord3);
    vs = (n0 + lane) * 4;
  }

  auto dma = [&](int buf, int kt) {
    uint8_t* sb = ring + buf * STAGE;
    const int koff = kt < KT ? (rev ? KT - 1 - kt : kt) * kStageStep : kOOB;
#pragma unroll
    for (int i = 0; i < DW; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_w, (lds_void_t*)(sb + (wave * DW + i) * 1024), 16,
                                               vw + i * stw + koff, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < DA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_a, (lds_void_t*)(sb + WB + (wave * DA + i) * 1024), 16,
                                               va + i * sta + koff, 0, 0, 0);
    if constexpr (G32) {
#pragma unroll
      for (int i = 0; i < DS; ++i) {
        const int d = wave * DS + i, g = d / (BN / 64), ch = d % (BN / 64);
        const int so = kt < KT ? ((2 * kt + g) * p.N + ch * 64) * 4 : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_s, (lds_void_t*)(sscale + (kt % SLOTS) * SB + g * BN * 4 + ch * 256),
                                                 4, vs + so, 0, 0, 0);
      }
    }
  };

  // DMA of a stage s >= KT (no operand data left). With ELDS, stage KT brings the row operands of the epilogue and
  // stage KT + 1 the column operands: slot q (1 KB at q * 1024 of the stage buffer) is the WG's 16-byte DMA
  // instruction wave * (DW + DA) + i. Slots past the operands copy the last operand chunk again into their own
  // (unused) 1 KB, so no instruction repeats another's destination: identical copies into one slot are dead stores
  // the compiler removes, and a stage issuing fewer than DPW instructions would break the ring's vmcnt arithmetic.
  // Later stages load nothing (out of range).
  auto dma_tail = [&](int buf, int st) {
    if constexpr (ELDS) {
      if (st == KT || st == KT + 1) {
        uint8_t* sb = ring + buf * STAGE;
        const bool rows = st == KT;
        const int nsl = rows ? kRowSlots : kColSlots;
        const int rows_x = rows ? rows_a : rows_w;
        const float* sv = rows ? p.s_row + m0 : p.s_w + n0;
        const void* iv = rows ? (const void*)p.out_row_idx : (const void*)p.bias;
        const int ioff = rows ? m0 : n0;
        const __amdgpu_buffer_rsrc_t rs_v = __builtin_amdgcn_make_buffer_rsrc((void*)sv, (short)0, rows_x * 4,
                                                                             kBufferWord3);
        const __amdgpu_buffer_rsrc_t rs_i = __builtin_amdgcn_make_buffer_rsrc(
            iv ? (void*)(static_cast<const int*>(iv) + ioff) : (void*)p.s_w, (short)0, iv ? rows_x * 4 : 0,
            kBufferWord3);
        // low-rank rows: t (row stride ldt) or l2t (row stride R)
        const int64_t lrs = rows ? p.ldt : (int64_t)LRS * 16;
        const uint16_t* lp = rows ? p.t + (int64_t)m0 * p.ldt : p.l2t + (int64_t)n0 * LRS * 16;
        const int lrec = LRS ? (int)((rows_x - 1) * lrs * 2 + kLrBytes) : 0;
        const __amdgpu_buffer_rsrc_t rs_l = __builtin_amdgcn_make_buffer_rsrc(
            LRS ? (void*)lp : (void*)p.s_w, (short)0, lrec, kBufferWord3);
        // The slot offsets come from a lane number the compiler cannot see through, so they are computed at each
        // call: in the persistent loop it would otherwise keep them for every tile (17 64-bit values, spilled).
        int lane_t = lane;
        asm volatile("" : "+v"(lane_t));
#pragma unroll
        for (int i = 0; i < DW + DA; ++i) {
          const int qd = wave * (DW + DA) + i;   // destination slot (distinct for every instruction of the WG)
          const int q = min(qd, nsl - 1);        // source chunk
          int vo = lane_t * 16;
          __amdgpu_buffer_rsrc_t rs = q == 0 ? rs_v : rs_i;
          if (q >= 2) {
            // packed byte of slot lane: line L = 16 (q - 2) + lane / 4, stored chunk (lane % 4) ^ swz(L % 16)
            const int pb = ((q - 2) * 16 + (lane_t >> 2)) * 64 + (((lane_t & 3) ^ swz(lane_t >> 2)) << 4);
            constexpr int kLb = kLrBytes > 0 ? kLrBytes : 1;   // (no low rank: never reached)
            const int row = pb / kLb, cb = pb % kLb;
            vo = row * (int)lrs * 2 + cb;   // below lrec, a 32-bit value
            rs = rs_l;
          }
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(sb + qd * 1024), 16, vo, 0, 0, 0);
        }
        if constexpr (G32) {
#pragma unroll
          for (int i = 0; i < DS; ++i)   // scale slots: out of range, as in dma()
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs_s, (lds_void_t*)(sscale + (st % SLOTS) * SB + (wave * DS + i) * 256),
                                                     4, vs + kOOB, 0, 0, 0);
        }
        return;
      }
    }
    dma(buf, st);
  };

  // MFMA operand reads: lane reads tile row (lane % 32) of each 32-row fragment, K chunk 2 s + lane / 32 of
  // substep s. Fragment rows are 32-aligned, so swz(row) = swz(lane % 16).
  const int sw = swz(lane & 15);
  const int kh = lane >> 5;
  const int fw_off = (wn * (BN / 2) + (lane & 31)) * kBKd;
  const int fa_off = WB + (wm * (BM / WMW) + (lane & 31)) * kBKd;

  using acc_t = typename std::conditional<G32, v16f, v16i>::type;
  acc_t acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = acc_t{};

  v4i f0[NF], f1[NF];
  auto rd = [&](v4i (&f)[NF], int buf, int s) {
    const uint8_t* sb = ring + buf * STAGE;
    const int c = ((2 * s + kh) ^ sw) << 4;
#pragma unroll
    for (int i = 0; i < TI; ++i) f[i] = *reinterpret_cast<const v4i*>(sb + fw_off + i * 32 * kBKd + c);
#pragma unroll
    for (int j = 0; j < TJ; ++j) f[TI + j] = *reinterpret_cast<const v4i*>(sb + fa_off + j * 32 * kBKd + c);
  };
  // Per-channel / int32: MFMA accumulation in VGPRs. Group-32: substep s of stage kt is K group g = 2 kt + s; its
  // int32 partial is converted and fma'd with s_w[g, n] into the fp32 accumulator, groups in order (deploy
  // semantics: pyraquant/quantizers_weight.py:96-109). Lane element r of tile i holds row
  // n = wn BN / 2 + 32 i + 8 (r / 4) + 4 (lane / 32) + r % 4.
  auto mm = [&](const v4i (&f)[NF], int kt, int s) {
    if constexpr (G32 && LRS == 0) {
      // Transposed tiles (no low-rank term to line up with): the activation fragment is the MFMA's first operand, so
      // lane l holds output column n = l % 32 of each tile and its 16 rows m; all 16 partials of a lane share one
      // scale s_w[g, n], one dword per weight tile and group instead of the 16-value stripe of the other layout.
      const float* sgt =
          reinterpret_cast<const float*>(sscale + (kt % SLOTS) * SB) + s * BN + wn * (BN / 2) + (lane & 31);
      float sv[TI];
#pragma unroll
      for (int i = 0; i < TI; ++i) sv[i] = sgt[i * 32];
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          const v16i part = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[TI + j], f[i], v16i{}, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(sv[i], (float)part[r], acc[i][j][r]);
        }
    } else if constexpr (G32) {
      const float* sg = reinterpret_cast<const float*>(sscale + (kt % SLOTS) * SB) + s * BN + wn * (BN / 2) + 4 * kh;
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        v4f s4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) s4[q] = *reinterpret_cast<const v4f*>(sg + i * 32 + 8 * q);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          const v16i part = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[i], f[TI + j], v16i{}, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(s4[r >> 2][r & 3], (float)part[r], acc[i][j][r]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[i], f[TI + j], acc[i][j], 0, 0, 0);
    }
  };

  // Instruction order inside one substep: the NF fragment reads of the next substep are spread over the first NF
  // MFMAs of this one. In the second substep of a stage the remaining MFMAs also carry the DMA of the stage NS
  // ahead (issued after the reads: the scheduler keeps LDS reads ahead of a later LDS-DMA it cannot
  // disambiguate). sched_barrier(0) keeps each substep's MFMAs on its side of the stage barrier.
  auto interleave = [&](auto with_dma) {
    if constexpr (G32) {
      __builtin_amdgcn_sched_barrier(0);
      return;
    }
#pragma unroll
    for (int q = 0; q < NF; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
    }
    if constexpr (decltype(with_dma)::value && kRest > 0) {
#pragma unroll
      for (int q = 0; q < kRest; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // MFMA
        __builtin_amdgcn_sched_group_barrier(0x010, kVPer, 0);   // VMEM (LDS-DMA)
      }
    } else if constexpr (kRest > 0) {
      __builtin_amdgcn_sched_group_barrier(0x008, kRest, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  using no_dma = std::integral_constant<bool, false>;
  using with_dma = std::integral_constant<bool, true>;

  // Ring: stage s lives in buffer s % NS. In the interleaved loop (the else branch below) the DMA of stage s is
  // issued after the barrier of iteration s - NS and must have landed at the barrier that ends iteration s - 1,
  // NS - 1 iterations later; in between, the DMAs of NS - 2 younger stages may still be in flight, hence
  // vmcnt((NS - 2) * DPW). Its prologue issues all NS stages at once; the first barrier waits for stage 0 only (the
  // explicit barrier: a fenced one would wait for every DMA in flight). Issuing stages 1 .. NS - 1 only after stage 0
  // had landed put a second memory latency in front of every tile. The ping-pong loop's ring is described in its
  // branch.
  Epi epi;
  const int nbase = n0 + wn * (BN / 2), mbase = m0 + wm * (BM / WMW);
  if constexpr (PP) {
    // Ping-pong. Waves 0-3 (group A) and 4-7 (group B) hold one wave per SIMD each. Time is cut into slots ended
    // by workgroup barriers; in every slot one group runs a compute phase (a stage's 16 MFMAs back to back, from
    // fragments already in registers) while the other runs a memory phase (the next stage's 12 fragment reads and
    // its share of a DMA), group B one slot behind group A:
    //   slot 2s: A reads stage s, B computes stage s - 1;   slot 2s + 1: A computes stage s, B reads stage s.
    // So each SIMD's MFMA pipe is fed by one wave at a time in runs of 16. Two waves that both interleave MFMAs and
    // LDS reads alternate issue instruction by instruction, which costs pipe cycles (c1 GEMM: 70 % -> 73 % MFMA busy,
    // 3-4 % faster; c2a, c2b 2.5 % faster; outputs bit-identical).
    // The ring: the prologue issues stages 0 .. NS - 2; the memory phase of stage s issues stage s + NS - 1 into the
    // buffer of stage s - 1, which both groups have read by then. Stage s + 1 must have landed (every wave's DMA)
    // at the barrier that ends slot 2s + 1: group A waits at the end of its compute phase, group B at the end of its
    // memory phase, each for all but its NS - 2 younger stages (vmcnt((NS - 2) DPW)), as in the interleaved loop.
    // Each group passes 2 KT + 2 barriers: B idles in the first slot, A in the last.
    const bool grp_b = wave >= NW / 2;
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) {
      if (st < KT) dma(st, st);
      else dma_tail(st, st);
    }
    wait_dma<(NS - 2) * DPW>();   // this wave's stage 0 has landed
    lds_barrier();                // every wave's has
    if (grp_b) lds_barrier();     // group B: one idle slot
    int b = 0;
    auto slot_pair = [&](int s, auto tail) {
      // memory phase: both substeps' fragments of stage s, and this wave's DMA of stage s + NS - 1 into the buffer of
      // stage s - 1, which every wave has read (group A read it two slots ago, group B one slot ago)
      rd(f0, b, 0);
      rd(f1, b, 1);
      const int bd = b == 0 ? NS - 1 : b - 1;
      if constexpr (decltype(tail)::value) dma_tail(bd, s + NS - 1);
      else dma(bd, s + NS - 1);
      if (grp_b) wait_dma<(NS - 2) * DPW>();   // stage s + 1 has landed (group B: at the end of its memory phase)
      lds_barrier();
      // compute phase: 16 MFMAs back to back
      mm(f0, s, 0);
      mm(f1, s, 1);
      if (!grp_b) wait_dma<(NS - 2) * DPW>();  // group A: at the end of its compute phase
      lds_barrier();
      b = b + 1 == NS ? 0 : b + 1;
    };
    int s = 0;
    for (; s < KT - NS + 1; ++s) slot_pair(s, std::integral_constant<bool, false>{});
    for (; s < KT; ++s) slot_pair(s, std::integral_constant<bool, true>{});
    if (!grp_b) lds_barrier();    // group A: one idle slot while group B computes the last stage
    if constexpr (!ELDS) epi.prefetch_rows(p, mbase, lane);
  } else {
#pragma unroll
    for (int st = 0; st < NS; ++st) {
      if (st < KT) dma(st, st);
      else dma_tail(st, st);
    }
    wait_dma<(NS - 1) * DPW>();   // this wave's stage 0 has landed
    lds_barrier();                // every wave's has
    __builtin_amdgcn_sched_barrier(0);
    rd(f0, 0, 0);
    auto iter = [&](int kt, int b, int bn, auto tail) {
      rd(f1, b, 1);
      mm(f0, kt, 0);
      interleave(no_dma{});
      wait_dma<(NS - 2) * DPW>();   // this wave's DMA of stage kt + 1 has landed
      lds_barrier();                // every wave's has, and every wave is done reading buffer b
      __builtin_amdgcn_sched_barrier(0);
      rd(f0, bn, 0);
      if constexpr (decltype(tail)::value) dma_tail(b, kt + NS);
      else dma(b, kt + NS);
      mm(f1, kt, 1);
      interleave(with_dma{});
    };
    int b = 0;
    int kt = 0;
    for (; kt < KT - NS; ++kt) {      // stages kt + NS < KT: operand DMA
      const int bn = b + 1 == NS ? 0 : b + 1;
      iter(kt, b, bn, no_dma{});
      b = bn;
    }
    for (; kt < KT - 1; ++kt) {       // the last NS - 1 iterations: epilogue operands (dma_tail)
      const int bn = b + 1 == NS ? 0 : b + 1;
      iter(kt, b, bn, with_dma{});
      b = bn;
    }
    // last stage: the epilogue's operands are fetched under its MFMAs
    if constexpr (!ELDS) epi.prefetch_rows(p, mbase, lane);
    rd(f1, b, 1);
    mm(f0, KT - 1, 0);
    mm(f1, KT - 1, 1);
  }
  wait_dma<0>();     // the epilogue operands, and the out-of-range DMAs of the last iterations, have landed
  __syncthreads();   // every wave is done reading the ring: it becomes the output staging area
  // the own-list claim of the next tile goes out now; its result is read after the epilogue, which covers its latency
  int own = 0;
  if (PERSIST && p.sched && wave == 0 && lane == 0) own = claim_own();
  if constexpr (ELDS) {
    // buffers of stages KT (rows) and KT + 1 (columns) hold the operands; staging in the NS - 2 others
    constexpr int kSpb = STAGE / Epi::kStageBytesL;
    const int k = wave / kSpb;
    uint8_t* stage = ring + ((KT + 2 + k) % NS) * STAGE + (wave % kSpb) * Epi::kStageBytesL;
    epi.run_lds(p, acc, wn * (BN / 2), wm * (BM / WMW), nbase, mbase, lane, stage, ring + ((KT + 1) % NS) * STAGE,
                ring + (KT % NS) * STAGE);
  } else {
    static_assert(ELDS || NW * Epi::kStageBytes <= NS * STAGE, "output staging must fit the LDS ring");
    epi.run(p, acc, nbase, mbase, lane, ring + wave * Epi::kStageBytes);
  }
  if constexpr (PERSIST) {
    // The next tile reaches every wave through the last 4 bytes of the row-operand buffer: its last DMA slot is
    // past the row operands (kRowSlots < 32), so the epilogue never reads it, and the next tile's DMA overwrites it
    // only after the second barrier.
    static_assert(kRowSlots < NW * (DW + DA), "the row buffer's last slot holds no epilogue operand");
    int* const slot = reinterpret_cast<int*>(ring + (KT % NS) * STAGE + STAGE - 4);
    if (wave == 0 && lane == 0) *slot = claim_rest(vb, own);
    lds_barrier();
    vb = *slot;
    lds_barrier();   // every wave has read it, and is done with the staging area, before the next tile's DMA
  } else {
    vb = nbt;
  }
  }
  // The last workgroup out leaves the scheduling buffer as it found it (zero) for the caller's next launch.
  if (PERSIST && p.sched && wave == 0 && lane == 0) {
    if (atomicAdd(p.sched + 8, 1) == (int)gridDim.x - 1) {
#pragma unroll
      for (int x = 0; x < 9; ++x) atomicExch(p.sched + x, 0);
    }
  }
}

// ---- launchers ---------------------------------------------------------------------------------------------
int grid_of(GemmArgs& a, int BM, int BN, int threads, dim3& grid) {
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  const int64_t nblocks = (int64_t)a.tiles_m * a.tiles_n;
  if (const int st = check_grid(nblocks, threads, "pq_int8_gemm")) return st;
  grid = dim3((unsigned)nblocks);
  return PQ_OK;
}

// Ring depth: as many 64-byte K stages as fit this workgroup's share of the 160 KB LDS (5 x 32 KB for 256 x 256
// blocks at one workgroup per CU, 3 x 24 KB for 256 x 128 blocks at two per CU), at most 8.
template <int TI, int TJ, int WMW, int OCC, int MODE>
constexpr int ring_stages() {
  constexpr int stage = (64 * TI + 32 * TJ * WMW) * kBKd, sb = MODE == kModeGroup32 ? 2 * 64 * TI * 4 : 0;
  constexpr int ns = (160 * 1024 / OCC - sb) / (stage + sb);   // NS operand stages + NS + 1 scale slots
  return ns < 8 ? ns : 8;
}

// Compute units of the stream's device, rounded down to a multiple of the 8 XCDs (a persistent grid keeps workgroup
// b on XCD b % 8); 0 if unknown.
int persistent_workgroups(hipStream_t stream) {
  static std::atomic<int> cached[64];
  int dev = -1;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 0;
  }
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  cus &= ~7;
  if (dev < 64) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

template <int TI, int TJ, int WMW, int OCC, bool PACKED, int MODE, int LRS, int LRDT, int ODT, bool ACC = false>
int launch_dma(GemmArgs& a, hipStream_t stream) {
  constexpr int NS = ring_stages<TI, TJ, WMW, OCC, MODE>();
  dim3 grid;
  const int st = grid_of(a, 32 * TJ * WMW, 64 * TI, 128 * WMW, grid);
  if (st != PQ_OK) return st;
  int* const sched = a.sched;   // the caller's scheduling buffer (or NULL): used by persistent launches only
  a.sched = nullptr;
  if constexpr (persistent_block<TI, TJ, WMW, NS, OCC, MODE, LRS, LRDT, ODT, ACC>()) {
    // one workgroup per CU; each XCD's share of workgroups claims that XCD's tiles (see the kernel)
    const int wg = persistent_workgroups(stream);
    if (wg > 0 && grid.x > (unsigned)wg) {
      grid.x = (unsigned)wg;
      a.sched = sched;
    }
  }
  hipLaunchKernelGGL((gemm_dma_kernel<TI, TJ, WMW, NS, OCC, PACKED, MODE, LRS, LRDT, ODT, ACC>), grid, dim3(128 * WMW), 0,
                     stream, a);
  return check_launch("int8_gemm");
}

// 128 x 128 blocks of the problem (the small-problem tile).
inline int64_t small_blocks(const GemmArgs& a) { return (int64_t)((a.M + 127) / 128) * ((a.N + 127) / 128); }

// Tile choice of the LDS-DMA kernel: 256 x 256 blocks of 8 waves at one workgroup per CU, or 128 x 128 blocks of 4
// waves at two per CU (or 128 x 64 when even those are too few to fill the chip).
// * Large problems (at least 1024 blocks of 256 x 128) take 256 x 256 blocks: a third less LDS-DMA traffic per MFMA
//   than two 256 x 128 workgroups of 4 waves (measured in the layer's back-to-back step, interleaved on one box: 2 %
//   faster at K = 3072, 6 % at K = 12288).
// * So do problems whose 256 x 256 blocks all fit in one round (at most one per CU) while their 128 x 128 blocks
//   would need more than one round of two per CU. A 256 x 256 block takes about 3x the time of a 128 x 128 block for
//   4x its work, so one round of them beats the extra round of small blocks. Measured at M = 4352 (FLUX's 1K token
//   count), bit-identical outputs: 56.7 -> 45.2 us at K = N = 3072, 182 -> 150 us at K = 12288, N = 3072, 226 ->
//   179 us at K = 15360; at M = 4096, K = N = 3072: 46.0 -> 44.4 us. Where the 128 x 128 blocks fit in one round
//   (M = 2048) or the 256 x 256 ones need a second (M = 8192), 128 x 128 stays faster (27.7 against 35.9 us, 92
//   against 94.6 us).
inline bool big_tiles(const GemmArgs& a, hipStream_t stream) {
  const int64_t tiles = (int64_t)((a.M + 127) / 128) * ((a.N + 255) / 256);
  if (tiles >= 1024) return true;
  const int64_t cus = persistent_workgroups(stream);
  const int64_t big = (int64_t)((a.M + 255) / 256) * ((a.N + 255) / 256);
  return cus > 0 && big <= cus && small_blocks(a) > 2 * cus;
}

template <bool PACKED, int MODE, int LRS, int LRDT, int ODT, bool ACC>
int dispatch_tiles(GemmArgs& a, hipStream_t stream) {
  if constexpr (MODE == kModeGroup32) {
    // fp32 accumulators live in VGPRs (the VALU rescales them every group): 128 x 128 blocks, two per CU; with
    // fewer than 512 of them, 128 x 64 blocks (the VALU-bound kernel then spreads over twice the CUs: measured
    // 1.2-1.5x faster at M = 2048 for the SDXL shapes, slower once the 128 x 128 blocks fill the chip). With a
    // low-rank epilogue always 128 x 64: at 128 x 128 its slices of t and l2t push the kernel past its 256 VGPRs
    // (5-49 spilled).
    if constexpr (LRS > 0) {
      return launch_dma<2, 1, 2, 2, PACKED, MODE, LRS, LRDT, ODT, ACC>(a, stream);
    } else {
      if (small_blocks(a) < 512) return launch_dma<2, 1, 2, 2, PACKED, MODE, LRS, LRDT, ODT, ACC>(a, stream);
      return launch_dma<2, 2, 2, 2, PACKED, MODE, LRS, LRDT, ODT, ACC>(a, stream);
    }
  } else {
    if (big_tiles(a, stream)) return launch_dma<4, 2, 4, 1, PACKED, MODE, LRS, LRDT, ODT, ACC>(a, stream);
    // fewer 128 x 128 blocks than half the CUs: 128 x 64 blocks (measured 1.3x faster at 80 blocks, even at 160)
    if (small_blocks(a) < 128) return launch_dma<2, 1, 2, 2, PACKED, MODE, LRS, LRDT, ODT, ACC>(a, stream);
    return launch_dma<2, 2, 2, 2, PACKED, MODE, LRS, LRDT, ODT, ACC>(a, stream);
  }
}

// low-rank slices held in registers: exactly R / 16 (R = 16, 32 or 64)
template <bool PACKED, int MODE, int DT, bool ACC>
int dispatch_rank(GemmArgs& a, hipStream_t stream) {
  if (a.R == 32) return dispatch_tiles<PACKED, MODE, 2, DT, DT, ACC>(a, stream);
  if (a.R == 16) return dispatch_tiles<PACKED, MODE, 1, DT, DT, ACC>(a, stream);
  return dispatch_tiles<PACKED, MODE, 4, DT, DT, ACC>(a, stream);
}

// The low-rank operands t / l2t share the output's 16-bit type (the reference computes t in lr_A's dtype and
// Int8Linear keeps lr_A in the model dtype, deploy/int8_exec.py:371-390).
template <bool PACKED, int MODE, bool ACC = false>
int dispatch_dtypes(GemmArgs& a, bool has_lr, int lr_dtype, int out_dtype, hipStream_t stream) {
  if (has_lr && lr_dtype != out_dtype)
    return set_error(PQ_EDTYPE, "pq_int8_gemm: low-rank dtype %d must equal the output dtype %d", lr_dtype, out_dtype);
  if (out_dtype == PQ_BF16) {
    if (!has_lr) return dispatch_tiles<PACKED, MODE, 0, PQ_BF16, PQ_BF16, ACC>(a, stream);
    return dispatch_rank<PACKED, MODE, PQ_BF16, ACC>(a, stream);
  } else if (out_dtype == PQ_F16) {
    if (!has_lr) return dispatch_tiles<PACKED, MODE, 0, PQ_F16, PQ_F16, ACC>(a, stream);
    return dispatch_rank<PACKED, MODE, PQ_F16, ACC>(a, stream);
  }
  return set_error(PQ_EDTYPE, "pq_int8_gemm: unsupported output dtype %d", out_dtype);
}

// Largest row stride of t: 255 rows of it plus one 128-byte row stay below 2^31 bytes.
constexpr int64_t kMaxLdt = 1LL << 22;

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
  // every buffer offset of one 256-row tile (row * ld + K offset) must stay below kOOB
  if (256 * lda + K > kOOB || 256 * ldw + K > kOOB) return set_error(PQ_ESHAPE, "%s: row stride too large", who);
  return PQ_OK;
}

}  // namespace
}  // namespace pq

using namespace pq;

extern "C" int pq_int8_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, const float* s_row,
                            const float* s_w, int64_t group, const float* bias, const void* t, int64_t ldt,
                            const void* l2t, int64_t R, int32_t lr_dtype, void* c, int64_t ldc,
                            int32_t out_dtype, const int32_t* out_row_idx, int64_t c_rows, int64_t M, int64_t N,
                            int64_t K, int32_t* sched, hipStream_t stream) {
  int st = check_common(a, lda, w, ldw, M, N, K, "pq_int8_gemm");
  if (st != PQ_OK) return st;
  if (M == 0) return PQ_OK;
  if ((uintptr_t)sched % 4) return set_error(PQ_EALIGN, "pq_int8_gemm: sched must be 4-byte aligned");
  if (out_row_idx && c_rows < 1)
    return set_error(PQ_ESHAPE, "pq_int8_gemm: a scatter needs the rows of c (c_rows=%lld)", (long long)c_rows);
  if (!s_row || !s_w || !c) return set_error(PQ_EINVAL, "pq_int8_gemm: null s_row / s_w / c");
  if (group != 0 && group != 32) return set_error(PQ_ESHAPE, "pq_int8_gemm: group must be 0 or 32, got %lld", (long long)group);
  if (group == 32 && (K / 32) * N * 4 > kOOB - 4096)
    return set_error(PQ_ESHAPE, "pq_int8_gemm: group-32 scales of %lld x %lld exceed the 32-bit buffer range", (long long)N, (long long)K);
  if (ldc < N || ldc % 4 != 0 || (uintptr_t)c % 8)
    return set_error(PQ_EALIGN, "pq_int8_gemm: c must be 8-byte aligned with ldc >= N, ldc %% 4 == 0");
  if (ldc > 0x7fffffffLL) return set_error(PQ_ESHAPE, "pq_int8_gemm: ldc %lld is 2^31 or more", (long long)ldc);
  if ((uintptr_t)s_w % 16 || (bias && (uintptr_t)bias % 16))
    return set_error(PQ_EALIGN, "pq_int8_gemm: s_w and bias must be 16-byte aligned");
  const bool has_lr = (t != nullptr) || (l2t != nullptr);
  if (has_lr) {
    if (!t || !l2t) return set_error(PQ_EINVAL, "pq_int8_gemm: low-rank needs both t and l2t");
    if (R != 16 && R != 32 && R != 64)
      return set_error(PQ_ESHAPE, "pq_int8_gemm: low-rank rank R=%lld must be 16, 32 or 64", (long long)R);
    if (ldt < R || ldt % 8 != 0 || (uintptr_t)t % 16 || (uintptr_t)l2t % 16)
      return set_error(PQ_EALIGN, "pq_int8_gemm: t, l2t must be 16-byte aligned with ldt %% 8 == 0");
    // the epilogue addresses a tile's 256 rows of t with 32-bit buffer offsets
    if (ldt > kMaxLdt) return set_error(PQ_ESHAPE, "pq_int8_gemm: ldt %lld exceeds %lld", (long long)ldt, (long long)kMaxLdt);
  }
  GemmArgs args{};
  args.a = a; args.w = w; args.s_row = s_row; args.s_w = s_w; args.bias = bias;
  args.t = static_cast<const uint16_t*>(t); args.l2t = static_cast<const uint16_t*>(l2t);
  args.c = c; args.out_row_idx = out_row_idx; args.c_rows = c_rows;
  args.lda = lda; args.ldw = ldw; args.ldt = ldt; args.ldc = ldc;
  args.M = (int)M; args.N = (int)N; args.K = (int)K; args.R = (int)R;
  args.sched = sched;
  if (group == 32) return dispatch_dtypes<false, kModeGroup32>(args, has_lr, lr_dtype, out_dtype, stream);
  return dispatch_dtypes<false, kModeChannel>(args, has_lr, lr_dtype, out_dtype, stream);
}

extern "C" int pq_int8_gemm_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c,
                                int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  int st = check_common(a, lda, w, ldw, M, N, K, "pq_int8_gemm_i32");
  if (st != PQ_OK) return st;
  if (M == 0) return PQ_OK;
  if (!c) return set_error(PQ_EINVAL, "pq_int8_gemm_i32: null c");
  if (ldc < N || ldc % 4 != 0 || (uintptr_t)c % 16)
    return set_error(PQ_EALIGN, "pq_int8_gemm_i32: c must be 16-byte aligned with ldc %% 4 == 0");
  if (ldc > 0x7fffffffLL) return set_error(PQ_ESHAPE, "pq_int8_gemm_i32: ldc %lld is 2^31 or more", (long long)ldc);
  GemmArgs args{};
  args.a = a; args.w = w; args.c = c;
  args.lda = lda; args.ldw = ldw; args.ldc = ldc;
  args.M = (int)M; args.N = (int)N; args.K = (int)K;
  if (big_tiles(args, stream)) return launch_dma<4, 2, 4, 1, false, kModeI32, 0, PQ_BF16, PQ_BF16>(args, stream);
  return launch_dma<2, 2, 2, 2, false, kModeI32, 0, PQ_BF16, PQ_BF16>(args, stream);
}

int pq::int8_gemm_packed(const int8_t* ap, const int8_t* wp, const float* s_row, const float* s_w, int64_t group,
                         const float* bias, const void* t, int64_t ldt, const void* l2t, int64_t R, int32_t lr_dtype,
                         void* c, int64_t ldc, int32_t out_dtype, const int32_t* out_row_idx, int64_t c_rows,
                         int64_t M, int64_t N, int64_t K, int32_t* sched, hipStream_t stream) {
  const bool accumulate = (out_dtype & PQ_ACCUMULATE) != 0;
  out_dtype &= ~PQ_ACCUMULATE;
  if (M < 0 || N < 1 || K < 1) return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: bad shape");
  if (K % 64 != 0 || N % 64 != 0)
    return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: need K %% 64 == 0 and N %% 64 == 0 (K=%lld, N=%lld)",
                     (long long)K, (long long)N);
  // packed offsets of one 256-row tile (16 blocks of K / 64 KB) must stay below kOOB
  if (M > 0x7fffffffLL - 512 || N > (1 << 30) || 16 * (K / 64) * 1024 + 1024 > kOOB)
    return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: shape too large");
  if (M == 0) return PQ_OK;
  if (!ap || !wp || !c) return set_error(PQ_EINVAL, "pq_int8_gemm_packed: null operand");
  if ((uintptr_t)ap % 16 || (uintptr_t)wp % 16) return set_error(PQ_EALIGN, "pq_int8_gemm_packed: ap / wp must be 16-byte aligned");
  if ((uintptr_t)sched % 4) return set_error(PQ_EALIGN, "pq_int8_gemm_packed: sched must be 4-byte aligned");
  GemmArgs args{};
  args.a = ap; args.w = wp; args.c = c;
  args.M = (int)M; args.N = (int)N; args.K = (int)K;
  args.sched = sched;
  if (accumulate && (out_dtype == PQ_I32 || group != 0))
    return set_error(PQ_EINVAL, "pq_int8_gemm_packed: PQ_ACCUMULATE takes a 16-bit output and per-channel weights");
  if (out_dtype == PQ_I32) {
    if (ldc < N || ldc % 4 != 0 || (uintptr_t)c % 16)
      return set_error(PQ_EALIGN, "pq_int8_gemm_packed: int32 c must be 16-byte aligned with ldc %% 4 == 0");
    if (ldc > 0x7fffffffLL) return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: ldc %lld is 2^31 or more", (long long)ldc);
    args.ldc = ldc;
    if (big_tiles(args, stream)) return launch_dma<4, 2, 4, 1, true, kModeI32, 0, PQ_BF16, PQ_BF16>(args, stream);
    return launch_dma<2, 2, 2, 2, true, kModeI32, 0, PQ_BF16, PQ_BF16>(args, stream);
  }
  if (!s_row || !s_w) return set_error(PQ_EINVAL, "pq_int8_gemm_packed: null s_row / s_w");
  if (out_row_idx && c_rows < 1)
    return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: a scatter needs the rows of c (c_rows=%lld)", (long long)c_rows);
  if (group != 0 && group != 32)
    return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: group must be 0 or 32, got %lld", (long long)group);
  if (group == 32 && (K / 32) * N * 4 > kOOB - 4096)
    return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: group-32 scales of %lld x %lld exceed the 32-bit buffer range", (long long)N, (long long)K);
  if (ldc < N || ldc % 4 != 0 || (uintptr_t)c % 8)
    return set_error(PQ_EALIGN, "pq_int8_gemm_packed: c must be 8-byte aligned with ldc >= N, ldc %% 4 == 0");
  if (ldc > 0x7fffffffLL) return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: ldc %lld is 2^31 or more", (long long)ldc);
  if ((uintptr_t)s_w % 16 || (bias && (uintptr_t)bias % 16))
    return set_error(PQ_EALIGN, "pq_int8_gemm_packed: s_w and bias must be 16-byte aligned");
  const bool has_lr = (t != nullptr) || (l2t != nullptr);
  if (has_lr) {
    if (!t || !l2t) return set_error(PQ_EINVAL, "pq_int8_gemm_packed: low-rank needs both t and l2t");
    if (R != 16 && R != 32 && R != 64)
      return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: low-rank rank R=%lld must be 16, 32 or 64", (long long)R);
    if (ldt < R || ldt % 8 != 0 || (uintptr_t)t % 16 || (uintptr_t)l2t % 16)
      return set_error(PQ_EALIGN, "pq_int8_gemm_packed: t, l2t must be 16-byte aligned with ldt %% 8 == 0");
    // the epilogue addresses a tile's 256 rows of t with 32-bit buffer offsets
    if (ldt > kMaxLdt) return set_error(PQ_ESHAPE, "pq_int8_gemm_packed: ldt %lld exceeds %lld", (long long)ldt, (long long)kMaxLdt);
  }
  args.s_row = s_row; args.s_w = s_w; args.bias = bias;
  args.t = static_cast<const uint16_t*>(t); args.l2t = static_cast<const uint16_t*>(l2t);
  args.out_row_idx = out_row_idx; args.c_rows = c_rows;
  args.ldt = ldt; args.ldc = ldc; args.R = (int)R;
  if (group == 32) return dispatch_dtypes<true, kModeGroup32>(args, has_lr, lr_dtype, out_dtype, stream);
  if (accumulate) return dispatch_dtypes<true, kModeChannel, true>(args, has_lr, lr_dtype, out_dtype, stream);
  return dispatch_dtypes<true, kModeChannel>(args, has_lr, lr_dtype, out_dtype, stream);
}

extern "C" int pq_int8_gemm_packed(const int8_t* ap, const int8_t* wp, const float* s_row, const float* s_w,
                                   int64_t group, const float* bias, const void* t, int64_t ldt, const void* l2t, int64_t R,
                                   int32_t lr_dtype, void* c, int64_t ldc, int32_t out_dtype,
                                   const int32_t* out_row_idx, int64_t c_rows, int64_t M, int64_t N, int64_t K,
                                   int32_t* sched, hipStream_t stream) {
  return pq::int8_gemm_packed(ap, wp, s_row, s_w, group, bias, t, ldt, l2t, R, lr_dtype, c, ldc, out_dtype, out_row_idx,
                              c_rows, M, N, K, sched, stream);
}
