// Routed-executor geometry and feathered fusion on the device, for gfx950.
//
// Reference: the routed FLUX executor builds row-run boxes of the selected leaves (flux/run_flux.py:340-355),
// maps them to packed-token cores, dilates them by the halo and extracts one patch per core, grouped by shape
// (flux/routing.py:202-315); after the transformer it blends the patch predictions into the background with a
// continuous feather weight (flux/routing.py:328-379). The reference does this on the host from a copy of the leaf
// mask (sel.cpu(), flux/run_flux.py:343) and with one torch slice / cat / blend op per patch. Here the mask stays on
// the device and each step is one kernel; nothing waits for the host.
//
// Patch table (int32 x kTableStride per patch, in the reference's extraction order: shapes ascending, then the order
// of the row-run boxes):
//   [0..3] halo box oy0, oy1, ox0, ox1 (packed-token coordinates, clamped to the grid)
//   [4..7] core box cy0, cy1, cx0, cx1
//   [8]    first row of the patch in the patch-order row list (rows of a patch are row-major)
//   [9]    index of the row-run box the patch came from
//   [10]   bucket (rank of the patch's shape among the distinct shapes)
//   [11]   0
// counts[0] = patches, counts[1] = rows, counts[2] = buckets, counts[3] = error bits (1: rows buffer too small).
#include "pq_common.h"

#include <algorithm>

namespace pq {
namespace {

constexpr int kTableStride = 12;
constexpr int kMaxBoxes = 2048;   // row-run boxes per mask (at most Lh * ceil(Lw / 2))

// Exclusive prefix sum over the workgroup (blockDim.x a multiple of 64, at most 1024). `sh` holds >= 16 ints.
__device__ int block_excl_scan(int v, int* sh, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[w] = x;
  __syncthreads();
  if (w == 0) {
    int s = lane < nw ? sh[lane] : 0;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int y = __shfl_up(s, o, 64);
      if (lane >= o) s += y;
    }
    if (lane < nw) sh[lane] = s;
  }
  __syncthreads();
  const int base = w > 0 ? sh[w - 1] : 0;
  total = sh[nw - 1];
  __syncthreads();
  return base + x - v;
}

// ---- union of the halo-dilated active leaves (the Linear-level gather list) -----------------------------------
// Token (y, x) is routed when some selected leaf (i, j), dilated by `halo` tokens and clamped to the grid, covers it
// (flux/routing.py:235-244 dilation). Dilation is separable: with R(y) the leaf rows whose dilated span holds y and
// C(x) the leaf columns whose dilated span holds x, (y, x) is covered iff ym(y) = OR_{i in R(y)} sel[i] has a bit in
// C(x). The mask is staged in LDS as one 64-bit word per leaf row (Lw <= 64). Workgroup g owns token rows
// [g H / G, (g + 1) H / G): it counts the covered tokens of every earlier row from ym alone (the union of the
// dilated column spans of ym's bits, merged left to right), which places its rows in the global list without a
// second pass or a scratch buffer, then compacts its own rows in order. The list is sorted and unique.
__device__ __forceinline__ uint64_t span_bits(int lo, int hi) {   // bits lo..hi (0 <= lo, hi <= 63), 0 if hi < lo
  if (hi < lo) return 0;
  const uint64_t top = hi == 63 ? ~0ull : ((2ull << hi) - 1);
  return top & ~((1ull << lo) - 1);
}

struct UnionGeom {
  int Lh, Lw, leaf, halo, H, W;
  // leaf indices whose dilated span [k leaf - halo, (k + 1) leaf + halo) holds coordinate c
  __device__ int lo(int c) const { const int a = c - halo - leaf + 1; return a <= 0 ? 0 : (a + leaf - 1) / leaf; }
  __device__ int hi(int c, int n) const { return min(n - 1, (c + halo) / leaf); }
  __device__ uint64_t row_mask(int y, const uint64_t* rbits) const {
    uint64_t m = 0;
    for (int i = lo(y), e = hi(y, Lh); i <= e; ++i) m |= rbits[i];
    return m;
  }
  // covered tokens of a row with leaf-column mask m: union of the clamped spans of its bits
  __device__ int row_count(uint64_t m) const {
    int n = 0, end = 0;
    while (m) {
      const int j = __builtin_ctzll(m);
      m &= m - 1;
      const int a = max(max(0, j * leaf - halo), end), b = min(W, (j + 1) * leaf + halo);
      if (b > a) n += b - a;
      end = max(end, b);
    }
    return n;
  }
};

__global__ __launch_bounds__(256) void route_union_kernel(const uint8_t* __restrict__ sel, UnionGeom g,
                                                          int32_t* __restrict__ rows, int32_t* __restrict__ count) {
  __shared__ int sh[32];
  __shared__ uint8_t sm[32768];
  __shared__ uint64_t rbits[1024];
  for (int i = threadIdx.x; i < g.Lh * g.Lw; i += blockDim.x) sm[i] = sel[i];
  __syncthreads();
  for (int i = threadIdx.x; i < g.Lh; i += blockDim.x) {
    uint64_t b = 0;
    for (int j = 0; j < g.Lw; ++j) b |= (uint64_t)(sm[i * g.Lw + j] != 0) << j;
    rbits[i] = b;
  }
  __syncthreads();
  const int G = gridDim.x;
  const int y0 = (int)((int64_t)blockIdx.x * g.H / G), y1 = (int)((int64_t)(blockIdx.x + 1) * g.H / G);
  int part = 0;
  for (int y = threadIdx.x; y < y0; y += blockDim.x) part += g.row_count(g.row_mask(y, rbits));
  int base;
  block_excl_scan(part, sh, base);
  for (int y = y0; y < y1; ++y) {
    const uint64_t ym = g.row_mask(y, rbits);
    for (int x0 = 0; x0 < g.W; x0 += blockDim.x) {
      const int x = x0 + threadIdx.x;
      const int cov = x < g.W && (ym & span_bits(g.lo(x), g.hi(x, g.Lw))) != 0;
      int tot;
      const int pos = block_excl_scan(cov, sh, tot);
      if (cov) rows[base + pos] = y * g.W + x;
      base += tot;
    }
  }
  if ((int)blockIdx.x == G - 1 && threadIdx.x == 0) count[0] = base;
}

// ---- patch table (flux/run_flux.py:340-355 boxes, flux/routing.py:202-315 cores / halos / order) --------------------
struct Box4 { int y0, y1, x0, x1; };

__global__ __launch_bounds__(1024) void route_table_kernel(const uint8_t* __restrict__ sel, int Lh, int Lw,
                                                           int leaf_latent, int halo, int H, int W, int offset,
                                                           int32_t* __restrict__ table, int32_t* __restrict__ counts) {
  __shared__ int sh[32];
  __shared__ Box4 core[kMaxBoxes];
  __shared__ int key[kMaxBoxes];        // (outer h) * 65536 + (outer w); -1 for a repeated core
  __shared__ int first[kMaxBoxes];      // 1 when no earlier kept box has the same shape
  __shared__ int area[kMaxBoxes];       // in extraction order
  __shared__ uint8_t sm[32768];         // the leaf mask (Lh * Lw <= 32768)
  const int tid = threadIdx.x;
  for (int i = tid; i < Lh * Lw; i += blockDim.x) sm[i] = sel[i];
  __syncthreads();

  // 1. row-run boxes: runs per leaf row, their offsets, then the boxes in the reference's order (rows, then runs)
  int runs = 0;
  if (tid < Lh) {
    for (int j = 0; j < Lw; ++j)
      if (sm[tid * Lw + j] && (j == 0 || !sm[tid * Lw + j - 1])) ++runs;
  }
  int nb;
  const int rb = block_excl_scan(runs, sh, nb);
  if (tid < Lh) {
    int b = rb;
    for (int j = 0; j < Lw;) {
      if (!sm[tid * Lw + j]) { ++j; continue; }
      const int js = j;
      while (j < Lw && sm[tid * Lw + j]) ++j;
      // latent box (i L, (i + 1) L, js L, j L) -> packed-token core (flux/routing.py:228-232)
      const int y0 = tid * leaf_latent, y1 = (tid + 1) * leaf_latent, x0 = js * leaf_latent, x1 = j * leaf_latent;
      if (b < kMaxBoxes)
        core[b] = Box4{(y0 + offset) / 2, (y1 + offset + 1) / 2, (x0 + offset) / 2, (x1 + offset + 1) / 2};
      ++b;
    }
  }
  __syncthreads();
  nb = min(nb, kMaxBoxes);

  // 2. repeated cores are skipped (flux/routing.py:276-278); shape of the dilated, clamped box (:235-244)
  for (int b = tid; b < nb; b += blockDim.x) {
    const Box4 c = core[b];
    bool dup = false;
    for (int q = 0; q < b && !dup; ++q) {
      const Box4 d = core[q];
      dup = d.y0 == c.y0 && d.y1 == c.y1 && d.x0 == c.x0 && d.x1 == c.x1;
    }
    const int oh = min(H, c.y1 + halo) - max(0, c.y0 - halo), ow = min(W, c.x1 + halo) - max(0, c.x0 - halo);
    key[b] = dup ? -1 : oh * 65536 + ow;
  }
  __syncthreads();
  for (int b = tid; b < nb; b += blockDim.x) {
    const int k = key[b];
    int f = k >= 0;
    for (int q = 0; q < b && f; ++q) f = key[q] != k;
    first[b] = f;
  }
  __syncthreads();

  // 3. extraction order: stable by shape (flux/routing.py:303 sorted(by_shape), insertion order inside a shape)
  for (int b = tid; b < nb; b += blockDim.x) {
    const int k = key[b];
    if (k < 0) continue;
    int r = 0, bucket = 0;
    for (int q = 0; q < nb; ++q) {
      const int kq = key[q];
      if (kq < 0) continue;
      r += kq < k || (kq == k && q < b);
      bucket += first[q] && kq < k;
    }
    const Box4 c = core[b];
    const int oy0 = max(0, c.y0 - halo), oy1 = min(H, c.y1 + halo);
    const int ox0 = max(0, c.x0 - halo), ox1 = min(W, c.x1 + halo);
    int32_t* e = table + (int64_t)r * kTableStride;
    e[0] = oy0; e[1] = oy1; e[2] = ox0; e[3] = ox1;
    e[4] = c.y0; e[5] = c.y1; e[6] = c.x0; e[7] = c.x1;
    e[9] = b; e[10] = bucket; e[11] = 0;
    area[r] = (oy1 - oy0) * (ox1 - ox0);
  }
  int kept = 0, buckets = 0;
  for (int b = tid; b < nb; b += blockDim.x) {
    kept += key[b] >= 0;
    buckets += first[b];
  }
  int np, nbk;
  block_excl_scan(kept, sh, np);
  block_excl_scan(buckets, sh, nbk);   // (barriers inside also order the area[] writes)

  // 4. first row of every patch: exclusive scan of the areas, two patches per thread
  const int a0 = 2 * tid < np ? area[2 * tid] : 0, a1 = 2 * tid + 1 < np ? area[2 * tid + 1] : 0;
  int total;
  const int o = block_excl_scan(a0 + a1, sh, total);
  if (2 * tid < np) table[(int64_t)(2 * tid) * kTableStride + 8] = o;
  if (2 * tid + 1 < np) table[(int64_t)(2 * tid + 1) * kTableStride + 8] = o + a0;
  if (tid == 0) {
    counts[0] = np;
    counts[1] = total;
    counts[2] = nbk;
    counts[3] = 0;
  }
}

// Row list in extraction order: patch p's rows are (oy0 + u) * W + ox0 + v, row-major over (u, v)
// (flux/routing.py:286-288 slices the [H, W] grid and reshapes the patch to rows).
__global__ __launch_bounds__(256) void route_rows_kernel(const int32_t* __restrict__ table,
                                                         int32_t* __restrict__ counts, int W,
                                                         int32_t* __restrict__ rows, int64_t max_rows) {
  const int np = counts[0];
  for (int p = blockIdx.x; p < np; p += gridDim.x) {
    const int32_t* e = table + (int64_t)p * kTableStride;
    const int oy0 = e[0], ox0 = e[2], ow = e[3] - e[2], n = (e[1] - e[0]) * ow;
    const int64_t off = e[8];
    if (off + n > max_rows) {
      if (threadIdx.x == 0) atomicOr(counts + 3, 1);
      continue;
    }
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
      const int u = t / ow;
      rows[off + t] = (oy0 + u) * W + ox0 + (t - u * ow);
    }
  }
}

// ---- row gather with a device-side count -----------------------------------------------------------------------
// dst row r = src row rows[r] for r < min(*count, n_max), in units of T (16 bytes when rows, strides and pointers
// allow, else 4 bytes): the patch extraction of hidden_states / img_ids, flux/routing.py:286-296.
template <typename T>
__global__ __launch_bounds__(256) void gather_rows_kernel(const T* __restrict__ src, int64_t ld_src,
                                                          const int32_t* __restrict__ rows,
                                                          const int32_t* __restrict__ count, int64_t n_max,
                                                          int row_dw, T* __restrict__ dst, int64_t ld_dst) {
  const int64_t n = min((int64_t)count[0], n_max);
  const int64_t total = n * row_dw;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / row_dw;
    const int c = (int)(i - r * row_dw);
    dst[r * ld_dst + c] = src[(int64_t)rows[r] * ld_src + c];
  }
}

// ---- feathered fusion (flux/routing.py:328-379) ---------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float round16(float v) {
  const uint32_t b = f32_to_16_bits<DT>(v);
  return DT == PQ_BF16 ? __uint_as_float(b << 16) : lo16_to_f32<DT>(b);
}

// 1-D feather weight of position u in a patch of extent n whose core is [i0, i1): 1 inside the core, the ramp
// tables across the halo (halo_feather_mask, flux/routing.py:46-71). ramp[2 (m (m - 1) / 2 + u) + {0, 1}] holds
// the rising / falling ramp of length m.
__device__ __forceinline__ float edge_weight(int u, int n, int i0, int i1, const float* ramp) {
  if (u < i0) return ramp[2 * (i0 * (i0 - 1) / 2 + u)];
  if (u >= i1) {
    const int m = n - i1;
    return ramp[2 * (m * (m - 1) / 2 + (u - i1)) + 1];
  }
  return 1.0f;
}

constexpr int kMaxFuseHalo = 64;   // ramp table in LDS: halo (halo + 1) floats

// One thread per (token, 8 channels), 32 tokens per workgroup. The workgroup first compacts, in table order, the
// patches whose halo box meets its token span (a block scan over the table), then every thread walks that short
// list: for each patch covering its token it queues the 16-bit beta and the row of the prediction, and the
// predictions of up to 4 queued patches are loaded together before they are accumulated in order.
// Arithmetic, in the 16-bit type with one rounding per torch op: beta = (fusion_beta * mask).clamp(0, 1);
// local += beta * out; beta_acc += beta; then
// out = (1 - clamp(beta_acc, 0, 1)) * bg + clamp(beta_acc, 0, 1) * where(beta_acc > 0, local / beta_acc, 0).
template <int DT>
__global__ __launch_bounds__(256) void fuse_patches_kernel(const uint16_t* __restrict__ bg, int64_t ldb,
                                                           const uint16_t* __restrict__ pout, int64_t ldp,
                                                           const int32_t* __restrict__ table,
                                                           const int32_t* __restrict__ counts,
                                                           const float* __restrict__ ramp, int halo,
                                                           float fusion_beta, int H, int W, int C,
                                                           uint16_t* __restrict__ out, int64_t ldo) {
  __shared__ int sh[32];
  __shared__ int plist[256];
  extern __shared__ float sramp[];   // halo (halo + 1) floats, sized at launch
  const int nch = C / 8;
  const int64_t n = (int64_t)H * W * nch;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = i < n;
  const int tok = live ? (int)(i / nch) : 0, ch = live ? (int)(i - (int64_t)tok * nch) * 8 : 0;
  const int y = tok / W, x = tok - y * W;
  v4u b = {0u, 0u, 0u, 0u};
  if (live) b = *reinterpret_cast<const v4u*>(bg + (int64_t)tok * ldb + ch);   // in flight during the scan
  for (int k = threadIdx.x; k < halo * (halo + 1); k += blockDim.x) sramp[k] = ramp[k];

  // token span of this workgroup
  const int64_t g0 = (int64_t)blockIdx.x * blockDim.x;
  const int t_first = (int)(g0 / nch), t_last = (int)((min(g0 + (int64_t)blockDim.x, n) - 1) / nch);
  const int yf = t_first / W, yl = t_last / W;
  const int xf = yf == yl ? t_first - yf * W : 0, xl = yf == yl ? t_last - yl * W : W - 1;

  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float bacc = 0.0f;
  float qb[4] = {0.f, 0.f, 0.f, 0.f};
  int64_t qo[4] = {0, 0, 0, 0};
  int nq = 0;
  auto flush = [&]() {
    v4u o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < nq) o[k] = *reinterpret_cast<const v4u*>(pout + qo[k] * ldp + ch);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k >= nq) break;
      const uint32_t ow[4] = {o[k].x, o[k].y, o[k].z, o[k].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[2 * c] = round16<DT>(acc[2 * c] + round16<DT>(qb[k] * lo16_to_f32<DT>(ow[c])));
        acc[2 * c + 1] = round16<DT>(acc[2 * c + 1] + round16<DT>(qb[k] * hi16_to_f32<DT>(ow[c])));
      }
      bacc = round16<DT>(bacc + qb[k]);
    }
    nq = 0;
  };

  const int np = counts[0];
  for (int base = 0; base < np; base += blockDim.x) {
    const int p = base + threadIdx.x;
    int hit = 0;
    if (p < np) {
      const int32_t* e = table + (int64_t)p * kTableStride;
      hit = !(e[0] > yl || e[1] <= yf || e[2] > xl || e[3] <= xf);
    }
    int nhit;
    const int pos = block_excl_scan(hit, sh, nhit);   // its barriers also publish sramp
    if (hit) plist[pos] = p;
    __syncthreads();
    for (int k = 0; k < nhit; ++k) {
      const int32_t* e = table + (int64_t)__builtin_amdgcn_readfirstlane(plist[k]) * kTableStride;
      const int oy0 = e[0], oy1 = e[1], ox0 = e[2], ox1 = e[3];
      if (!live || y < oy0 || y >= oy1 || x < ox0 || x >= ox1) continue;
      const int ph = oy1 - oy0, pw = ox1 - ox0, u = y - oy0, v = x - ox0;
      const float wy = edge_weight(u, ph, e[4] - oy0, e[5] - oy0, sramp);
      const float wx = edge_weight(v, pw, e[6] - ox0, e[7] - ox0, sramp);
      const float m = round16<DT>(fminf(fmaxf(fminf(wy, wx), 0.0f), 1.0f));   // mask.clamp(0, 1).to(dtype)
      const float beta = fminf(fmaxf(round16<DT>(fusion_beta * m), 0.0f), 1.0f);
      const int64_t row = (int64_t)e[8] + (int64_t)u * pw + v;
      qb[0] = nq == 0 ? beta : qb[0]; qo[0] = nq == 0 ? row : qo[0];
      qb[1] = nq == 1 ? beta : qb[1]; qo[1] = nq == 1 ? row : qo[1];
      qb[2] = nq == 2 ? beta : qb[2]; qo[2] = nq == 2 ? row : qo[2];
      qb[3] = nq == 3 ? beta : qb[3]; qo[3] = nq == 3 ? row : qo[3];
      if (++nq == 4) flush();
    }
    __syncthreads();   // plist is rewritten by the next round
  }
  if (nq) flush();
  if (!live) return;
  const float bm = fminf(fmaxf(bacc, 0.0f), 1.0f);
  const float den = fmaxf(bacc, round16<DT>(1e-8f));
  const float keep = round16<DT>(1.0f - bm);
  const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
  uint32_t r[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float res[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float bgv = h ? hi16_to_f32<DT>(bw[k]) : lo16_to_f32<DT>(bw[k]);
      const float comb = bacc > 0.0f ? round16<DT>(acc[2 * k + h] / den) : 0.0f;
      res[h] = round16<DT>(round16<DT>(keep * bgv) + round16<DT>(bm * comb));
    }
    r[k] = f32_to_16_bits<DT>(res[0]) | (f32_to_16_bits<DT>(res[1]) << 16);
  }
  *reinterpret_cast<v4u*>(out + (int64_t)tok * ldo + ch) = v4u{r[0], r[1], r[2], r[3]};
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace pq

using namespace pq;

extern "C" int pq_route_union_rows(const uint8_t* sel, int64_t Lh, int64_t Lw, int64_t leaf_tokens, int64_t halo,
                                   int64_t H, int64_t W, int32_t* rows, int32_t* count, hipStream_t stream) {
  if (!sel || !rows || !count) return set_error(PQ_EINVAL, "pq_route_union_rows: null pointer");
  if (Lh <= 0 || Lw <= 0 || leaf_tokens <= 0 || halo < 0 || H <= 0 || W <= 0 || H * W > (1LL << 30))
    return set_error(PQ_ESHAPE, "pq_route_union_rows: bad geometry Lh=%lld Lw=%lld leaf=%lld halo=%lld H=%lld W=%lld",
                     (long long)Lh, (long long)Lw, (long long)leaf_tokens, (long long)halo, (long long)H, (long long)W);
  if (Lw > 64 || Lh > 1024 || Lh * Lw > 32768)
    return set_error(PQ_ESHAPE, "pq_route_union_rows: leaf grid %lldx%lld (at most 64 columns, 1024 rows, 32768 "
                     "leaves)", (long long)Lh, (long long)Lw);
  if (Lh * leaf_tokens > H || Lw * leaf_tokens > W)
    return set_error(PQ_ESHAPE, "pq_route_union_rows: leaf grid %lldx%lld of %lld tokens exceeds the %lldx%lld grid",
                     (long long)Lh, (long long)Lw, (long long)leaf_tokens, (long long)H, (long long)W);
  const UnionGeom g{(int)Lh, (int)Lw, (int)leaf_tokens, (int)halo, (int)H, (int)W};
  hipLaunchKernelGGL(route_union_kernel, dim3((unsigned)std::min<int64_t>(H, 256)), dim3(256), 0, stream, sel, g,
                     rows, count);
  return check_launch("route_union");
}

extern "C" int pq_route_patches(const uint8_t* sel, int64_t Lh, int64_t Lw, int64_t leaf_latent, int64_t halo,
                                int64_t H, int64_t W, int64_t packing_offset, int32_t* table, int32_t* counts,
                                int32_t* rows, int64_t max_rows, hipStream_t stream) {
  if (!sel || !table || !counts || (!rows && max_rows > 0)) return set_error(PQ_EINVAL, "pq_route_patches: null pointer");
  if (Lh <= 0 || Lw <= 0 || Lh > 1024 || Lh * Lw > 32768 || Lh * ((Lw + 1) / 2) > kMaxBoxes || halo < 0 || H <= 0 ||
      W <= 0 ||
      H > 32767 || W > 32767 || max_rows < 0)
    return set_error(PQ_ESHAPE, "pq_route_patches: bad geometry Lh=%lld Lw=%lld halo=%lld H=%lld W=%lld",
                     (long long)Lh, (long long)Lw, (long long)halo, (long long)H, (long long)W);
  if (leaf_latent <= 0 || leaf_latent % 2)
    return set_error(PQ_EINVAL, "pq_route_patches: leaf edge %lld must be positive and even (2x2 packing)",
                     (long long)leaf_latent);
  if (packing_offset != 0 && packing_offset != 1)
    return set_error(PQ_EINVAL, "pq_route_patches: packing offset must be 0 or 1, got %lld", (long long)packing_offset);
  if ((Lh * leaf_latent + packing_offset + 1) / 2 > H || (Lw * leaf_latent + packing_offset + 1) / 2 > W)
    return set_error(PQ_ESHAPE, "pq_route_patches: leaf grid %lldx%lld of %lld latent cells exceeds the %lldx%lld "
                     "token grid", (long long)Lh, (long long)Lw, (long long)leaf_latent, (long long)H, (long long)W);
  hipLaunchKernelGGL(route_table_kernel, dim3(1), dim3(1024), 0, stream, sel, (int)Lh, (int)Lw, (int)leaf_latent,
                     (int)halo, (int)H, (int)W, (int)packing_offset, table, counts);
  int st = check_launch("route_table");
  if (st != PQ_OK || max_rows == 0) return st;
  hipLaunchKernelGGL(route_rows_kernel, dim3(256), dim3(256), 0, stream, table, counts, (int)W, rows, max_rows);
  return check_launch("route_rows");
}

extern "C" int pq_gather_rows(const void* src, int64_t ld_src_bytes, const int32_t* rows, const int32_t* count,
                              int64_t n_max, int64_t row_bytes, void* dst, int64_t ld_dst_bytes, hipStream_t stream) {
  if (!src || !rows || !count || !dst) return set_error(PQ_EINVAL, "pq_gather_rows: null pointer");
  if (row_bytes <= 0 || row_bytes % 4 || ld_src_bytes % 4 || ld_dst_bytes % 4 || ld_src_bytes < row_bytes ||
      ld_dst_bytes < row_bytes || n_max < 0)
    return set_error(PQ_EALIGN, "pq_gather_rows: row bytes %lld and strides %lld / %lld must be multiples of 4",
                     (long long)row_bytes, (long long)ld_src_bytes, (long long)ld_dst_bytes);
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 3)
    return set_error(PQ_EALIGN, "pq_gather_rows: pointers must be 4-byte aligned");
  if (n_max == 0) return PQ_OK;
  const bool wide = row_bytes % 16 == 0 && ld_src_bytes % 16 == 0 && ld_dst_bytes % 16 == 0 && aligned16(src) &&
                    aligned16(dst);
  const int unit = wide ? 16 : 4;
  const int64_t work = n_max * (row_bytes / unit);
  const unsigned grid = (unsigned)std::min<int64_t>((work + 255) / 256, 4096);
  if (wide)
    hipLaunchKernelGGL(gather_rows_kernel<v4u>, dim3(grid), dim3(256), 0, stream, (const v4u*)src, ld_src_bytes / 16,
                       rows, count, n_max, (int)(row_bytes / 16), (v4u*)dst, ld_dst_bytes / 16);
  else
    hipLaunchKernelGGL(gather_rows_kernel<uint32_t>, dim3(grid), dim3(256), 0, stream, (const uint32_t*)src,
                       ld_src_bytes / 4, rows, count, n_max, (int)(row_bytes / 4), (uint32_t*)dst, ld_dst_bytes / 4);
  return check_launch("gather_rows");
}

extern "C" int pq_fuse_patches(const void* background, int64_t ldb, const void* patch_out, int64_t ldp,
                               const int32_t* table, const int32_t* counts, const float* ramp, int64_t halo,
                               float fusion_beta,
                               int64_t H, int64_t W, int64_t C, int32_t dtype, void* out, int64_t ldo,
                               hipStream_t stream) {
  if (!background || !table || !counts || !ramp || !out || !patch_out)
    return set_error(PQ_EINVAL, "pq_fuse_patches: null pointer");
  if (!(fusion_beta >= 0.0f && fusion_beta <= 1.0f))
    return set_error(PQ_EINVAL, "pq_fuse_patches: fusion_beta must be in [0,1], got %g", (double)fusion_beta);
  if (H <= 0 || W <= 0 || C <= 0 || C % 8 || ldb < C || ldo < C || ldp < C || H * W > (1LL << 30) ||
      H * W * (C / 8) > (1LL << 40))
    return set_error(PQ_ESHAPE, "pq_fuse_patches: bad shape H=%lld W=%lld C=%lld (C must be a multiple of 8)",
                     (long long)H, (long long)W, (long long)C);
  if (ldb % 8 || ldp % 8 || ldo % 8 || !aligned16(background) || !aligned16(patch_out) || !aligned16(out))
    return set_error(PQ_EALIGN, "pq_fuse_patches: 16-byte aligned rows required");
  if (dtype != PQ_BF16 && dtype != PQ_F16) return set_error(PQ_EDTYPE, "pq_fuse_patches: dtype %d", dtype);
  if (halo < 0 || halo > kMaxFuseHalo)
    return set_error(PQ_EINVAL, "pq_fuse_patches: halo %lld outside [0, %d]", (long long)halo, kMaxFuseHalo);
  const int64_t n = H * W * (C / 8);
  if (const int st = check_grid((n + 255) / 256, 256, "pq_fuse_patches")) return st;
  const dim3 grid((unsigned)((n + 255) / 256));
  const size_t lds = sizeof(float) * (size_t)std::max<int64_t>(halo * (halo + 1), 1);
  if (dtype == PQ_BF16)
    hipLaunchKernelGGL(fuse_patches_kernel<PQ_BF16>, grid, dim3(256), lds, stream, (const uint16_t*)background, ldb,
                       (const uint16_t*)patch_out, ldp, table, counts, ramp, (int)halo, fusion_beta, (int)H, (int)W, (int)C,
                       (uint16_t*)out, ldo);
  else
    hipLaunchKernelGGL(fuse_patches_kernel<PQ_F16>, grid, dim3(256), lds, stream, (const uint16_t*)background, ldb,
                       (const uint16_t*)patch_out, ldp, table, counts, ramp, (int)halo, fusion_beta, (int)H, (int)W, (int)C,
                       (uint16_t*)out, ldo);
  return check_launch("fuse_patches");
}
