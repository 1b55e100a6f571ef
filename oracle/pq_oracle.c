/*
 * pq_oracle.c -- CPU restatement of PyraQuant's INT8 deployment hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker of the HIP library, never part of it: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py load it. The product path
 * (pyraquant_amd) never calls into it and has no CPU fallback.
 *
 * Every function cites the reference lines it restates (paths relative to the PyraQuant repository).
 * Floating point: plain IEEE-754 binary32 arithmetic in source order (built with -O2 -ffp-contract=off,
 * no fast-math, SSE on x86-64), round-to-nearest-even; nearbyintf() is round half to even, the rounding
 * of torch.round.
 *
 * Each function is pinned by checks that do not restate it (tests/test_oracle_cpu.py): golden fixtures computed by
 * torch's CPU operators on the reference's torch lines (tests/golden/), torch._int_mm, exact-rational and float64
 * arithmetic, closed-form special cases and invariants. lowrank_down is pinned only to a tolerance (the
 * reference's library GEMM fixes no accumulation order).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define PQO_BF16 0
#define PQO_F16 1

/* ---- 16-bit float helpers ------------------------------------------------------------------------------ */
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float half_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: value = man * 2^-24 exactly */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

static uint16_t f32_to_half(float f) {
  /* round to nearest even, overflow to inf, NaN -> quiet NaN */
  const uint32_t u = f2u(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (au >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);        /* >= 65520 rounds to inf */
  if (au < 0x38800000u) {                                           /* below 2^-14: subnormal half */
    const float a = u2f(au);
    const float scaled = a * 16777216.0f;                           /* exact: a * 2^24 */
    const float r = nearbyintf(scaled);                             /* half-even to an integer count */
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t mant = au & 0x7fffffu;
  uint32_t e = (au >> 23) - 112u;
  uint32_t h = (e << 10) | (mant >> 13);
  const uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static inline float to_f32(uint16_t b, int dtype) {
  return dtype == PQO_BF16 ? u2f((uint32_t)b << 16) : half_to_f32(b);
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline uint16_t from_f32(float f, int dtype) { return dtype == PQO_BF16 ? f32_to_bf16(f) : f32_to_half(f); }

void pqo_to_f32(const uint16_t* in, int dtype, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = to_f32(in[i], dtype);
}
void pqo_from_f32(const float* in, int dtype, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = from_f32(in[i], dtype);
}

/* ---- A. per-token activation quantizer ------------------------------------------------------------------
 * deploy/int8_exec.py:508-509 (torch twin of _quant_rows_kernel :78-101; QDQ twin pyraquant/quant_unet.py:52-54):
 *   sc = |x|.amax(1).clamp_min(1e-8) / 127 ; q = round(x / sc).clamp(-127, 127)
 * Source row r = row_idx ? row_idx[m] : m (the routed gather). */
void pqo_quant_rows(const uint16_t* x, int dtype, int64_t M, int64_t K, int64_t ldx, const int32_t* row_idx,
                    int8_t* q, float* s) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const int64_t r = row_idx ? (int64_t)row_idx[m] : m;
    const uint16_t* xr = x + r * ldx;
    float a = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float v = fabsf(to_f32(xr[k], dtype));
      if (v > a) a = v;
    }
    if (a < 1e-8f) a = 1e-8f;
    const float sc = a / 127.0f;
    for (int64_t k = 0; k < K; ++k) {
      float v = nearbyintf(to_f32(xr[k], dtype) / sc);
      if (v > 127.0f) v = 127.0f;
      if (v < -127.0f) v = -127.0f;
      q[m * K + k] = (int8_t)v;
    }
    s[m] = sc;
  }
}

/* ---- B / G. weight RTN ----------------------------------------------------------------------------------
 * per-channel (group == 0): deploy/int8_exec.py:355-357
 *   s = |w|.amax(1).clamp_min(1e-8) / 127 ; q = round(w / s).clamp(-127, 127)
 * group-g (g | K): pyraquant/quantizers_weight.py:96-109 (qdq_weight with w_bits = 8, group_size = g)
 *   scale[n, j] = |w[n, j*g:(j+1)*g]|.amax().clamp_min(1e-8) / 127 ; q = round(w / scale).clamp(-127, 127)
 * s layout: [N] (per-channel) or [N, K/g] (the reference's [out, in/g] layout). */
void pqo_quant_weight(const float* w, int64_t N, int64_t K, int64_t group, int8_t* q, float* s) {
  const int64_t g = group > 0 ? group : K;
  const int64_t G = K / g;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t j = 0; j < G; ++j) {
      const float* wr = w + n * K + j * g;
      float a = 0.0f;
      for (int64_t k = 0; k < g; ++k) {
        const float v = fabsf(wr[k]);
        if (v > a) a = v;
      }
      if (a < 1e-8f) a = 1e-8f;
      const float sc = a / 127.0f;
      for (int64_t k = 0; k < g; ++k) {
        float v = nearbyintf(wr[k] / sc);
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        q[n * K + j * g + k] = (int8_t)v;
      }
      s[n * G + j] = sc;
    }
  }
}

/* ---- C. int32 accumulator: acc[m, n] = sum_k a[m, k] * w[n, k] ------------------------------------------
 * deploy/int8_exec.py:259 (torch._int_mm(xq, w_int8.t())) and the K loop of :168-173. Exact integers. */
void pqo_gemm_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c, int64_t M, int64_t N,
                  int64_t K) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const int8_t* ar = a + m * lda;
    for (int64_t n = 0; n < N; ++n) {
      const int8_t* wr = w + n * ldw;
      int32_t acc = 0;
      for (int64_t k = 0; k < K; ++k) acc += (int32_t)ar[k] * (int32_t)wr[k];
      c[m * N + n] = acc;
    }
  }
}

/* Group-32 partial accumulators: part[m, n, j] = sum_{k in group j} a[m, k] * w[n, k] (exact). */
void pqo_gemm_group_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t group, int32_t* part,
                        int64_t M, int64_t N, int64_t K) {
  const int64_t G = K / group;
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      for (int64_t j = 0; j < G; ++j) {
        int32_t acc = 0;
        for (int64_t k = j * group; k < (j + 1) * group; ++k) acc += (int32_t)a[m * lda + k] * (int32_t)w[n * ldw + k];
        part[(m * N + n) * G + j] = acc;
      }
    }
  }
}

/* ---- E. low-rank down-projection: t = bf16(x @ L1), fp32 accumulation in k order ----------------------
 * deploy/int8_exec.py:390 (t = x2.to(lr_A.dtype) @ lr_A). L1 is [K, R] row-major (the reference layout).
 * The accumulation order of the reference's library GEMM is not fixed; comparisons use a tolerance. */
void pqo_lowrank_down(const uint16_t* x, int dtype, int64_t M, int64_t K, int64_t ldx, const int32_t* row_idx,
                      const uint16_t* l1, int64_t R, uint16_t* t) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const int64_t r = row_idx ? (int64_t)row_idx[m] : m;
    for (int64_t j = 0; j < R; ++j) {
      float acc = 0.0f;
      for (int64_t k = 0; k < K; ++k) acc += to_f32(x[r * ldx + k], dtype) * to_f32(l1[k * R + j], dtype);
      t[m * R + j] = from_f32(acc, dtype);
    }
  }
}

/* ---- C / D / G epilogue: fp32 result before the 16-bit rounding ------------------------------------------
 * per-channel (group == 0): y = (float)acc * (s_row[m] * s_w[n])          deploy/int8_exec.py:176 / :303 / :120
 * group-g               : y = s_row[m] * fma-sum_j s_w[n, j] * (float)part  (sequential j, fmaf)
 * low-rank (t != NULL)  : y = y + sum_r (float)t[m, r] * (float)l2[r, n]     deploy/int8_exec.py:304-307
 * bias (bias != NULL)   : y = y + bias[n]                                     deploy/int8_exec.py:178 / :308-309
 * acc is [M, N] int32 (group == 0) or part [M, N, K/g] (group > 0); s_w is [N] or [N, K/g];
 * l2 is [R, N] (the reference's lr_B layout); t is [M, R] 16-bit of lr_dtype. */
void pqo_epilogue_f32(const int32_t* acc, int64_t group, int64_t G, const float* s_row, const float* s_w,
                      const float* bias, const uint16_t* t, const uint16_t* l2, int64_t R, int lr_dtype, float* y,
                      int64_t M, int64_t N) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      float v;
      if (group == 0) {
        v = (float)acc[m * N + n] * (s_row[m] * s_w[n]);
      } else {
        float sum = 0.0f;
        for (int64_t j = 0; j < G; ++j) sum = fmaf(s_w[n * G + j], (float)acc[(m * N + n) * G + j], sum);
        v = sum * s_row[m];
      }
      if (t) {
        float lr = 0.0f;
        for (int64_t r = 0; r < R; ++r) lr += to_f32(t[m * R + r], lr_dtype) * to_f32(l2[r * N + n], lr_dtype);
        v = v + lr;
      }
      if (bias) v = v + bias[n];
      y[m * N + n] = v;
    }
  }
}

/* ---- I. routed row geometry (config 4): union of halo-dilated active leaves ------------------------------
 * Leaf (i, j) of a (gh x gw) leaf grid covers tokens [i*leaf, (i+1)*leaf) x [j*leaf, (j+1)*leaf) of the
 * (gh*leaf) x (gw*leaf) token grid; it is dilated by `halo` tokens per side and clamped to the grid
 * (flux/routing.py:235-244). Brute force over a boolean canvas; rows are y * W + x, ascending, unique.
 * Returns the row count; rows may be NULL to count only. */
int64_t pqo_route_rows_union(const uint8_t* mask, int64_t gh, int64_t gw, int64_t leaf, int64_t halo, int32_t* rows) {
  const int64_t H = gh * leaf, W = gw * leaf;
  uint8_t* canvas = (uint8_t*)calloc((size_t)(H * W), 1);
  if (!canvas) return -1;
  for (int64_t i = 0; i < gh; ++i)
    for (int64_t j = 0; j < gw; ++j) {
      if (!mask[i * gw + j]) continue;
      for (int64_t y = i * leaf - halo; y < (i + 1) * leaf + halo; ++y)
        for (int64_t x = j * leaf - halo; x < (j + 1) * leaf + halo; ++x)
          if (y >= 0 && y < H && x >= 0 && x < W) canvas[y * W + x] = 1;
    }
  int64_t cnt = 0;
  for (int64_t p = 0; p < H * W; ++p)
    if (canvas[p]) {
      if (rows) rows[cnt] = (int32_t)p;
      ++cnt;
    }
  free(canvas);
  return cnt;
}
