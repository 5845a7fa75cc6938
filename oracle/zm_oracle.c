/*
 * zm_oracle.c -- CPU restatement of ggml's routed-expert MUL_MAT_ID path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never shipped.
 *
 * Pinning status (what fixes each function's output besides this file):
 *   - Q2_K x Q8_K dot: bit-exact against ggml's stock AVX2 kernel as copied in
 *     /root/reference/bench/q2k_dot_bench.cpp:31-63, built into oracle/_ref.
 *   - Q4_K x Q8_K dot: bit-exact against the reference's 512-bit kernel
 *     (bench/q3k_q4k_dot_bench.cpp:73-125, itself checked bit-exact against
 *     ggml's stock at :187-200), built into oracle/_ref.
 *   - Q5_K and Q6_K dots: per-block integer sums pinned against a brute force
 *     over the dequantized weights as below; float order "parity unpinned"
 *     beyond 1e-6 rel (no stock copy of either kernel in the reference tree).
 *   - Q3_K and IQ2_XXS dots: per-block integer sums pinned against a brute
 *     force over the dequantized weights (dequant(w) . dequant(q8) is an
 *     exact integer multiple); float accumulation order follows the AVX2
 *     lane structure of patches/ggml/0009...:34-95 (IQ2_XXS) and the Q2_K
 *     lane structure (Q3_K): float order "parity unpinned" beyond 1e-6 rel.
 *   - Dequant formulas: pinned by round-trip of hand-built blocks and by the
 *     identity dot(dequant(w), dequant(q8)) == block-dot (tests/).
 *   - quantize_row_q8_K: restated from ggml (scale -127/max, round-half-even,
 *     16-element sums); pinned by closed-form cases in tests/ (exact for
 *     hand-picked rows); bit identity with ggml's own build "parity unpinned".
 *   - K-quant / IQ2_XXS weight quantizers: produce valid blocks; ggml's byte
 *     choices are "parity unpinned" (the op is checked on identical bytes).
 *   - IQ4_XS: per-block integer sums pinned by brute force over the dequant
 *     (exact); table values ggml's published kvalues_iq4nl, "parity unpinned"
 *     (not in the reference tree); float order unpinned.
 *   - IQ3_XXS: per-block integer sums pinned by brute force over the dequant;
 *     the grid is a stand-in (ggml's iq3xxs_grid is not in the reference
 *     tree): "parity unpinned" for its values; float order unpinned.
 *   - IQ2_XXS grid: a stand-in table (ggml's 256 x u64 values are not in the
 *     reference tree); the sign table is closed form (0009...:69-75).
 *   - Router, bucketing, SwiGLU, combine: closed forms, brute-force checked.
 */
#include "zm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ helpers */

float zmo_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* IEEE round-to-nearest-even float -> half (what F16C's _cvtss_sh(x, 0) does). */
uint16_t zmo_fp32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf / nan */
    return sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0);
  if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
    return sign | 0x7c00u;
  if (ax < 0x38800000u) { /* result subnormal or zero */
    if (ax < 0x33000000u) return sign; /* < 2^-25: rounds to 0 */
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    /* value = m * 2^(e-150); subnormal unit = 2^-24 -> q = m * 2^(e-126) */
    const uint32_t rshift = 126 - e; /* >= 1 */
    uint32_t q = m >> rshift;
    const uint32_t rem = m & ((1u << rshift) - 1);
    const uint32_t half = 1u << (rshift - 1);
    if (rem > half || (rem == half && (q & 1))) ++q;
    return sign | (uint16_t)q;
  }
  /* normal */
  uint32_t e = (ax >> 23) - 112;
  uint32_t m = ax & 0x7fffffu;
  uint32_t q = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) ++q;
  return sign | (uint16_t)q;
}

size_t zmo_row_size(int type, int64_t n) {
  const int64_t nb = n / ZMO_QK_K;
  switch (type) {
  case ZMO_TYPE_Q2_K: return (size_t)nb * sizeof(zmo_block_q2_K);
  case ZMO_TYPE_Q3_K: return (size_t)nb * sizeof(zmo_block_q3_K);
  case ZMO_TYPE_Q4_K: return (size_t)nb * sizeof(zmo_block_q4_K);
  case ZMO_TYPE_Q5_K: return (size_t)nb * sizeof(zmo_block_q5_K);
  case ZMO_TYPE_Q6_K: return (size_t)nb * sizeof(zmo_block_q6_K);
  case ZMO_TYPE_IQ2_XXS: return (size_t)nb * sizeof(zmo_block_iq2_xxs);
  case ZMO_TYPE_IQ4_XS: return (size_t)nb * sizeof(zmo_block_iq4_xs);
  case ZMO_TYPE_IQ3_XXS: return (size_t)nb * sizeof(zmo_block_iq3_xxs);
  case ZMO_TYPE_Q8_K: return (size_t)nb * sizeof(zmo_block_q8_K);
  case ZMO_TYPE_F32: return (size_t)n * 4;
  default: return 0;
  }
}

/* ggml-quants.c nearest_int: adding 1.5*2^23 rounds half to even. */
int zmo_nearest_int(float fval) {
  float val = fval + 12582912.f;
  int i;
  memcpy(&i, &val, sizeof(int));
  return (i & 0x007fffff) - 0x00400000;
}

/* exp(x): Cody-Waite reduction by ln2 (two-part constant) and a degree-7
 * Taylor polynomial on |r| <= ln2/2 (truncation < 4e-9 relative), scaled by
 * 2^n.  Every step is an IEEE add/mul/fma, so the HIP library's copy of this
 * function returns the same bits. */
float zmo_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.972084045410156f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412701138295233249664306640625e-4f; /* 1/5040 */
  p = fmaf(p, r, 1.388888922519981861114501953125e-3f); /* 1/720 */
  p = fmaf(p, r, 8.33333376795053482055664062500e-3f);  /* 1/120 */
  p = fmaf(p, r, 4.16666679084300994873046875000e-2f);  /* 1/24 */
  p = fmaf(p, r, 1.66666671633720397949218750000e-1f);  /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

static uint64_t splitmix64(uint64_t *s) {
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

/* Portable seeded normals: splitmix64 uniforms + Box-Muller (both outputs).
 * splitmix64's state after c calls is seed + c * gamma, so pair p (outputs
 * 2p, 2p+1) starts from seed + 2p * gamma: the pairs are independent and are
 * filled in parallel, with the same values as the sequential recurrence. */
void zmo_fill_normal(uint64_t seed, float mean, float sd, float *out, int64_t n) {
  const int64_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static) if (pairs > 65536)
  for (int64_t p = 0; p < pairs; ++p) {
    uint64_t s = seed + (uint64_t)(2 * p) * 0x9e3779b97f4a7c15ull;
    const double u1 = ((splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740993.0);
    const double u2 = (splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586476925286766559 * u2;
    out[2 * p] = (float)(mean + sd * r * cos(t));
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + sd * r * sin(t));
  }
}

/* ------------------------------------------------------------ IQ2_XXS tables */

/* ksigns_iq2xs[i] = i | parity(i) << 7: the 8th sign keeps the count of
 * negative signs even (patches/ggml/0009...:69-75 computes exactly this). */
uint8_t zmo_ksigns_iq2xs(int i) {
  int p = __builtin_popcount((unsigned)i & 127u) & 1;
  return (uint8_t)((i & 127) | (p << 7));
}

/* Stand-in grid: the 256 vectors v in {1,3,5}^8 with sum(v) = 0 mod 4 of
 * smallest norm (ties: lexicographic, coordinate 0 most significant), each
 * coordinate stored as one byte 1->0x08, 3->0x19, 5->0x2b (the byte values
 * ggml's grid uses).  ggml's own table is a different selection of such
 * vectors and is loaded at run time by callers that have it. */
void zmo_iq2xxs_standin_grid(uint64_t grid[256]) {
  static const uint8_t bytev[3] = {0x08, 0x19, 0x2b};
  /* enumerate 3^8 = 6561 digit vectors; keep sum-of-digits even */
  int count = 0;
  for (int norm = 0; norm < 200 && count < 256; ++norm) {
    for (int idx = 0; idx < 6561 && count < 256; ++idx) {
      int t = idx, dig[8], sd = 0, nn = 0;
      for (int j = 7; j >= 0; --j) {
        dig[j] = t % 3;
        t /= 3;
      }
      for (int j = 0; j < 8; ++j) {
        const int v = 1 + 2 * dig[j];
        sd += dig[j];
        nn += v * v;
      }
      if (sd & 1) continue;
      if (nn != norm) continue;
      uint64_t g = 0;
      for (int j = 0; j < 8; ++j) g |= (uint64_t)bytev[dig[j]] << (8 * j);
      grid[count++] = g;
    }
  }
}

static uint64_t g_iq2xxs_grid[256];
static int g_iq2xxs_ready = 0;

const uint64_t *zmo_iq2xxs_grid(void) {
  if (!g_iq2xxs_ready) {
    zmo_iq2xxs_standin_grid(g_iq2xxs_grid);
    g_iq2xxs_ready = 1;
  }
  return g_iq2xxs_grid;
}

void zmo_set_iq2xxs_grid(const uint64_t grid[256]) {
  memcpy(g_iq2xxs_grid, grid, sizeof(g_iq2xxs_grid));
  g_iq2xxs_ready = 1;
}

/* ------------------------------------------------------------ IQ4_XS table */

static int8_t g_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

const int8_t *zmo_iq4nl_table(void) { return g_iq4nl; }
void zmo_set_iq4nl_table(const int8_t table[16]) { memcpy(g_iq4nl, table, 16); }

/* ----------------------------------------------------------- IQ3_XXS grid */

/* Stand-in grid: the 256 vectors of four 3-bit digits d with
 * d0 + 2 d1 + 4 d2 + 8 d3 = 0 mod 16 (one in 16 of the 4096 digit vectors,
 * spread evenly), in increasing order of d0 + 8 d1 + 64 d2 + 512 d3, each digit stored
 * as one byte 4 + 8 d (62 for d = 7): the byte levels ggml's grid uses.
 * ggml's own table is a different selection and is loaded at run time by
 * callers that have it. */
void zmo_iq3xxs_standin_grid(uint32_t grid[256]) {
  static const uint8_t lev[8] = {4, 12, 20, 28, 36, 44, 52, 62};
  int n = 0;
  for (int v = 0; v < 4096 && n < 256; ++v) {
    const int d0 = v & 7, d1 = (v >> 3) & 7, d2 = (v >> 6) & 7, d3 = (v >> 9) & 7;
    if ((d0 + 2 * d1 + 4 * d2 + 8 * d3) % 16) continue;
    grid[n++] = (uint32_t)lev[d0] | ((uint32_t)lev[d1] << 8) | ((uint32_t)lev[d2] << 16) | ((uint32_t)lev[d3] << 24);
  }
}

static uint32_t g_iq3xxs_grid[256];
static int g_iq3xxs_ready = 0;

const uint32_t *zmo_iq3xxs_grid(void) {
  if (!g_iq3xxs_ready) {
    zmo_iq3xxs_standin_grid(g_iq3xxs_grid);
    g_iq3xxs_ready = 1;
  }
  return g_iq3xxs_grid;
}

void zmo_set_iq3xxs_grid(const uint32_t grid[256]) {
  memcpy(g_iq3xxs_grid, grid, sizeof(g_iq3xxs_grid));
  g_iq3xxs_ready = 1;
}

/* ---------------------------------------------------------------- Q8_K quant */

/* ggml quantize_row_q8_K_ref: per 256 values take the signed value of largest
 * magnitude (first one on ties), iscale = -127/max, q = min(127, round(iscale x)),
 * d = 1/iscale, bsums = sums of 16 consecutive q.  The reference restates the
 * same rounding in tests/test_real_tensor_numerics.cpp:115-126 (signed max,
 * scale |max|/127, nearest integer clamped to +-127). */
void zmo_quantize_row_q8_K(const float *x, zmo_block_q8_K *y, int64_t k) {
  const int64_t nb = k / ZMO_QK_K;
  for (int64_t i = 0; i < nb; ++i, x += ZMO_QK_K) {
    float max = 0, amax = 0;
    for (int j = 0; j < ZMO_QK_K; ++j) {
      const float ax = fabsf(x[j]);
      if (ax > amax) {
        amax = ax;
        max = x[j];
      }
    }
    if (amax == 0.0f) {
      y[i].d = 0;
      memset(y[i].qs, 0, sizeof(y[i].qs));
      memset(y[i].bsums, 0, sizeof(y[i].bsums));
      continue;
    }
    const float iscale = -127.f / max;
    for (int j = 0; j < ZMO_QK_K; ++j) {
      const int v = zmo_nearest_int(iscale * x[j]);
      y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < ZMO_QK_K / 16; ++j) {
      int sum = 0;
      for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
      y[i].bsums[j] = (int16_t)sum;
    }
    y[i].d = 1 / iscale;
  }
}

/* ------------------------------------------------------- weight quantizers */

/* Weighted least-squares fit of x ~ scale*L + min with L in [0, nmax],
 * searching nstep+1 candidate inverse scales around nmax/(max-min)
 * (the make_qkx2_quants method of ggml-quants.c). Returns scale; *neg_min
 * receives -min (>= 0). */
static float fit_scale_min(int n, int nmax, const float *x, const float *w, uint8_t *L, float *neg_min,
                           float rmin, float rdelta, int nstep, int use_mad) {
  float mn = x[0], mx = x[0], sw = w[0], sx = w[0] * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < mn) mn = x[i];
    if (x[i] > mx) mx = x[i];
    sw += w[i];
    sx += w[i] * x[i];
  }
  if (mn > 0) mn = 0;
  if (mx == mn) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    *neg_min = -mn;
    return 0.f;
  }
  float iscale = nmax / (mx - mn);
  float scale = 1 / iscale;
  float best = 0;
  for (int i = 0; i < n; ++i) {
    int l = zmo_nearest_int(iscale * (x[i] - mn));
    l = l < 0 ? 0 : (l > nmax ? nmax : l);
    L[i] = (uint8_t)l;
    float diff = scale * l + mn - x[i];
    diff = use_mad ? fabsf(diff) : diff * diff;
    best += w[i] * diff;
  }
  uint8_t aux[32];
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rmin + rdelta * is + nmax) / (mx - mn);
    float sl = 0, sl2 = 0, sxl = 0;
    for (int i = 0; i < n; ++i) {
      int l = zmo_nearest_int(iscale * (x[i] - mn));
      l = l < 0 ? 0 : (l > nmax ? nmax : l);
      aux[i] = (uint8_t)l;
      sl += w[i] * l;
      sl2 += w[i] * l * l;
      sxl += w[i] * l * x[i];
    }
    const float D = sw * sl2 - sl * sl;
    if (D > 0) {
      float ts = (sw * sxl - sx * sl) / D;
      float tm = (sl2 * sx - sl * sxl) / D;
      if (tm > 0) {
        tm = 0;
        ts = sxl / sl2;
      }
      float err = 0;
      for (int i = 0; i < n; ++i) {
        float diff = ts * aux[i] + tm - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        err += w[i] * diff;
      }
      if (err < best) {
        memcpy(L, aux, (size_t)n);
        best = err;
        scale = ts;
        mn = tm;
      }
    }
  }
  *neg_min = -mn;
  return scale;
}

void zmo_quantize_row_q2_K(const float *x, zmo_block_q2_K *y, int64_t k) {
  const int64_t nb = k / ZMO_QK_K;
  uint8_t L[256];
  float w[16], mins[16], scales[16];
  for (int64_t i = 0; i < nb; ++i, x += ZMO_QK_K) {
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 16; ++j) {
      for (int l = 0; l < 16; ++l) w[l] = fabsf(x[16 * j + l]);
      scales[j] = fit_scale_min(16, 3, x + 16 * j, w, L + 16 * j, &mins[j], -0.5f, 0.1f, 15, 1);
      if (scales[j] > max_scale) max_scale = scales[j];
      if (mins[j] > max_min) max_min = mins[j];
    }
    if (max_scale > 0) {
      const float is = 15.f / max_scale;
      for (int j = 0; j < 16; ++j) {
        int l = zmo_nearest_int(is * scales[j]);
        y[i].scales[j] = (uint8_t)(l > 15 ? 15 : l);
      }
      y[i].d = zmo_fp32_to_fp16(max_scale / 15.f);
    } else {
      memset(y[i].scales, 0, 16);
      y[i].d = 0;
    }
    if (max_min > 0) {
      const float is = 15.f / max_min;
      for (int j = 0; j < 16; ++j) {
        int l = zmo_nearest_int(is * mins[j]);
        y[i].scales[j] |= (uint8_t)((l > 15 ? 15 : l) << 4);
      }
      y[i].dmin = zmo_fp32_to_fp16(max_min / 15.f);
    } else {
      y[i].dmin = 0;
    }
    for (int j = 0; j < 16; ++j) {
      const float d = zmo_fp16_to_fp32(y[i].d) * (y[i].scales[j] & 0xF);
      if (d == 0.0f) continue;
      const float dm = zmo_fp16_to_fp32(y[i].dmin) * (y[i].scales[j] >> 4);
      for (int ii = 0; ii < 16; ++ii) {
        int l = zmo_nearest_int((x[16 * j + ii] + dm) / d);
        L[16 * j + ii] = (uint8_t)(l < 0 ? 0 : (l > 3 ? 3 : l));
      }
    }
    for (int j = 0; j < ZMO_QK_K; j += 128)
      for (int l = 0; l < 32; ++l)
        y[i].qs[j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
  }
}

/* symmetric fit with L in [-nmax, nmax-1] and rmse refinement (ggml make_q3_quants) */
static float fit_symmetric(int n, int nmax, const float *x, int8_t *L) {
  float max = 0, amax = 0;
  for (int i = 0; i < n; ++i) {
    const float ax = fabsf(x[i]);
    if (ax > amax) {
      amax = ax;
      max = x[i];
    }
  }
  if (amax < 1e-15f) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  const float iscale = -nmax / max;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = zmo_nearest_int(iscale * x[i]);
    l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
    L[i] = (int8_t)l;
    const float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  for (int itry = 0; itry < 5; ++itry) {
    int changed = 0;
    for (int i = 0; i < n; ++i) {
      const float w = x[i] * x[i];
      float slx = sumlx - w * x[i] * L[i];
      if (slx > 0) {
        float sl2 = suml2 - w * L[i] * L[i];
        int nl = zmo_nearest_int(x[i] * sl2 / slx);
        nl = nl < -nmax ? -nmax : (nl > nmax - 1 ? nmax - 1 : nl);
        if (nl != L[i]) {
          slx += w * x[i] * nl;
          sl2 += w * nl * nl;
          if (sl2 > 0 && slx * slx * suml2 > sumlx * sumlx * sl2) {
            L[i] = (int8_t)nl;
            sumlx = slx;
            suml2 = sl2;
            ++changed;
          }
        }
      }
    }
    if (!changed) break;
  }
  for (int i = 0; i < n; ++i) L[i] = (int8_t)(L[i] + nmax);
  return suml2 > 0 ? sumlx / suml2 : 0.f;
}

void zmo_quantize_row_q3_K(const float *x, zmo_block_q3_K *y, int64_t k) {
  const int64_t nb = k / ZMO_QK_K;
  int8_t L[256];
  float scales[16];
  for (int64_t i = 0; i < nb; ++i, x += ZMO_QK_K) {
    float max_scale = 0, amax = 0;
    for (int j = 0; j < 16; ++j) {
      scales[j] = fit_symmetric(16, 4, x + 16 * j, L + 16 * j);
      const float s = fabsf(scales[j]);
      if (s > amax) {
        amax = s;
        max_scale = scales[j];
      }
    }
    memset(y[i].scales, 0, 12);
    if (max_scale != 0.0f) {
      const float is = -32.f / max_scale;
      for (int j = 0; j < 16; ++j) {
        int l = zmo_nearest_int(is * scales[j]);
        l = (l < -32 ? -32 : (l > 31 ? 31 : l)) + 32;
        if (j < 8) y[i].scales[j] = (uint8_t)(l & 0xF);
        else y[i].scales[j - 8] |= (uint8_t)((l & 0xF) << 4);
        l >>= 4;
        y[i].scales[j % 4 + 8] |= (uint8_t)(l << (2 * (j / 4)));
      }
      y[i].d = zmo_fp32_to_fp16(1 / is);
    } else {
      y[i].d = 0;
    }
    for (int j = 0; j < 16; ++j) {
      int sc = j < 8 ? (y[i].scales[j] & 0xF) : (y[i].scales[j - 8] >> 4);
      sc = (sc | (((y[i].scales[8 + j % 4] >> (2 * (j / 4))) & 3) << 4)) - 32;
      const float d = zmo_fp16_to_fp32(y[i].d) * sc;
      if (d == 0.0f) continue;
      for (int ii = 0; ii < 16; ++ii) {
        int l = zmo_nearest_int(x[16 * j + ii] / d);
        l = l < -4 ? -4 : (l > 3 ? 3 : l);
        L[16 * j + ii] = (int8_t)(l + 4);
      }
    }
    memset(y[i].hmask, 0, 32);
    int m = 0;
    uint8_t hm = 1;
    for (int j = 0; j < ZMO_QK_K; ++j) {
      if (L[j] > 3) {
        y[i].hmask[m] |= hm;
        L[j] -= 4;
      }
      if (++m == 32) {
        m = 0;
        hm <<= 1;
      }
    }
    for (int j = 0; j < ZMO_QK_K; j += 128)
      for (int l = 0; l < 32; ++l)
        y[i].qs[j / 4 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6));
  }
}

/* Q4_K 6-bit scale/min unpack (ggml get_scale_min_k4; kquant_matmul.cu:41-48). */
static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
  }
}

void zmo_quantize_row_q4_K(const float *x, zmo_block_q4_K *y, int64_t k) {
  const int64_t nb = k / ZMO_QK_K;
  uint8_t L[256];
  float w[32], mins[8], scales[8];
  for (int64_t i = 0; i < nb; ++i, x += ZMO_QK_K) {
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
      float s2 = 0;
      for (int l = 0; l < 32; ++l) s2 += x[32 * j + l] * x[32 * j + l];
      const float av = sqrtf(s2 / 32);
      for (int l = 0; l < 32; ++l) w[l] = av + fabsf(x[32 * j + l]);
      scales[j] = fit_scale_min(32, 15, x + 32 * j, w, L + 32 * j, &mins[j], -1.f, 0.1f, 20, 0);
      if (scales[j] > max_scale) max_scale = scales[j];
      if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    memset(y[i].scales, 0, 12);
    for (int j = 0; j < 8; ++j) {
      int ls = zmo_nearest_int(inv_scale * scales[j]);
      int lm = zmo_nearest_int(inv_min * mins[j]);
      ls = ls > 63 ? 63 : ls;
      lm = lm > 63 ? 63 : lm;
      if (j < 4) {
        y[i].scales[j] = (uint8_t)ls;
        y[i].scales[j + 4] = (uint8_t)lm;
      } else {
        y[i].scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        y[i].scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
        y[i].scales[j - 0] |= (uint8_t)((lm >> 4) << 6);
      }
    }
    y[i].d = zmo_fp32_to_fp16(max_scale / 63.f);
    y[i].dmin = zmo_fp32_to_fp16(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
      uint8_t sc, m;
      scale_min_k4(j, y[i].scales, &sc, &m);
      const float d = zmo_fp16_to_fp32(y[i].d) * sc;
      if (d == 0.0f) continue;
      const float dm = zmo_fp16_to_fp32(y[i].dmin) * m;
      for (int ii = 0; ii < 32; ++ii) {
        int l = zmo_nearest_int((x[32 * j + ii] + dm) / d);
        L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : (l > 15 ? 15 : l));
      }
    }
    for (int j = 0; j < ZMO_QK_K; j += 64)
      for (int l = 0; l < 32; ++l) y[i].qs[j / 2 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
  }
}

/* Q5_K: as Q4_K with 5-bit values (0..31): the low nibbles packed as Q4_K's
 * qs, bit 4 of weight 64c + 32g + l in bit 2c + g of qh[l]
 * (dequant at kquant_matmul.cu:94-117). */
void zmo_quantize_row_q5_K(const float *x, zmo_block_q5_K *y, int64_t k) {
  const int64_t nb = k / ZMO_QK_K;
  uint8_t L[256];
  float w[32], mins[8], scales[8];
  for (int64_t i = 0; i < nb; ++i, x += ZMO_QK_K) {
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
      float s2 = 0;
      for (int l = 0; l < 32; ++l) s2 += x[32 * j + l] * x[32 * j + l];
      const float av = sqrtf(s2 / 32);
      for (int l = 0; l < 32; ++l) w[l] = av + fabsf(x[32 * j + l]);
      scales[j] = fit_scale_min(32, 31, x + 32 * j, w, L + 32 * j, &mins[j], -0.5f, 0.1f, 15, 0);
      if (scales[j] > max_scale) max_scale = scales[j];
      if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    memset(y[i].scales, 0, 12);
    for (int j = 0; j < 8; ++j) {
      int ls = zmo_nearest_int(inv_scale * scales[j]);
      int lm = zmo_nearest_int(inv_min * mins[j]);
      ls = ls > 63 ? 63 : ls;
      lm = lm > 63 ? 63 : lm;
      if (j < 4) {
        y[i].scales[j] = (uint8_t)ls;
        y[i].scales[j + 4] = (uint8_t)lm;
      } else {
        y[i].scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        y[i].scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
        y[i].scales[j - 0] |= (uint8_t)((lm >> 4) << 6);
      }
    }
    y[i].d = zmo_fp32_to_fp16(max_scale / 63.f);
    y[i].dmin = zmo_fp32_to_fp16(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
      uint8_t sc, m;
      scale_min_k4(j, y[i].scales, &sc, &m);
      const float d = zmo_fp16_to_fp32(y[i].d) * sc;
      if (d == 0.0f) continue;
      const float dm = zmo_fp16_to_fp32(y[i].dmin) * m;
      for (int ii = 0; ii < 32; ++ii) {
        int l = zmo_nearest_int((x[32 * j + ii] + dm) / d);
        L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : (l > 31 ? 31 : l));
      }
    }
    memset(y[i].qh, 0, 32);
    for (int c = 0; c < 4; ++c)
      for (int l = 0; l < 32; ++l) {
        const int lo = L[64 * c + l], hi = L[64 * c + 32 + l];
        y[i].qs[32 * c + l] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
        y[i].qh[l] |= (uint8_t)(((lo >> 4) << (2 * c)) | ((hi >> 4) << (2 * c + 1)));
      }
  }
}

/* Q6_K: 16 sub-blocks of 16 with a signed 8-bit scale each, values q - 32 for
 * 6-bit q; weight 128h + 32g + l (l < 32) keeps its low nibble in
 * ql[64h + 32(g&1) + l] (high nibble when g >= 2) and its top two bits at
 * bit 2g of qh[32h + l] (dequant at kquant_matmul.cu:119-140). */
void zmo_quantize_row_q6_K(const float *x, zmo_block_q6_K *y, int64_t k) {
  const int64_t nb = k / ZMO_QK_K;
  int8_t L[256];
  float scales[16];
  for (int64_t i = 0; i < nb; ++i, x += ZMO_QK_K) {
    float max_scale = 0, amax = 0;
    for (int j = 0; j < 16; ++j) {
      scales[j] = fit_symmetric(16, 32, x + 16 * j, L + 16 * j);
      const float a = fabsf(scales[j]);
      if (a > amax) {
        amax = a;
        max_scale = scales[j];
      }
    }
    if (max_scale == 0.0f) {
      memset(&y[i], 0, sizeof(y[i]));
      continue;
    }
    const float iscale = -128.f / max_scale;
    y[i].d = zmo_fp32_to_fp16(1 / iscale);
    for (int j = 0; j < 16; ++j) {
      const int l = zmo_nearest_int(iscale * scales[j]);
      y[i].scales[j] = (int8_t)(l > 127 ? 127 : (l < -128 ? -128 : l));
    }
    for (int j = 0; j < 16; ++j) {
      const float d = zmo_fp16_to_fp32(y[i].d) * y[i].scales[j];
      if (d == 0.0f) {
        for (int ii = 0; ii < 16; ++ii) L[16 * j + ii] = 32;
        continue;
      }
      for (int ii = 0; ii < 16; ++ii) {
        int l = zmo_nearest_int(x[16 * j + ii] / d);
        l = l < -32 ? -32 : (l > 31 ? 31 : l);
        L[16 * j + ii] = (int8_t)(l + 32);
      }
    }
    for (int h = 0; h < 2; ++h)
      for (int l = 0; l < 32; ++l) {
        const int q0 = L[128 * h + l], q1 = L[128 * h + 32 + l], q2 = L[128 * h + 64 + l], q3 = L[128 * h + 96 + l];
        y[i].ql[64 * h + l] = (uint8_t)((q0 & 15) | ((q2 & 15) << 4));
        y[i].ql[64 * h + 32 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
        y[i].qh[32 * h + l] = (uint8_t)((q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6));
      }
  }
}

/* IQ2_XXS: per 8-weight group the sign pattern (even count of negatives; on
 * an odd count the smallest-magnitude weight keeps a positive sign) and the
 * nearest grid vector to |x|/scale; per 32-weight sub-block a 4-bit scale
 * ls with value d*(0.5+ls)*0.25; block d in fp16. */
/* gt: the grid as floats, transposed: gt[256 * j + g] = byte j of grid[g].
 * The squared error of every grid point is summed j = 0..7 in order; the
 * points are scanned 8 at a time (8 independent sums, one vector lane each),
 * the first minimum wins. */
__attribute__((optimize("O3"))) static int nearest_grid(const float *a, float inv, const float *gt, float *err_out) {
  float s[8];
  for (int j = 0; j < 8; ++j) s[j] = a[j] * inv;
  int best = 0;
  float be = 3.4e38f;
  for (int g0 = 0; g0 < 256; g0 += 8) {
    float e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < 8; ++j) {
      const float *row = gt + 256 * j + g0;
      for (int q = 0; q < 8; ++q) {
        const float dd = s[j] - row[q];
        e[q] += dd * dd;
      }
    }
    for (int q = 0; q < 8; ++q)
      if (e[q] < be) {
        be = e[q];
        best = g0 + q;
      }
  }
  if (err_out) *err_out = be;
  return best;
}

void zmo_quantize_row_iq2_xxs(const float *x, zmo_block_iq2_xxs *y, int64_t k) {
  float grid[256 * 8];
  {
    const uint64_t *g64 = zmo_iq2xxs_grid();
    for (int g = 0; g < 256; ++g)
      for (int j = 0; j < 8; ++j) grid[256 * j + g] = (float)((g64[g] >> (8 * j)) & 0xff);
  }
  const int64_t nb = k / ZMO_QK_K;
  for (int64_t i = 0; i < nb; ++i, x += ZMO_QK_K) {
    float sub_scale[8];
    float a[256];
    uint8_t sign7[32];
    for (int g = 0; g < 32; ++g) {
      int neg = 0, minj = 0;
      float mina = 3.4e38f;
      for (int j = 0; j < 8; ++j) {
        a[8 * g + j] = fabsf(x[8 * g + j]);
        if (x[8 * g + j] < 0) ++neg;
        if (a[8 * g + j] < mina) {
          mina = a[8 * g + j];
          minj = j;
        }
      }
      uint8_t s = 0;
      for (int j = 0; j < 8; ++j)
        if (x[8 * g + j] < 0) s |= (uint8_t)(1u << j);
      if (neg & 1) s ^= (uint8_t)(1u << minj);
      sign7[g] = s; /* full 8-bit pattern with even parity */
    }
    /* per-sub-block scale in grid units: search candidates around max|a|/43 */
    float max_sub = 0;
    for (int ib = 0; ib < 8; ++ib) {
      float amax = 0;
      for (int j = 0; j < 32; ++j)
        if (a[32 * ib + j] > amax) amax = a[32 * ib + j];
      float best_s = amax / 43.f, best_e = 3.4e38f;
      if (amax > 0) {
        for (int t = 0; t < 8; ++t) {
          const float s = amax / (18.f + 4.f * t);
          float e = 0;
          for (int gg = 0; gg < 4; ++gg) {
            float ge;
            nearest_grid(a + 32 * ib + 8 * gg, 1.f / s, grid, &ge);
            e += ge * s * s;
          }
          if (e < best_e) {
            best_e = e;
            best_s = s;
          }
        }
      }
      sub_scale[ib] = best_s;
      if (best_s > max_sub) max_sub = best_s;
    }
    /* value = d * (0.5 + ls) * 0.25 * grid ; sub scale s = d*(0.5+ls)*0.25 */
    const float d = max_sub / (0.25f * 15.5f);
    y[i].d = zmo_fp32_to_fp16(d);
    const float dq = zmo_fp16_to_fp32(y[i].d);
    for (int ib = 0; ib < 8; ++ib) {
      int ls = 0;
      if (dq > 0) {
        ls = zmo_nearest_int(sub_scale[ib] / (0.25f * dq) - 0.5f);
        ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
      }
      const float s = dq * (0.5f + ls) * 0.25f;
      uint32_t aux0 = 0, aux1 = (uint32_t)ls << 28;
      for (int gg = 0; gg < 4; ++gg) {
        const int gi = s > 0 ? nearest_grid(a + 32 * ib + 8 * gg, 1.f / s, grid, NULL) : 0;
        aux0 |= (uint32_t)gi << (8 * gg);
        aux1 |= (uint32_t)(sign7[4 * ib + gg] & 127u) << (7 * gg);
      }
      y[i].qs[4 * ib + 0] = (uint16_t)(aux0 & 0xffff);
      y[i].qs[4 * ib + 1] = (uint16_t)(aux0 >> 16);
      y[i].qs[4 * ib + 2] = (uint16_t)(aux1 & 0xffff);
      y[i].qs[4 * ib + 3] = (uint16_t)(aux1 >> 16);
    }
  }
}

/* IQ4_XS: per 32-weight sub-block a 6-bit scale ls (value ls - 32) and 4-bit
 * indices into the 16-entry table; weight = d * (ls - 32) * table[idx]
 * (dequant at kernels/quant/iq4xs_matmul.cu:80-99).  The scale of a
 * sub-block maps its largest |x| to the table's largest |value|; the block d
 * fits the largest sub-block scale into ls - 32 in [-32, 31]; indices are
 * the nearest table values under the stored scale. */
static int nearest_iq4(const int8_t *t, float v) {
  int best = 0;
  float be = fabsf(v - t[0]);
  for (int i = 1; i < 16; ++i) {
    const float e = fabsf(v - t[i]);
    if (e < be) {
      be = e;
      best = i;
    }
  }
  return best;
}

void zmo_quantize_row_iq4_xs(const float *x, zmo_block_iq4_xs *y, int64_t k) {
  const int8_t *t = zmo_iq4nl_table();
  int tmax = 0;
  for (int i = 0; i < 16; ++i) tmax = abs(t[i]) > tmax ? abs(t[i]) : tmax;
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i, x += ZMO_QK_K) {
    float sc[8], amax_sc = 0.f;
    for (int ib = 0; ib < 8; ++ib) {
      float amax = 0.f, mx = 0.f;
      for (int j = 0; j < 32; ++j) {
        const float a = fabsf(x[32 * ib + j]);
        if (a > amax) {
          amax = a;
          mx = x[32 * ib + j];
        }
      }
      /* the extreme maps to -tmax (the table's most negative value) */
      sc[ib] = amax > 0.f ? -mx / (float)tmax : 0.f;
      if (fabsf(sc[ib]) > amax_sc) amax_sc = fabsf(sc[ib]);
    }
    memset(&y[i], 0, sizeof(y[i]));
    if (amax_sc == 0.f) {
      for (int ib = 0; ib < 8; ++ib) { /* ls = 32: value 0 */
        y[i].scales_l[ib / 2] |= (uint8_t)(0 << (4 * (ib & 1)));
        y[i].scales_h |= (uint16_t)(2 << (2 * ib));
      }
      continue;
    }
    const float d = amax_sc / 32.f;
    y[i].d = zmo_fp32_to_fp16(d);
    const float dd = zmo_fp16_to_fp32(y[i].d);
    for (int ib = 0; ib < 8; ++ib) {
      int ls = dd > 0.f ? zmo_nearest_int(sc[ib] / dd) : 0;
      ls = (ls < -32 ? -32 : (ls > 31 ? 31 : ls)) + 32;
      y[i].scales_l[ib / 2] |= (uint8_t)((ls & 15) << (4 * (ib & 1)));
      y[i].scales_h |= (uint16_t)((ls >> 4) << (2 * ib));
      const float s = dd * (float)(ls - 32);
      for (int j = 0; j < 16; ++j) {
        const int lo = s != 0.f ? nearest_iq4(t, x[32 * ib + j] / s) : 8;
        const int hi = s != 0.f ? nearest_iq4(t, x[32 * ib + 16 + j] / s) : 8;
        y[i].qs[16 * ib + j] = (uint8_t)(lo | (hi << 4));
      }
    }
  }
}

/* IQ3_XXS: per 8-weight group an 8-bit sign pattern of even parity (7 bits
 * stored, as IQ2_XXS) and two grid indices (four |values| each); per
 * 32-weight sub-block a 4-bit scale ls with value d * (0.5 + ls) * 0.5
 * (dequant at kernels/quant/iq3_matmul.cu:104-122). */
static int nearest_grid4(const float *a, float inv, const uint32_t *grid) {
  int best = 0;
  float be = 3.4e38f;
  for (int g = 0; g < 256; ++g) {
    float e = 0;
    for (int j = 0; j < 4; ++j) {
      const float dd = a[j] * inv - (float)((grid[g] >> (8 * j)) & 0xff);
      e += dd * dd;
    }
    if (e < be) {
      be = e;
      best = g;
    }
  }
  return best;
}

void zmo_quantize_row_iq3_xxs(const float *x, zmo_block_iq3_xxs *y, int64_t k) {
  const uint32_t *grid = zmo_iq3xxs_grid();
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i, x += ZMO_QK_K) {
    float a[256], sub[8], max_sub = 0.f;
    uint8_t sign[32];
    for (int g = 0; g < 32; ++g) {
      int neg = 0, minj = 0;
      float mina = 3.4e38f;
      uint8_t sg = 0;
      for (int j = 0; j < 8; ++j) {
        a[8 * g + j] = fabsf(x[8 * g + j]);
        if (x[8 * g + j] < 0) {
          ++neg;
          sg |= (uint8_t)(1u << j);
        }
        if (a[8 * g + j] < mina) {
          mina = a[8 * g + j];
          minj = j;
        }
      }
      if (neg & 1) sg ^= (uint8_t)(1u << minj);
      sign[g] = sg;
    }
    for (int ib = 0; ib < 8; ++ib) {
      float amax = 0.f;
      for (int j = 0; j < 32; ++j) amax = a[32 * ib + j] > amax ? a[32 * ib + j] : amax;
      sub[ib] = amax / 62.f;
      max_sub = sub[ib] > max_sub ? sub[ib] : max_sub;
    }
    memset(&y[i], 0, sizeof(y[i]));
    if (max_sub == 0.f) continue;
    y[i].d = zmo_fp32_to_fp16(max_sub / (0.5f * 15.5f));
    const float dq = zmo_fp16_to_fp32(y[i].d);
    for (int ib = 0; ib < 8; ++ib) {
      int ls = dq > 0.f ? zmo_nearest_int(sub[ib] / (0.5f * dq) - 0.5f) : 0;
      ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
      const float s = dq * (0.5f + ls) * 0.5f;
      uint32_t aux = (uint32_t)ls << 28;
      for (int l = 0; l < 4; ++l) {
        for (int h = 0; h < 2; ++h)
          y[i].qs[8 * ib + 2 * l + h] = (uint8_t)(s > 0.f ? nearest_grid4(a + 32 * ib + 8 * l + 4 * h, 1.f / s, grid) : 0);
        aux |= (uint32_t)(sign[4 * ib + l] & 127u) << (7 * l);
      }
      memcpy(y[i].qs + 64 + 4 * ib, &aux, 4);
    }
  }
}

void zmo_quantize_rows(int type, const float *x, void *dst, int64_t rows, int64_t n) {
  const size_t rs = zmo_row_size(type, n);
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t r = 0; r < rows; ++r) {
    void *out = (char *)dst + (size_t)r * rs;
    const float *xr = x + r * n;
    switch (type) {
    case ZMO_TYPE_Q2_K: zmo_quantize_row_q2_K(xr, (zmo_block_q2_K *)out, n); break;
    case ZMO_TYPE_Q3_K: zmo_quantize_row_q3_K(xr, (zmo_block_q3_K *)out, n); break;
    case ZMO_TYPE_Q4_K: zmo_quantize_row_q4_K(xr, (zmo_block_q4_K *)out, n); break;
    case ZMO_TYPE_Q5_K: zmo_quantize_row_q5_K(xr, (zmo_block_q5_K *)out, n); break;
    case ZMO_TYPE_Q6_K: zmo_quantize_row_q6_K(xr, (zmo_block_q6_K *)out, n); break;
    case ZMO_TYPE_IQ2_XXS: zmo_quantize_row_iq2_xxs(xr, (zmo_block_iq2_xxs *)out, n); break;
    case ZMO_TYPE_IQ4_XS: zmo_quantize_row_iq4_xs(xr, (zmo_block_iq4_xs *)out, n); break;
    case ZMO_TYPE_IQ3_XXS: zmo_quantize_row_iq3_xxs(xr, (zmo_block_iq3_xxs *)out, n); break;
    case ZMO_TYPE_Q8_K: zmo_quantize_row_q8_K(xr, (zmo_block_q8_K *)out, n); break;
    default: break;
    }
  }
}

/* ------------------------------------------------------------------ dequant */

/* dequantize_row_q2_K (kquant_matmul.cu:55-72 restates it). */
static void dequant_q2_K(const zmo_block_q2_K *x, float *y, int64_t k) {
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d), mn = zmo_fp16_to_fp32(x[i].dmin);
    const uint8_t *q = x[i].qs;
    int is = 0;
    for (int n = 0; n < ZMO_QK_K; n += 128) {
      int shift = 0;
      for (int j = 0; j < 4; ++j) {
        uint8_t sc = x[i].scales[is++];
        float dl = d * (sc & 0xF), ml = mn * (sc >> 4);
        for (int l = 0; l < 16; ++l) *y++ = dl * ((q[l] >> shift) & 3) - ml;
        sc = x[i].scales[is++];
        dl = d * (sc & 0xF);
        ml = mn * (sc >> 4);
        for (int l = 0; l < 16; ++l) *y++ = dl * ((q[l + 16] >> shift) & 3) - ml;
        shift += 2;
      }
      q += 32;
    }
  }
}

/* 16 signed 6-bit Q3_K scales (value - 32), kquant_matmul.cu:161-175. */
static void q3_scales(const uint8_t *s12, int8_t *out) {
  uint32_t aux[4];
  memcpy(aux, s12, 12);
  const uint32_t kmask1 = 0x03030303, kmask2 = 0x0f0f0f0f;
  const uint32_t tmp = aux[2];
  aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
  aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
  aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
  aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
  const uint8_t *b = (const uint8_t *)aux;
  for (int i = 0; i < 16; ++i) out[i] = (int8_t)(b[i] - 32);
}

/* dequantize_row_q3_K: the hmask pointer does not advance (kquant_matmul.cu:186-200). */
static void dequant_q3_K(const zmo_block_q3_K *x, float *y, int64_t k) {
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d_all = zmo_fp16_to_fp32(x[i].d);
    int8_t sc[16];
    q3_scales(x[i].scales, sc);
    const uint8_t *q = x[i].qs, *hm = x[i].hmask;
    uint8_t m = 1;
    int is = 0;
    for (int n = 0; n < ZMO_QK_K; n += 128) {
      int shift = 0;
      for (int j = 0; j < 4; ++j) {
        float dl = d_all * sc[is++];
        for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l] >> shift) & 3) - ((hm[l] & m) ? 0 : 4));
        dl = d_all * sc[is++];
        for (int l = 0; l < 16; ++l) *y++ = dl * ((int8_t)((q[l + 16] >> shift) & 3) - ((hm[l + 16] & m) ? 0 : 4));
        shift += 2;
        m <<= 1;
      }
      q += 32;
    }
  }
}

/* dequantize_row_q4_K (kquant_matmul.cu:74-92). */
static void dequant_q4_K(const zmo_block_q4_K *x, float *y, int64_t k) {
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d), mn = zmo_fp16_to_fp32(x[i].dmin);
    const uint8_t *q = x[i].qs;
    int is = 0;
    for (int j = 0; j < ZMO_QK_K; j += 64) {
      uint8_t sc, m;
      scale_min_k4(is + 0, x[i].scales, &sc, &m);
      const float d1 = d * sc, m1 = mn * m;
      scale_min_k4(is + 1, x[i].scales, &sc, &m);
      const float d2 = d * sc, m2 = mn * m;
      for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
      for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
      q += 32;
      is += 2;
    }
  }
}

/* dequantize_row_q5_K (kquant_matmul.cu:94-117). */
static void dequant_q5_K(const zmo_block_q5_K *x, float *y, int64_t k) {
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d), mn = zmo_fp16_to_fp32(x[i].dmin);
    for (int c = 0; c < 4; ++c) {
      uint8_t sc, m;
      scale_min_k4(2 * c, x[i].scales, &sc, &m);
      const float d1 = d * sc, m1 = mn * m;
      scale_min_k4(2 * c + 1, x[i].scales, &sc, &m);
      const float d2 = d * sc, m2 = mn * m;
      const uint8_t *q = x[i].qs + 32 * c;
      for (int l = 0; l < 32; ++l) *y++ = d1 * ((q[l] & 0xF) + ((x[i].qh[l] >> (2 * c)) & 1 ? 16 : 0)) - m1;
      for (int l = 0; l < 32; ++l) *y++ = d2 * ((q[l] >> 4) + ((x[i].qh[l] >> (2 * c + 1)) & 1 ? 16 : 0)) - m2;
    }
  }
}

/* Q6_K value of weight t of a block, q6 - 32 in [-32, 31]. */
static inline int q6_value(const zmo_block_q6_K *x, int t) {
  const int h = t / 128, g = (t % 128) / 32, l = t % 32;
  const uint8_t b = x->ql[64 * h + 32 * (g & 1) + l];
  const int lo = g < 2 ? (b & 0xF) : (b >> 4);
  return (lo | (((x->qh[32 * h + l] >> (2 * g)) & 3) << 4)) - 32;
}

/* dequantize_row_q6_K (kquant_matmul.cu:119-140): sub-block t/16. */
static void dequant_q6_K(const zmo_block_q6_K *x, float *y, int64_t k) {
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d);
    for (int t = 0; t < ZMO_QK_K; ++t) *y++ = d * x[i].scales[t / 16] * q6_value(&x[i], t);
  }
}

/* IQ4_XS 6-bit sub-block scale (value ls - 32). */
static inline int iq4_ls(const zmo_block_iq4_xs *x, int ib) {
  return (((x->scales_l[ib / 2] >> (4 * (ib & 1))) & 0xF) | (((x->scales_h >> (2 * ib)) & 3) << 4)) - 32;
}

/* dequantize_row_iq4_xs (kernels/quant/iq4xs_matmul.cu:80-99): sub-block ib,
 * byte j of its 16 qs bytes: low nibble -> weight 32ib + j, high -> 32ib + 16 + j. */
static void dequant_iq4_xs(const zmo_block_iq4_xs *x, float *y, int64_t k) {
  const int8_t *t = zmo_iq4nl_table();
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d);
    for (int ib = 0; ib < 8; ++ib) {
      const float dl = d * (float)iq4_ls(&x[i], ib);
      for (int j = 0; j < 16; ++j) y[32 * ib + j] = dl * (float)t[x[i].qs[16 * ib + j] & 0xF];
      for (int j = 0; j < 16; ++j) y[32 * ib + 16 + j] = dl * (float)t[x[i].qs[16 * ib + j] >> 4];
    }
    y += ZMO_QK_K;
  }
}

/* dequantize_row_iq3_xxs (kernels/quant/iq3_matmul.cu:104-122): sub-block
 * ib: scales+signs word u = qs[64 + 4ib ..]; group l of 8 weights: grid
 * entries qs[8ib + 2l] (weights 0..3) and qs[8ib + 2l + 1] (4..7), signs
 * ksigns_iq2xs[(u >> 7l) & 127], value d * (0.5 + (u >> 28)) * 0.5 * grid. */
static void dequant_iq3_xxs(const zmo_block_iq3_xxs *x, float *y, int64_t k) {
  const uint32_t *grid = zmo_iq3xxs_grid();
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d);
    for (int ib = 0; ib < 8; ++ib) {
      uint32_t u;
      memcpy(&u, x[i].qs + 64 + 4 * ib, 4);
      const float db = d * (0.5f + (float)(u >> 28)) * 0.5f;
      for (int l = 0; l < 4; ++l) {
        const uint8_t signs = zmo_ksigns_iq2xs((int)((u >> (7 * l)) & 127));
        for (int j = 0; j < 8; ++j) {
          const uint32_t g = grid[x[i].qs[8 * ib + 2 * l + (j >> 2)]];
          const float v = db * (float)((g >> (8 * (j & 3))) & 0xff);
          *y++ = ((signs >> j) & 1) ? -v : v;
        }
      }
    }
  }
}

/* dequantize_row_iq2_xxs (iq2_matmul.cu:73-91). */
static void dequant_iq2_xxs(const zmo_block_iq2_xxs *x, float *y, int64_t k) {
  const uint64_t *grid = zmo_iq2xxs_grid();
  for (int64_t i = 0; i < k / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d);
    for (int ib = 0; ib < 8; ++ib) {
      const uint32_t a0 = x[i].qs[4 * ib] | ((uint32_t)x[i].qs[4 * ib + 1] << 16);
      const uint32_t a1 = x[i].qs[4 * ib + 2] | ((uint32_t)x[i].qs[4 * ib + 3] << 16);
      const float db = d * (0.5f + (a1 >> 28)) * 0.25f;
      for (int l = 0; l < 4; ++l) {
        const uint64_t g = grid[(a0 >> (8 * l)) & 0xff];
        const uint8_t signs = zmo_ksigns_iq2xs((a1 >> (7 * l)) & 127);
        for (int j = 0; j < 8; ++j)
          *y++ = db * (float)((g >> (8 * j)) & 0xff) * ((signs >> j) & 1 ? -1.f : 1.f);
      }
    }
  }
}

void zmo_dequantize_row(int type, const void *src, float *y, int64_t n) {
  switch (type) {
  case ZMO_TYPE_Q2_K: dequant_q2_K((const zmo_block_q2_K *)src, y, n); break;
  case ZMO_TYPE_Q3_K: dequant_q3_K((const zmo_block_q3_K *)src, y, n); break;
  case ZMO_TYPE_Q4_K: dequant_q4_K((const zmo_block_q4_K *)src, y, n); break;
  case ZMO_TYPE_Q5_K: dequant_q5_K((const zmo_block_q5_K *)src, y, n); break;
  case ZMO_TYPE_Q6_K: dequant_q6_K((const zmo_block_q6_K *)src, y, n); break;
  case ZMO_TYPE_IQ2_XXS: dequant_iq2_xxs((const zmo_block_iq2_xxs *)src, y, n); break;
  case ZMO_TYPE_IQ4_XS: dequant_iq4_xs((const zmo_block_iq4_xs *)src, y, n); break;
  case ZMO_TYPE_IQ3_XXS: dequant_iq3_xxs((const zmo_block_iq3_xxs *)src, y, n); break;
  case ZMO_TYPE_Q8_K: {
    const zmo_block_q8_K *b = (const zmo_block_q8_K *)src;
    for (int64_t i = 0; i < n / ZMO_QK_K; ++i)
      for (int j = 0; j < ZMO_QK_K; ++j) *y++ = b[i].d * b[i].qs[j];
    break;
  }
  case ZMO_TYPE_F32: memcpy(y, src, (size_t)n * 4); break;
  default: break;
  }
}

/* --------------------------------------------------------------------- dots */

/* _mm256 hsum order used by every x86 dot: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). */
static inline float hsum8(const float a[8]) {
  const float r0 = a[4] + a[0], r1 = a[5] + a[1], r2 = a[6] + a[2], r3 = a[7] + a[3];
  return (r0 + r2) + (r1 + r3);
}

/* ggml_vec_dot_q2_K_q8_K, AVX2 branch (bench/q2k_dot_bench.cpp:31-63).
 * Lane l of the 8-float accumulator takes the mins term
 * m[2l]*bsum[2l] + m[2l+1]*bsum[2l+1] (fma with -dx*dmin) and the integer sum
 * over bytes [4l, 4l+4) of every 32-weight chunk scaled by its 16-weight
 * sub-block scale (fma with dx*d). */
static float dot_q2_K(int n, const zmo_block_q2_K *x, const zmo_block_q8_K *y) {
  float acc[8] = {0};
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = y[i].d * zmo_fp16_to_fp32(x[i].d);
    const float dmin = -y[i].d * zmo_fp16_to_fp32(x[i].dmin);
    int32_t prod[8], sumi[8] = {0};
    for (int l = 0; l < 8; ++l)
      prod[l] = (x[i].scales[2 * l] >> 4) * y[i].bsums[2 * l] + (x[i].scales[2 * l + 1] >> 4) * y[i].bsums[2 * l + 1];
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(dmin, (float)prod[l], acc[l]);
    for (int j = 0; j < 2; ++j)
      for (int sh = 0; sh < 4; ++sh)
        for (int t = 0; t < 32; ++t) {
          const int q2 = (x[i].qs[32 * j + t] >> (2 * sh)) & 3;
          const int sc = x[i].scales[8 * j + 2 * sh + (t >= 16)] & 0xF;
          sumi[t >> 2] += sc * q2 * y[i].qs[128 * j + 32 * sh + t];
        }
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
  }
  return hsum8(acc);
}

/* Q3_K: integer sum per lane class as for Q2_K (values q - 4*(!hbit) in
 * [-4,3], 6-bit signed scales), one fma per lane per block.  Float order:
 * parity unpinned (ggml's stock AVX2 Q3_K is not in the reference tree). */
static float dot_q3_K(int n, const zmo_block_q3_K *x, const zmo_block_q8_K *y) {
  float acc[8] = {0};
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = y[i].d * zmo_fp16_to_fp32(x[i].d);
    int8_t sc[16];
    q3_scales(x[i].scales, sc);
    int32_t sumi[8] = {0};
    for (int j = 0; j < 2; ++j)
      for (int sh = 0; sh < 4; ++sh)
        for (int t = 0; t < 32; ++t) {
          const int q2 = (x[i].qs[32 * j + t] >> (2 * sh)) & 3;
          const int hb = (x[i].hmask[t] >> (4 * j + sh)) & 1;
          const int q = q2 - (hb ? 0 : 4);
          sumi[t >> 2] += sc[8 * j + 2 * sh + (t >= 16)] * q * y[i].qs[128 * j + 32 * sh + t];
        }
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
  }
  return hsum8(acc);
}

/* ggml_vec_dot_q4_K_q8_K, x86 order (bench/q3k_q4k_dot_bench.cpp:73-125):
 * 8-lane acc of d*sumi (lane l = bytes [4l,4l+4) of each 32-weight half-chunk,
 * scaled by its 32-weight sub-block scale) and a 4-lane acc_m of
 * dmin*(m[2l]*s32[2l] + m[2l+1]*s32[2l+1]) where s32 are 32-weight bsums. */
static float dot_q4_K(int n, const zmo_block_q4_K *x, const zmo_block_q8_K *y) {
  float acc[8] = {0}, accm[4] = {0};
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = y[i].d * zmo_fp16_to_fp32(x[i].d);
    const float dmin = -y[i].d * zmo_fp16_to_fp32(x[i].dmin);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; ++j) scale_min_k4(j, x[i].scales, &sc[j], &m[j]);
    int32_t s32[8];
    for (int j = 0; j < 8; ++j) s32[j] = y[i].bsums[2 * j] + y[i].bsums[2 * j + 1];
    for (int l = 0; l < 4; ++l) {
      const int32_t prod = m[2 * l] * s32[2 * l] + m[2 * l + 1] * s32[2 * l + 1];
      accm[l] = fmaf(dmin, (float)prod, accm[l]);
    }
    int32_t sumi[8] = {0};
    for (int j = 0; j < 4; ++j)
      for (int t = 0; t < 32; ++t) {
        const uint8_t b = x[i].qs[32 * j + t];
        sumi[t >> 2] += sc[2 * j] * (b & 0xF) * y[i].qs[64 * j + t];
        sumi[t >> 2] += sc[2 * j + 1] * (b >> 4) * y[i].qs[64 * j + 32 + t];
      }
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
  }
  const float m01 = accm[0] + accm[2], m23 = accm[1] + accm[3];
  return hsum8(acc) + (m01 + m23);
}

/* Q5_K: the Q4_K structure with 5-bit values -- 8-lane acc of d*sumi (lane l
 * = bytes [4l,4l+4) of each 32-weight sub-block) and the mins term
 * dmin * sum m_j*s32_j summed in integers per block and accumulated as one
 * scalar.  Float order: parity unpinned (ggml's stock Q5_K dot is not in the
 * reference tree). */
static float dot_q5_K(int n, const zmo_block_q5_K *x, const zmo_block_q8_K *y) {
  float acc[8] = {0}, summs = 0;
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = y[i].d * zmo_fp16_to_fp32(x[i].d);
    const float dmin = -y[i].d * zmo_fp16_to_fp32(x[i].dmin);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; ++j) scale_min_k4(j, x[i].scales, &sc[j], &m[j]);
    int32_t prod = 0;
    for (int j = 0; j < 8; ++j) prod += m[j] * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
    summs = fmaf(dmin, (float)prod, summs);
    int32_t sumi[8] = {0};
    for (int j = 0; j < 8; ++j)
      for (int t = 0; t < 32; ++t) {
        const uint8_t b = x[i].qs[32 * (j / 2) + t];
        const int q = ((j & 1) ? (b >> 4) : (b & 0xF)) | (((x[i].qh[t] >> j) & 1) << 4);
        sumi[t >> 2] += sc[j] * q * y[i].qs[32 * j + t];
      }
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
  }
  return hsum8(acc) + summs;
}

/* Q6_K: per-lane integer sums of sc * (q6 - 32) * q8 (lane l = bytes
 * [4l,4l+4) of each 32-weight chunk), one fma per lane per block.  Float
 * order: parity unpinned, as for Q5_K. */
static float dot_q6_K(int n, const zmo_block_q6_K *x, const zmo_block_q8_K *y) {
  float acc[8] = {0};
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = y[i].d * zmo_fp16_to_fp32(x[i].d);
    int32_t sumi[8] = {0};
    for (int t = 0; t < ZMO_QK_K; ++t) sumi[(t & 31) >> 2] += x[i].scales[t / 16] * q6_value(&x[i], t) * y[i].qs[t];
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
  }
  return hsum8(acc);
}

/* IQ4_XS: isum = sum_ib (ls - 32) * sum table[q] * q8 per block, one fma
 * with d * d_y per block.  Float order: parity unpinned (ggml's stock
 * IQ4_XS dot is not in the reference tree). */
static float dot_iq4_xs(int n, const zmo_block_iq4_xs *x, const zmo_block_q8_K *y) {
  const int8_t *t = zmo_iq4nl_table();
  float acc = 0.f;
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    int32_t isum = 0;
    for (int ib = 0; ib < 8; ++ib) {
      int32_t s = 0;
      for (int j = 0; j < 16; ++j) {
        s += t[x[i].qs[16 * ib + j] & 0xF] * y[i].qs[32 * ib + j];
        s += t[x[i].qs[16 * ib + j] >> 4] * y[i].qs[32 * ib + 16 + j];
      }
      isum += iq4_ls(&x[i], ib) * s;
    }
    acc = fmaf(zmo_fp16_to_fp32(x[i].d) * y[i].d, (float)isum, acc);
  }
  return acc;
}

/* ggml_vec_dot_iq3_xxs_q8_K in the stock AVX2 order that the reference holds
 * as source (bench/iq3k/iq3_dot_bench.c:17-37, ref()): int32 lane l (of 8)
 * sums (2 ls + 1) * grid * sign * q8 over bytes [4l, 4l+4) of every 32-weight
 * sub-block of a block (the even and odd sub-blocks in two accumulators, added
 * lane-wise at the end of the block: the same integers), one fma per block and
 * lane with d = fp16(d) * d_y, result 0.25 * hsum8.  That file needs ggml's
 * ggml-common.h (absent here), so it is not built: the integer sums are pinned
 * by brute force, the float order only by this restatement. */
static float dot_iq3_xxs(int n, const zmo_block_iq3_xxs *x, const zmo_block_q8_K *y) {
  const uint32_t *grid = zmo_iq3xxs_grid();
  float acc[8] = {0};
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d) * y[i].d;
    int32_t sumi[8] = {0};
    for (int ib = 0; ib < 8; ++ib) {
      uint32_t u;
      memcpy(&u, x[i].qs + 64 + 4 * ib, 4);
      const int32_t ls = 2 * (int32_t)(u >> 28) + 1;
      for (int lane = 0; lane < 8; ++lane) {
        /* bytes 4*lane .. 4*lane+3 of the sub-block: grid entry qs[8 ib + lane],
         * sign group lane / 2 (8 signs per 7-bit index) */
        const uint8_t signs = zmo_ksigns_iq2xs((int)((u >> (7 * (lane >> 1))) & 127));
        const uint32_t g4 = grid[x[i].qs[8 * ib + lane]];
        int32_t s4 = 0;
        for (int j = 0; j < 4; ++j) {
          const int g = (int)((g4 >> (8 * j)) & 0xff);
          const int q8 = y[i].qs[32 * ib + 4 * lane + j];
          s4 += ((signs >> (4 * (lane & 1) + j)) & 1) ? -g * q8 : g * q8;
        }
        sumi[lane] += ls * s4;
      }
    }
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
  }
  return 0.25f * hsum8(acc);
}

/* ggml_vec_dot_iq2_xxs_q8_K, AVX2 / AVX-512BW order (patches/ggml/0009...:34-95,
 * bench/kernels/iq2xxs_dot_bench.cpp:26-50): lane l sums (2ls+1)*grid*sign*q8
 * over bytes [4l,4l+4) of each 32-weight sub-block; one fma per block with
 * d = fp16(d)*dy; result 0.125 * hsum. */
static float dot_iq2_xxs(int n, const zmo_block_iq2_xxs *x, const zmo_block_q8_K *y) {
  const uint64_t *grid = zmo_iq2xxs_grid();
  float acc[8] = {0};
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = zmo_fp16_to_fp32(x[i].d) * y[i].d;
    int32_t sumi[8] = {0};
    for (int ib = 0; ib < 8; ++ib) {
      const uint32_t a0 = x[i].qs[4 * ib] | ((uint32_t)x[i].qs[4 * ib + 1] << 16);
      const uint32_t a1 = x[i].qs[4 * ib + 2] | ((uint32_t)x[i].qs[4 * ib + 3] << 16);
      const int ls = 2 * (int)(a1 >> 28) + 1;
      for (int t = 0; t < 32; ++t) {
        const int l = t >> 3, j = t & 7;
        const int g = (int)((grid[(a0 >> (8 * l)) & 0xff] >> (8 * j)) & 0xff);
        const uint8_t s = zmo_ksigns_iq2xs((a1 >> (7 * l)) & 127);
        const int q8 = ((s >> j) & 1) ? -y[i].qs[32 * ib + t] : y[i].qs[32 * ib + t];
        sumi[t >> 2] += ls * g * q8;
      }
    }
    for (int l = 0; l < 8; ++l) acc[l] = fmaf(d, (float)sumi[l], acc[l]);
  }
  return 0.125f * hsum8(acc);
}

float zmo_vec_dot_q8_K(int type, int n, const void *x, const zmo_block_q8_K *y) {
  switch (type) {
  case ZMO_TYPE_Q2_K: return dot_q2_K(n, (const zmo_block_q2_K *)x, y);
  case ZMO_TYPE_Q3_K: return dot_q3_K(n, (const zmo_block_q3_K *)x, y);
  case ZMO_TYPE_Q4_K: return dot_q4_K(n, (const zmo_block_q4_K *)x, y);
  case ZMO_TYPE_Q5_K: return dot_q5_K(n, (const zmo_block_q5_K *)x, y);
  case ZMO_TYPE_Q6_K: return dot_q6_K(n, (const zmo_block_q6_K *)x, y);
  case ZMO_TYPE_IQ2_XXS: return dot_iq2_xxs(n, (const zmo_block_iq2_xxs *)x, y);
  case ZMO_TYPE_IQ4_XS: return dot_iq4_xs(n, (const zmo_block_iq4_xs *)x, y);
  case ZMO_TYPE_IQ3_XXS: return dot_iq3_xxs(n, (const zmo_block_iq3_xxs *)x, y);
  default: return NAN;
  }
}

void zmo_block_dots(int type, int n, const void *vx, const zmo_block_q8_K *y, int32_t *isum, int32_t *imin) {
  float w[256];
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    int32_t s = 0, mm = 0;
    if (type == ZMO_TYPE_Q2_K) {
      const zmo_block_q2_K *x = (const zmo_block_q2_K *)vx + i;
      for (int j = 0; j < 16; ++j) mm += (x->scales[j] >> 4) * y[i].bsums[j];
      for (int t = 0; t < 256; ++t) {
        const int h = t / 128, r = t % 128, sh = r / 32, l = r % 32;
        s += (x->scales[t / 16] & 0xF) * ((x->qs[32 * h + l] >> (2 * sh)) & 3) * y[i].qs[t];
      }
    } else if (type == ZMO_TYPE_Q3_K) {
      const zmo_block_q3_K *x = (const zmo_block_q3_K *)vx + i;
      int8_t sc[16];
      q3_scales(x->scales, sc);
      for (int t = 0; t < 256; ++t) {
        const int h = t / 128, r = t % 128, sh = r / 32, l = r % 32;
        const int q = ((x->qs[32 * h + l] >> (2 * sh)) & 3) - (((x->hmask[l] >> (4 * h + sh)) & 1) ? 0 : 4);
        s += sc[t / 16] * q * y[i].qs[t];
      }
    } else if (type == ZMO_TYPE_Q4_K) {
      const zmo_block_q4_K *x = (const zmo_block_q4_K *)vx + i;
      uint8_t sc, m;
      for (int j = 0; j < 8; ++j) {
        scale_min_k4(j, x->scales, &sc, &m);
        mm += m * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        for (int l = 0; l < 32; ++l) {
          const int t = 32 * j + l;
          const uint8_t b = x->qs[32 * (j / 2) + l];
          s += sc * ((j & 1) ? (b >> 4) : (b & 0xF)) * y[i].qs[t];
        }
      }
    } else if (type == ZMO_TYPE_Q5_K) {
      /* from the dequant with d = 1, dmin = 0: exact integers sc * q */
      zmo_block_q5_K one = ((const zmo_block_q5_K *)vx)[i];
      one.d = 0x3c00;
      one.dmin = 0;
      dequant_q5_K(&one, w, 256);
      uint8_t sc, m;
      for (int j = 0; j < 8; ++j) {
        scale_min_k4(j, one.scales, &sc, &m);
        mm += m * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
      }
      for (int t = 0; t < 256; ++t) s += (int32_t)lrintf(w[t]) * y[i].qs[t];
    } else if (type == ZMO_TYPE_Q6_K) {
      const zmo_block_q6_K *x = (const zmo_block_q6_K *)vx + i;
      for (int t = 0; t < 256; ++t) s += x->scales[t / 16] * q6_value(x, t) * y[i].qs[t];
    } else if (type == ZMO_TYPE_IQ3_XXS) {
      /* (2ls+1)*grid*sign = 4 * dequant / d: reuse the dequant as integers */
      zmo_block_iq3_xxs one = ((const zmo_block_iq3_xxs *)vx)[i];
      one.d = 0x3c00;
      dequant_iq3_xxs(&one, w, 256);
      for (int t = 0; t < 256; ++t) s += (int32_t)lrintf(w[t] * 4.0f) * y[i].qs[t];
    } else if (type == ZMO_TYPE_IQ4_XS) {
      /* (ls - 32) * table value = dequant / d: reuse the dequant as integers */
      zmo_block_iq4_xs one = ((const zmo_block_iq4_xs *)vx)[i];
      one.d = 0x3c00;
      dequant_iq4_xs(&one, w, 256);
      for (int t = 0; t < 256; ++t) s += (int32_t)lrintf(w[t]) * y[i].qs[t];
    } else if (type == ZMO_TYPE_IQ2_XXS) {
      /* (2ls+1)*grid*sign = 8 * dequant / d: reuse the dequant as integers */
      zmo_block_iq2_xxs one = ((const zmo_block_iq2_xxs *)vx)[i];
      one.d = 0x3c00; /* 1.0 */
      dequant_iq2_xxs(&one, w, 256);
      for (int t = 0; t < 256; ++t) s += (int32_t)lrintf(w[t] * 8.0f) * y[i].qs[t];
    }
    isum[i] = s;
    imin[i] = mm;
  }
}

/* ----------------------------------------------------------------- the op */

static int type_ok(int t) {
  return t == ZMO_TYPE_Q2_K || t == ZMO_TYPE_Q3_K || t == ZMO_TYPE_Q4_K || t == ZMO_TYPE_Q5_K || t == ZMO_TYPE_Q6_K ||
         t == ZMO_TYPE_IQ2_XXS || t == ZMO_TYPE_IQ3_XXS || t == ZMO_TYPE_IQ4_XS;
}

int zmo_mul_mat_id(const zmo_tensor *src0, const zmo_tensor *src1, const zmo_tensor *ids, zmo_tensor *dst,
                   int nthreads) {
  if (!type_ok(src0->type) || src1->type != ZMO_TYPE_F32 || ids->type != ZMO_TYPE_I32 || dst->type != ZMO_TYPE_F32)
    return -1;
  const int64_t ne00 = src0->ne[0], ne01 = src0->ne[1], n_as = src0->ne[2];
  const int64_t ne11 = src1->ne[1], ne12 = src1->ne[2];
  const int64_t n_ids = ids->ne[0];
  if (ne00 % ZMO_QK_K || src1->ne[0] != ne00 || dst->ne[0] != ne01 || dst->ne[1] != n_ids || dst->ne[2] != ne12 ||
      ids->ne[1] != ne12)
    return -1;
  /* (i) quantize every src1 row to Q8_K (serial, as patch 0002 does for small src1) */
  const int64_t nbq = ne00 / ZMO_QK_K;
  zmo_block_q8_K *q8 = (zmo_block_q8_K *)malloc(sizeof(zmo_block_q8_K) * (size_t)(nbq * ne11 * ne12));
  for (int64_t i12 = 0; i12 < ne12; ++i12)
    for (int64_t i11 = 0; i11 < ne11; ++i11)
      zmo_quantize_row_q8_K((const float *)((const char *)src1->data + i11 * src1->nb[1] + i12 * src1->nb[2]),
                            q8 + (i12 * ne11 + i11) * nbq, ne00);
  int bad = 0;
  /* (ii) routes; negative id -> zero output row (0002...:50-54) */
  for (int64_t t = 0; t < ne12; ++t) {
    for (int64_t id = 0; id < n_ids; ++id) {
      const int32_t e = *(const int32_t *)((const char *)ids->data + t * ids->nb[1] + id * ids->nb[0]);
      float *out = (float *)((char *)dst->data + id * dst->nb[1] + t * dst->nb[2]);
      if (e < 0) {
        for (int64_t r = 0; r < ne01; ++r) out[r] = 0.0f;
        continue;
      }
      if (e >= n_as) {
        bad = 1;
        continue;
      }
      const zmo_block_q8_K *yq = q8 + (t * ne11 + (id % ne11)) * nbq;
      const char *wbase = (const char *)src0->data + e * src0->nb[2];
      /* (iii) one vec_dot per output element */
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
      for (int64_t r = 0; r < ne01; ++r)
        out[r] = zmo_vec_dot_q8_K(src0->type, (int)ne00, wbase + r * src0->nb[1], yq);
    }
  }
  free(q8);
  return bad ? -2 : 0;
}

/* ------------------------------------------------------ router & bucketing */

static float gate_value(int gating, float x) {
  if (gating == ZMO_GATING_SIGMOID) return 1.0f / (1.0f + zmo_expf(-x));
  if (gating == ZMO_GATING_SQRT_SOFTPLUS) {
    const float sp = x > 0.0f ? x + log1pf(zmo_expf(-x)) : log1pf(zmo_expf(x));
    return sqrtf(sp);
  }
  return x;
}

/* better(a, b): a outranks b (higher score; lower index on ties) */
static inline int outranks(float sa, int ia, float sb, int ib) { return sa > sb || (sa == sb && ia < ib); }

/* moe_routed::gate_probs / select_ids / route_weights (moe_routed_ggml.hpp:52-141),
 * restated with core/moe_router.cpp:6-37 and glm5next_router.cu:33-93.
 * Softmax sums in double (ggml_vec_soft_max_f32 accumulates ggml_float).
 * Top-k order: descending score, lowest expert index first on ties. */
void zmo_router(const zmo_router_spec *spec, const float *logits, const float *logit_bias, const float *sel_bias,
                int S, int32_t *ids, float *weights) {
  const int E = spec->n_experts, K = spec->topk;
  float *p = (float *)malloc(sizeof(float) * (size_t)E);
  float *sel = (float *)malloc(sizeof(float) * (size_t)E);
  for (int s = 0; s < S; ++s) {
    const float *l = logits + (size_t)s * E;
    for (int e = 0; e < E; ++e) p[e] = logit_bias ? l[e] + logit_bias[e] : l[e];
    if (spec->gating == ZMO_GATING_SOFTMAX) {
      float mx = p[0];
      for (int e = 1; e < E; ++e) mx = p[e] > mx ? p[e] : mx;
      double sum = 0.0;
      for (int e = 0; e < E; ++e) {
        p[e] = zmo_expf(p[e] - mx);
        sum += (double)p[e];
      }
      const float inv = (float)(1.0 / sum);
      for (int e = 0; e < E; ++e) p[e] *= inv;
    } else {
      for (int e = 0; e < E; ++e) p[e] = gate_value(spec->gating, p[e]);
    }
    for (int e = 0; e < E; ++e) sel[e] = sel_bias ? p[e] + sel_bias[e] : p[e];
    if (spec->n_groups > 1 && spec->n_groups_used > 0 && spec->n_groups_used < spec->n_groups &&
        E % spec->n_groups == 0) {
      const int G = spec->n_groups, gs = E / G;
      float gscore[64];
      int keep[64] = {0};
      for (int g = 0; g < G; ++g) {
        int b1 = -1, b2 = -1;
        for (int j = 0; j < gs; ++j) {
          const int e = g * gs + j;
          if (b1 < 0 || outranks(sel[e], e, sel[b1], b1)) {
            b2 = b1;
            b1 = e;
          } else if (b2 < 0 || outranks(sel[e], e, sel[b2], b2)) {
            b2 = e;
          }
        }
        gscore[g] = gs >= 2 ? sel[b1] + sel[b2] : sel[b1];
      }
      for (int r = 0; r < spec->n_groups_used; ++r) {
        int best = -1;
        for (int g = 0; g < G; ++g)
          if (!keep[g] && (best < 0 || outranks(gscore[g], g, gscore[best], best))) best = g;
        keep[best] = 1;
      }
      for (int e = 0; e < E; ++e)
        if (!keep[e / gs]) sel[e] = -INFINITY;
    }
    /* top-k by repeated selection */
    unsigned char *taken = (unsigned char *)calloc((size_t)E, 1);
    for (int k = 0; k < K; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e)
        if (!taken[e] && (best < 0 || outranks(sel[e], e, sel[best], best))) best = e;
      taken[best] = 1;
      ids[(size_t)s * K + k] = best;
      weights[(size_t)s * K + k] = p[best];
    }
    free(taken);
    if (spec->weights_norm) {
      double sum = 0.0;
      for (int k = 0; k < K; ++k) sum += (double)weights[(size_t)s * K + k];
      float fs = (float)sum;
      if (fs < 6.103515625e-5f) fs = 6.103515625e-5f;
      for (int k = 0; k < K; ++k) weights[(size_t)s * K + k] = weights[(size_t)s * K + k] / fs;
    }
    if (spec->weights_scale != 0.0f && spec->weights_scale != 1.0f)
      for (int k = 0; k < K; ++k) weights[(size_t)s * K + k] = weights[(size_t)s * K + k] * spec->weights_scale;
  }
  free(p);
  free(sel);
}

/* make_branch_inputs (moe_partial_route_ggml.hpp:21-35): ids' = route_map[ids],
 * w' = w * route_mask[ids]; mask defaults to (route_map >= 0). */
void zmo_apply_slot_table(const int32_t *route_map, const float *route_mask, int S, int K, int32_t *ids,
                          float *weights) {
  for (int i = 0; i < S * K; ++i) {
    const int e = ids[i];
    if (e < 0) continue;
    const float m = route_mask ? route_mask[e] : (route_map[e] >= 0 ? 1.0f : 0.0f);
    ids[i] = route_map[e];
    weights[i] = weights[i] * m;
  }
}

/* Stable counting sort of pairs (s*K+k) by expert (batched_dispatch_pipeline.cpp:1181-1202). */
int zmo_bucket(const int32_t *ids, int S, int K, int E, int32_t *counts, int32_t *offs, int32_t *pairs) {
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int i = 0; i < S * K; ++i)
    if (ids[i] >= 0 && ids[i] < E) counts[ids[i]]++;
  offs[0] = 0;
  for (int e = 0; e < E; ++e) offs[e + 1] = offs[e] + counts[e];
  int32_t *cur = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E > 0 ? E : 1));
  for (int e = 0; e < E; ++e) cur[e] = offs[e];
  for (int i = 0; i < S * K; ++i)
    if (ids[i] >= 0 && ids[i] < E) pairs[cur[ids[i]]++] = i;
  free(cur);
  return offs[E];
}

/* ggml_swiglu_split: silu(g) * u with silu(x) = x / (1 + exp(-x)). */
void zmo_swiglu(const float *g, const float *u, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float s = g[i] / (1.0f + zmo_expf(-g[i]));
    out[i] = s * u[i];
  }
}

/* one expert FFN for one Q8_K input row: y[H] = down . swiglu(gate . x, up . x) */
static void expert_ffn_row(int H, int F, int tg, int tu, int td, const char *wg, const char *wu, const char *wd,
                           const zmo_block_q8_K *xq, float *y, int nthreads) {
  const size_t rg = zmo_row_size(tg, H), ru = zmo_row_size(tu, H), rd = zmo_row_size(td, F);
  float *g = (float *)malloc(sizeof(float) * (size_t)F * 3);
  float *u = g + F, *a = u + F;
  zmo_block_q8_K *aq = (zmo_block_q8_K *)malloc(sizeof(zmo_block_q8_K) * (size_t)(F / ZMO_QK_K));
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
  for (int n = 0; n < F; ++n) {
    g[n] = zmo_vec_dot_q8_K(tg, H, wg + (size_t)n * rg, xq);
    u[n] = zmo_vec_dot_q8_K(tu, H, wu + (size_t)n * ru, xq);
  }
  zmo_swiglu(g, u, a, F);
  zmo_quantize_row_q8_K(a, aq, F);
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
  for (int h = 0; h < H; ++h) y[h] = zmo_vec_dot_q8_K(td, F, wd + (size_t)h * rd, aq);
  free(aq);
  free(g);
}

void zmo_moe_forward(const zmo_moe_desc *d, const float *x, const int32_t *ids, const float *weights, float *out,
                     int nthreads) {
  const int H = d->H, F = d->F, K = d->K, S = d->S;
  const size_t eg = zmo_row_size(d->type_gate, H) * (size_t)F;
  const size_t eu = zmo_row_size(d->type_up, H) * (size_t)F;
  const size_t ed = zmo_row_size(d->type_down, F) * (size_t)H;
  zmo_block_q8_K *xq = (zmo_block_q8_K *)malloc(sizeof(zmo_block_q8_K) * (size_t)(H / ZMO_QK_K));
  float *y = (float *)malloc(sizeof(float) * (size_t)H * (size_t)(K + 1));
  for (int s = 0; s < S; ++s) {
    zmo_quantize_row_q8_K(x + (size_t)s * H, xq, H);
    for (int k = 0; k < K; ++k) {
      const int e = ids[(size_t)s * K + k];
      float *yk = y + (size_t)k * H;
      if (e < 0) {
        for (int h = 0; h < H; ++h) yk[h] = 0.0f;
        continue;
      }
      expert_ffn_row(H, F, d->type_gate, d->type_up, d->type_down, (const char *)d->w_gate + (size_t)e * eg,
                     (const char *)d->w_up + (size_t)e * eu, (const char *)d->w_down + (size_t)e * ed, xq, yk,
                     nthreads);
    }
    /* ggml_mul(down, weights) then sum_topk: ((w0*y0 + w1*y1) + w2*y2) + ... */
    float *o = out + (size_t)s * H;
    for (int h = 0; h < H; ++h) {
      float acc = weights[(size_t)s * K] * y[h];
      for (int k = 1; k < K; ++k) acc = acc + weights[(size_t)s * K + k] * y[(size_t)k * H + h];
      o[h] = acc;
    }
    if (d->ws_gate) {
      float *ys = y + (size_t)K * H;
      expert_ffn_row(H, d->F_shared, d->type_shared, d->type_shared, d->type_shared, (const char *)d->ws_gate,
                     (const char *)d->ws_up, (const char *)d->ws_down, xq, ys, nthreads);
      for (int h = 0; h < H; ++h) o[h] = o[h] + ys[h];
    }
  }
  free(y);
  free(xq);
}

/* ggml_mul_mat(router, cur) with f32 weights: plain fp32 dot per expert,
 * accumulated in double (the float order of ggml_vec_dot_f32 is parity
 * unpinned; the double sum is within 1 ulp of any order's result). */
void zmo_router_gemv(const float *W, const float *x, int H, int E, int S, float *logits) {
  for (int s = 0; s < S; ++s)
    for (int e = 0; e < E; ++e) {
      double acc = 0.0;
      for (int i = 0; i < H; ++i) acc += (double)W[(size_t)e * H + i] * (double)x[(size_t)s * H + i];
      logits[(size_t)s * E + e] = (float)acc;
    }
}

/* ====================================================================== *
 * AVX-512 restatement of the reference's CPU expert path (the CPU baseline).
 *
 * The reference times ggml's CPU MUL_MAT_ID on AVX-512 hosts: per layer the
 * src1 row is quantized to Q8_K on one thread (patches/ggml/0002...:18-45),
 * threads split the output rows of the gate, up and down matrices, and each
 * row is one ggml_vec_dot_<type>_q8_K (models/qwen/ggml_qwen_cpu_moe.cpp:49-57;
 * 512-bit dots as in bench/q3k_q4k_dot_bench.cpp:73-125).  This restatement
 * keeps that structure and computes every dot with VNNI (vpdpbusd) in the
 * integer grouping of the oracle dots above, so its results are bit-identical
 * to zmo_moe_forward (checked by tests/test_oracle.py): per block the integer
 * lane sums of 4 consecutive bytes of each 32-weight chunk are formed exactly
 * (vpdpbusd of the unsigned 2-bit values against the signed Q8_K bytes, times
 * the chunk's 16-weight sub-block scale), folded to the 8 lanes of the
 * oracle's accumulator, and added with the same fmas and the same final hsum.
 * Types other than Q2_K / Q3_K use the oracle dots.
 * ====================================================================== */

#if defined(__x86_64__)
#include <immintrin.h>

#define ZMO_AVX512 __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,avx512dq,fma")))

/* lane l of 16 -> sub-block scale index 4k + (l >> 2) of 64-byte chunk pair k */
ZMO_AVX512 static inline __m512i scale_index(int k) {
  return _mm512_setr_epi32(4 * k, 4 * k, 4 * k, 4 * k, 4 * k + 1, 4 * k + 1, 4 * k + 1, 4 * k + 1, 4 * k + 2,
                           4 * k + 2, 4 * k + 2, 4 * k + 2, 4 * k + 3, 4 * k + 3, 4 * k + 3, 4 * k + 3);
}
/* per 16-bit word shift: s0 for the low 32 bytes, s1 for the high 32 */
ZMO_AVX512 static inline __m512i shift_pair(int s0, int s1) {
  return _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_set1_epi16((short)s0)), _mm256_set1_epi16((short)s1), 1);
}
ZMO_AVX512 static inline float finish8(__m256 acc) {
  float a[8];
  _mm256_storeu_ps(a, acc);
  return hsum8(a);
}

ZMO_AVX512 static float dot_q2_K_avx512(int n, const zmo_block_q2_K *x, const zmo_block_q8_K *y) {
  const __m512i m3 = _mm512_set1_epi8(3);
  const __m512i sh[2] = {shift_pair(0, 2), shift_pair(4, 6)};
  const __m512i idx[4] = {scale_index(0), scale_index(1), scale_index(2), scale_index(3)};
  __m256 acc = _mm256_setzero_ps();
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = y[i].d * zmo_fp16_to_fp32(x[i].d);
    const float dmin = -y[i].d * zmo_fp16_to_fp32(x[i].dmin);
    const __m128i sc8 = _mm_loadu_si128((const __m128i *)x[i].scales);
    /* mins: lane l = m[2l] * bsum[2l] + m[2l+1] * bsum[2l+1] */
    const __m256i m16 = _mm256_cvtepu8_epi16(_mm_and_si128(_mm_srli_epi16(sc8, 4), _mm_set1_epi8(0x0F)));
    const __m256i prod = _mm256_madd_epi16(m16, _mm256_loadu_si256((const __m256i *)y[i].bsums));
    acc = _mm256_fmadd_ps(_mm256_set1_ps(dmin), _mm256_cvtepi32_ps(prod), acc);
    const __m512i sc32 = _mm512_and_si512(_mm512_cvtepu8_epi32(sc8), _mm512_set1_epi32(0xF));
    __m512i sumi = _mm512_setzero_si512();
    for (int j = 0; j < 2; ++j) {
      const __m512i q = _mm512_broadcast_i64x4(_mm256_loadu_si256((const __m256i *)(x[i].qs + 32 * j)));
      for (int h = 0; h < 2; ++h) {
        const int k = 2 * j + h;
        const __m512i w = _mm512_and_si512(_mm512_srlv_epi16(q, sh[h]), m3);
        const __m512i q8 = _mm512_loadu_si512((const void *)(y[i].qs + 64 * k));
        const __m512i dp = _mm512_dpbusd_epi32(_mm512_setzero_si512(), w, q8);
        sumi = _mm512_add_epi32(sumi, _mm512_mullo_epi32(dp, _mm512_permutexvar_epi32(idx[k], sc32)));
      }
    }
    const __m256i s8 = _mm256_add_epi32(_mm512_castsi512_si256(sumi), _mm512_extracti64x4_epi64(sumi, 1));
    acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(s8), acc);
  }
  return finish8(acc);
}

ZMO_AVX512 static float dot_q3_K_avx512(int n, const zmo_block_q3_K *x, const zmo_block_q8_K *y) {
  const __m512i m3 = _mm512_set1_epi8(3), m1 = _mm512_set1_epi8(1);
  const __m512i sh[2] = {shift_pair(0, 2), shift_pair(4, 6)};
  const __m512i hs[4] = {shift_pair(0, 1), shift_pair(2, 3), shift_pair(4, 5), shift_pair(6, 7)};
  const __m512i idx[4] = {scale_index(0), scale_index(1), scale_index(2), scale_index(3)};
  __m256 acc = _mm256_setzero_ps();
  for (int i = 0; i < n / ZMO_QK_K; ++i) {
    const float d = y[i].d * zmo_fp16_to_fp32(x[i].d);
    int8_t sc[16];
    q3_scales(x[i].scales, sc);
    const __m512i sc32 = _mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)sc));
    /* 4 * (high bit clear): bit 2k (low half) / 2k+1 (high half) of hmask[t] */
    const __m512i nh = _mm512_broadcast_i64x4(
        _mm256_xor_si256(_mm256_loadu_si256((const __m256i *)x[i].hmask), _mm256_set1_epi8(-1)));
    __m512i sumi = _mm512_setzero_si512();
    for (int j = 0; j < 2; ++j) {
      const __m512i q = _mm512_broadcast_i64x4(_mm256_loadu_si256((const __m256i *)(x[i].qs + 32 * j)));
      for (int h = 0; h < 2; ++h) {
        const int k = 2 * j + h;
        const __m512i w = _mm512_and_si512(_mm512_srlv_epi16(q, sh[h]), m3);
        const __m512i n4 = _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(nh, hs[k]), m1), 2);
        const __m512i q8 = _mm512_loadu_si512((const void *)(y[i].qs + 64 * k));
        const __m512i dp = _mm512_sub_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), w, q8),
                                            _mm512_dpbusd_epi32(_mm512_setzero_si512(), n4, q8));
        sumi = _mm512_add_epi32(sumi, _mm512_mullo_epi32(dp, _mm512_permutexvar_epi32(idx[k], sc32)));
      }
    }
    const __m256i s8 = _mm256_add_epi32(_mm512_castsi512_si256(sumi), _mm512_extracti64x4_epi64(sumi, 1));
    acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(s8), acc);
  }
  return finish8(acc);
}

int zmo_cpu_has_avx512(void) {
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
         __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni") &&
         __builtin_cpu_supports("avx512dq");
}
#else
int zmo_cpu_has_avx512(void) { return 0; }
#endif

/* vec_dot with the AVX-512 kernels where the host has them (Q2_K, Q3_K); the
 * oracle dot otherwise.  Bit-identical either way. */
float zmo_vec_dot_q8_K_fast(int type, int n, const void *x, const zmo_block_q8_K *y) {
#if defined(__x86_64__)
  static int have = -1;
  if (have < 0) have = zmo_cpu_has_avx512();
  if (have && type == ZMO_TYPE_Q2_K) return dot_q2_K_avx512(n, (const zmo_block_q2_K *)x, y);
  if (have && type == ZMO_TYPE_Q3_K) return dot_q3_K_avx512(n, (const zmo_block_q3_K *)x, y);
#endif
  return zmo_vec_dot_q8_K(type, n, x, y);
}

/* The layer as ggml's CPU graph runs it (mul_mat_id gate, up, swiglu,
 * mul_mat_id down, mul, sum_topk; moe_routed_ggml.hpp:166-214): per token the
 * Q8_K of x on one thread, gate and up rows of all K routes split over the
 * threads in one parallel region, SwiGLU and the Q8_K of every route's act on
 * one thread, the down rows of all routes in a second region, then the
 * k-ascending weighted sum.  Same values as zmo_moe_forward, bit for bit
 * (no shared expert). */
void zmo_moe_forward_fast(const zmo_moe_desc *d, const float *x, const int32_t *ids, const float *weights,
                          float *out, int nthreads) {
  const int H = d->H, F = d->F, K = d->K, S = d->S;
  const size_t rg = zmo_row_size(d->type_gate, H), ru = zmo_row_size(d->type_up, H), rd = zmo_row_size(d->type_down, F);
  const size_t eg = rg * (size_t)F, eu = ru * (size_t)F, ed = rd * (size_t)H;
  const int nbH = H / ZMO_QK_K, nbF = F / ZMO_QK_K;
  zmo_block_q8_K *xq = (zmo_block_q8_K *)malloc(sizeof(zmo_block_q8_K) * (size_t)nbH);
  zmo_block_q8_K *aq = (zmo_block_q8_K *)malloc(sizeof(zmo_block_q8_K) * (size_t)nbF * (size_t)K);
  float *g = (float *)malloc(sizeof(float) * (size_t)F * (size_t)K * 3);
  float *u = g + (size_t)F * K, *a = u + (size_t)F * K;
  float *y = (float *)malloc(sizeof(float) * (size_t)H * (size_t)K);
  for (int s = 0; s < S; ++s) {
    const int32_t *id = ids + (size_t)s * K;
    zmo_quantize_row_q8_K(x + (size_t)s * H, xq, H);
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
    for (int r = 0; r < K * F; ++r) {
      const int k = r / F, nrow = r % F;
      if (id[k] < 0) continue;
      g[r] = zmo_vec_dot_q8_K_fast(d->type_gate, H, (const char *)d->w_gate + (size_t)id[k] * eg + (size_t)nrow * rg, xq);
      u[r] = zmo_vec_dot_q8_K_fast(d->type_up, H, (const char *)d->w_up + (size_t)id[k] * eu + (size_t)nrow * ru, xq);
    }
    for (int k = 0; k < K; ++k) {
      if (id[k] < 0) continue;
      zmo_swiglu(g + (size_t)k * F, u + (size_t)k * F, a + (size_t)k * F, F);
      zmo_quantize_row_q8_K(a + (size_t)k * F, aq + (size_t)k * nbF, F);
    }
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static)
    for (int r = 0; r < K * H; ++r) {
      const int k = r / H, h = r % H;
      y[r] = id[k] < 0 ? 0.0f
                       : zmo_vec_dot_q8_K_fast(d->type_down, F,
                                               (const char *)d->w_down + (size_t)id[k] * ed + (size_t)h * rd,
                                               aq + (size_t)k * nbF);
    }
    float *o = out + (size_t)s * H;
    for (int h = 0; h < H; ++h) {
      float acc = weights[(size_t)s * K] * y[h];
      for (int k = 1; k < K; ++k) acc = acc + weights[(size_t)s * K + k] * y[(size_t)k * H + h];
      o[h] = acc;
    }
  }
  free(y);
  free(g);
  free(aq);
  free(xq);
}
