// zm_f32.hpp -- the FP32-activation side of the expert path: quantized
// weights times unquantized f32 activations (the per-type launchers and the
// FP32 MUL_MAT_ID hook), the stand-alone SwiGLU with its non-finite counters,
// the scatter-accumulate of expert rows into token rows, and the GLM5Next
// router post-processing.  None of these quantize the activations: they are
// the reference's CUDA-executor semantics
// (/root/reference/kernels/quant/kquant_matmul.cu:575-700,
//  kernels/math/expert_activation.cu:31-70, kernels/math/expert_accum.cu:22-60,
//  kernels/models/glm5next_router.cu:33-105), not ggml's CPU ones.
#pragma once

#include "zm_device.hpp"

namespace zm {

// ============================================================ per-lane dequant
//
// One wave covers one 256-weight super-block: lane l owns weights 4l..4l+3.
// The x slice of a lane is then one float4, contiguous across the wave (LDS
// reads without bank conflicts) and reused for every row the wave holds.
// Formulas: ggml's dequantize_row_* (restated from
// /root/reference/kernels/quant/kquant_matmul.cu:55-92,161-200 and
// kernels/quant/iq2_matmul.cu:73-91): w = d*sc*q - dmin*m for Q2_K/Q4_K,
// d*(sc-32)*(q - 4*!h) for Q3_K, d*sc*(q | h<<4) - dmin*m for Q5_K,
// (d*(ls-32))*table[q] for IQ4_XS (kernels/quant/iq4xs_matmul.cu:80-99),
// d*(0.5+s)*0.5*grid*sign for IQ3_XXS (kernels/quant/iq3_matmul.cu:104-122),
// (d*sc)*(q6 - 32) for Q6_K (kquant_matmul.cu:94-147), d*(0.5+s)*0.25*grid*sign
// for IQ2_XXS.
__device__ __forceinline__ uint32_t byte_at(const uint8_t *p) { return *p; }

template <int T>
__device__ __forceinline__ float4 deq4(const uint8_t *blk, int lane, const uint64_t *s_grid) {
  float w[4];
  if constexpr (T == T_Q2_K) {
    const int half = lane >> 5, j = (lane >> 3) & 3, lo = (lane & 7) * 4;
    const uint32_t q = ld4(blk + 16 + 32 * half + lo);
    const uint32_t sc = byte_at(blk + 8 * half + 2 * j + (lo >> 4));
    const uint32_t dd = ld4(blk + 80);
    const float dl = h2f((uint16_t)dd) * (float)(sc & 15);
    const float ml = h2f((uint16_t)(dd >> 16)) * (float)(sc >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = dl * (float)((q >> (8 * i + 2 * j)) & 3) - ml;
  } else if constexpr (T == T_Q3_K) {
    const int half = lane >> 5, j = (lane >> 3) & 3, lo = (lane & 7) * 4;
    const uint32_t q = ld4(blk + 32 + 32 * half + lo);
    const uint32_t hm = ld4(blk + lo);
    const int si = 8 * half + 2 * j + (lo >> 4);
    const uint32_t low4 = si < 8 ? (byte_at(blk + 96 + si) & 15) : (byte_at(blk + 96 + si - 8) >> 4);
    const uint32_t high2 = (byte_at(blk + 104 + (si & 3)) >> (2 * (si >> 2))) & 3;
    const float dl = h2f(ld2(blk + 108)) * (float)((int)(low4 | (high2 << 4)) - 32);
    const int bit = 4 * half + j;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int qv = (int)((q >> (8 * i + 2 * j)) & 3) - (((hm >> (8 * i + bit)) & 1) ? 0 : 4);
      w[i] = dl * (float)qv;
    }
  } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
    const int j = lane >> 4, l = (4 * lane) & 63, hi = l >> 5;
    constexpr int QS = T == T_Q5_K ? 48 : 16;
    const uint32_t q = ld4(blk + QS + 32 * j + (l & 31));
    uint32_t nib = hi ? ((q >> 4) & 0x0f0f0f0fu) : (q & 0x0f0f0f0fu);
    if constexpr (T == T_Q5_K) nib |= ((ld4(blk + 16 + (l & 31)) >> (2 * j + hi)) & 0x01010101u) << 4;
    const int sub = 2 * j + hi;
    const uint8_t *s = blk + 4;
    uint32_t sc, m;
    if (sub < 4) {
      sc = byte_at(s + sub) & 63;
      m = byte_at(s + sub + 4) & 63;
    } else {
      sc = (byte_at(s + sub + 4) & 15) | ((byte_at(s + sub - 4) >> 6) << 4);
      m = (byte_at(s + sub + 4) >> 4) | ((byte_at(s + sub) >> 6) << 4);
    }
    const uint32_t dd = ld4(blk);
    const float d1 = h2f((uint16_t)dd) * (float)sc;
    const float m1 = h2f((uint16_t)(dd >> 16)) * (float)m;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = d1 * (float)((nib >> (8 * i)) & 31) - m1;
  } else if constexpr (T == T_Q6_K) {
    // weights 4*lane.. = 128h + 32g + l..l+3
    const int h = lane >> 5, g = (lane >> 3) & 3, l = (4 * lane) & 31;
    const uint32_t q = ld4(blk + 64 * h + 32 * (g & 1) + l);
    const uint32_t lo = g < 2 ? (q & 0x0f0f0f0fu) : ((q >> 4) & 0x0f0f0f0fu);
    const uint32_t v = lo | (((ld4(blk + 128 + 32 * h + l) >> (2 * g)) & 0x03030303u) << 4);
    const int sc = (int)(int8_t)byte_at(blk + 192 + 8 * h + 2 * g + (l >> 4));
    const float dl = h2f(ld2(blk + 208)) * (float)sc;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = dl * (float)((int)((v >> (8 * i)) & 63) - 32);
  } else if constexpr (T == T_IQ3_XXS) {
    // weights 4*lane.. = sub-block ib, group l, half h: grid entry
    // qs[8ib + 2l + h], signs ksigns[(u >> 7l) & 127] bits 4h..4h+3
    const int ib = lane >> 3, l = (lane >> 1) & 3, h = lane & 1;
    const uint32_t idx = byte_at(blk + 2 + 8 * ib + 2 * l + h);
    const uint32_t u = ld4(blk + 66 + 4 * ib);
    const float db = h2f(ld2(blk)) * (0.5f + (float)(u >> 28)) * 0.5f;
    const uint32_t gv = reinterpret_cast<const uint32_t *>(s_grid)[idx];
    const uint32_t si = (u >> (7 * l)) & 127;
    const uint32_t signs = si | ((__builtin_popcount(si) & 1) << 7);  // ksigns_iq2xs
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = db * (float)((gv >> (8 * i)) & 255);
      w[i] = ((signs >> (4 * h + i)) & 1) ? -v : v;
    }
  } else if constexpr (T == T_IQ4_XS) {
    // weights 4*lane.. = sub-block ib, positions j0..j0+3: low nibbles of qs
    // bytes 16ib + j0.. for j0 < 16, high nibbles of 16ib + j0 - 16.. otherwise
    const int ib = lane >> 3, j0 = (4 * lane) & 31;
    const uint32_t q = ld4(blk + 8 + 16 * ib + (j0 & 15));
    const uint32_t idx = j0 < 16 ? (q & 0x0f0f0f0fu) : ((q >> 4) & 0x0f0f0f0fu);
    const uint32_t hdr = ld4(blk), sl = ld4(blk + 4);
    const float dl = h2f((uint16_t)(hdr & 0xffffu)) * (float)iq4_scale(hdr, sl, ib);
    const uint32_t v = lut16(idx, (uint32_t)s_grid[0], (uint32_t)(s_grid[0] >> 32), (uint32_t)s_grid[1],
                             (uint32_t)(s_grid[1] >> 32));
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = dl * (float)(int)(int8_t)(v >> (8 * i));
  } else {  // IQ2_XXS
    const int ib = lane >> 3, l = (lane >> 1) & 3, hb = lane & 1;
    const uint32_t a0 = ld4(blk + 2 + 8 * ib), a1 = ld4(blk + 6 + 8 * ib);
    const float db = h2f(ld2(blk)) * (0.5f + (float)(a1 >> 28)) * 0.25f;
    const uint64_t g = s_grid[(a0 >> (8 * l)) & 255];
    const uint32_t gv = (uint32_t)(g >> (32 * hb));
    const uint32_t si = (a1 >> (7 * l)) & 127;
    const uint32_t signs = si | ((__builtin_popcount(si) & 1) << 7);  // ksigns_iq2xs
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = db * (float)((gv >> (8 * i)) & 255);
      w[i] = ((signs >> (4 * hb + i)) & 1) ? -v : v;
    }
  }
  return make_float4(w[0], w[1], w[2], w[3]);
}

// ============================================================ f32 matmul
//
// y[tok, route, o] = sum_i W[m][o][i] * x[tok, route % x_routes, i], where the
// matrix m is ids[tok, route] (MUL_MAT_ID; m < 0 -> 0, m >= E -> NaN, as
// native_f32_matmul_id, kquant_matmul.cu:656-664), `route` for the grouped
// form, 0 for the plain launchers.  Grid: x = row groups of 4 waves x RPW rows,
// y = token tiles of NT (NT = 1 with ids), z = routes.  x is staged in LDS
// CH super-blocks at a time; each wave dequantizes its RPW rows once per block
// and applies them to all NT tokens.  Sum order: per lane sequential over
// blocks, then a fixed wave tree (deterministic, not the reference's order).
struct F32MMArgs {
  const uint8_t *w;
  size_t w_row, w_mat;           // bytes
  const float *x;
  size_t x_tok, x_route;         // floats
  int x_routes;
  float *y;
  size_t y_tok, y_route;         // floats
  const uint8_t *ids;            // I32, null: no ids
  size_t id_tok, id_route;       // bytes
  int E;
  int I, O, n_tok;
  int mat_by_route;              // no ids: matrix = route (grouped) or 0
  const uint64_t *grid;
};

constexpr int F32_CH = 16;
constexpr int F32_RPW = 4;

template <int T, int NT>
__global__ __launch_bounds__(256) void k_f32_mm(F32MMArgs a) {
  __shared__ float4 s_x[NT][F32_CH * 64];
  __shared__ uint64_t s_grid[T == T_IQ2_XXS ? 256 : (T == T_IQ3_XXS ? 128 : (T == T_IQ4_XS ? 2 : 1))];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int route = blockIdx.z, t0 = blockIdx.y * NT;
  const int row0 = (blockIdx.x * 4 + wave) * F32_RPW;
  int m = 0;
  if (a.ids) {
    m = *reinterpret_cast<const int32_t *>(a.ids + (size_t)t0 * a.id_tok + (size_t)route * a.id_route);
    if (m < 0 || m >= a.E) {
      if (lane < F32_RPW && row0 + lane < a.O)
        a.y[(size_t)t0 * a.y_tok + (size_t)route * a.y_route + row0 + lane] = m < 0 ? 0.0f : __int_as_float(0x7fc00000);
      return;  // uniform over the workgroup: no barrier follows
    }
  } else if (a.mat_by_route) {
    m = route;
  }
  if constexpr (T == T_IQ2_XXS) {
    s_grid[threadIdx.x] = a.grid[threadIdx.x];
  } else if constexpr (T == T_IQ3_XXS) {
    if (threadIdx.x < 128) s_grid[threadIdx.x] = a.grid[threadIdx.x];
  } else if constexpr (T == T_IQ4_XS) {
    if (threadIdx.x < 2) s_grid[threadIdx.x] = a.grid[threadIdx.x];
  }
  constexpr int BB = block_bytes(T);
  const int nb = a.I / QK;
  const uint8_t *wr[F32_RPW];
#pragma unroll
  for (int r = 0; r < F32_RPW; ++r) wr[r] = a.w + (size_t)m * a.w_mat + (size_t)min(row0 + r, a.O - 1) * a.w_row;
  const float *xr[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    xr[t] = a.x + (size_t)min(t0 + t, a.n_tok - 1) * a.x_tok + (size_t)(route % a.x_routes) * a.x_route;
  float acc[F32_RPW][NT];
#pragma unroll
  for (int r = 0; r < F32_RPW; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[r][t] = 0.0f;

  for (int c0 = 0; c0 < nb; c0 += F32_CH) {
    const int cn = min(F32_CH, nb - c0);
    for (int v = threadIdx.x; v < cn * 64; v += 256) {
#pragma unroll
      for (int t = 0; t < NT; ++t) s_x[t][v] = reinterpret_cast<const float4 *>(xr[t] + (size_t)c0 * QK)[v];
    }
    __syncthreads();
#pragma unroll 2
    for (int b = 0; b < cn; ++b) {
      float4 wv[F32_RPW];
#pragma unroll
      for (int r = 0; r < F32_RPW; ++r) wv[r] = deq4<T>(wr[r] + (size_t)(c0 + b) * BB, lane, s_grid);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float4 xv = s_x[t][b * 64 + lane];
#pragma unroll
        for (int r = 0; r < F32_RPW; ++r)
          acc[r][t] += ((wv[r].x * xv.x + wv[r].y * xv.y) + (wv[r].z * xv.z + wv[r].w * xv.w));
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < F32_RPW; ++r)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float v = group_sum<64>(acc[r][t]);
      if (lane == 0 && row0 + r < a.O && t0 + t < a.n_tok)
        a.y[(size_t)(t0 + t) * a.y_tok + (size_t)route * a.y_route + row0 + r] = v;
    }
}

// ============================================================ SwiGLU
// prod = clamp(silu(g) * u) (default) or silu(min(g, L)) * clamp(u) (fused
// clamp), clamp applied when > 0; bad[0] += #(g or u NaN), bad[1] += #(else
// g or u Inf)  (kernels/math/expert_activation.cu:31-59).  One counter update
// per wave.
__global__ __launch_bounds__(256) void k_swiglu(float *__restrict__ prod, const float *__restrict__ gate,
                                                const float *__restrict__ up, int n, float clamp, int fused,
                                                int *__restrict__ bad) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const bool in = i < n;
  const float g0 = in ? gate[i] : 0.0f, u0 = in ? up[i] : 0.0f;
  const bool is_nan = __builtin_isnan(g0) || __builtin_isnan(u0);
  const bool is_inf = !is_nan && (__builtin_isinf(g0) || __builtin_isinf(u0));
  if (bad) {
    const int nn = __builtin_popcountll(__ballot(is_nan)), ni = __builtin_popcountll(__ballot(is_inf));
    if ((threadIdx.x & 63) == 0) {
      if (nn) atomicAdd(&bad[0], nn);
      if (ni) atomicAdd(&bad[1], ni);
    }
  }
  if (!in) return;
  float g = g0, u = u0, out;
  if (fused) {
    if (clamp > 0.0f) {
      g = fminf(g, clamp);
      u = fmaxf(-clamp, fminf(clamp, u));
    }
    out = g / (1.0f + exp_f32(-g)) * u;
  } else {
    out = g / (1.0f + exp_f32(-g)) * u;
    if (clamp > 0.0f) out = fmaxf(-clamp, fminf(clamp, out));
  }
  prod[i] = out;
}

// ============================================================ scatter-accumulate
// dst[tok[i]][d] += w[i] * src[i][d] (w null: += src), rows with tok outside
// [0, S) skipped (kernels/math/expert_accum.cu:22-37).  One workgroup per
// source row; rows of one call must target distinct tokens (no atomics).
__global__ __launch_bounds__(256) void k_scatter_accum(const float *__restrict__ src, const int *__restrict__ tok,
                                                       const float *__restrict__ w, float *__restrict__ dst, int D,
                                                       int S) {
  const int i = blockIdx.x;
  const int s = tok[i];
  if (s < 0 || s >= S) return;
  const float wt = w ? w[i] : 1.0f;
  const float *sr = src + (size_t)i * D;
  float *ds = dst + (size_t)s * D;
  for (int d = threadIdx.x; d < D; d += 256) ds[d] = __builtin_fmaf(wt, sr[d], ds[d]);
}

// ============================================================ GLM5Next router top-k
// Per token: probs = softmax(logits) | gate(logits) written back over the
// logits; K rounds of "best = argmax(prob + bias), ties to the lower index";
// weight = unbiased prob; the chosen prob is then replaced by -FLT_MAX (also
// in the written-back row); optional 1/max(sum, 2^-14) normalisation and
// scale (kernels/models/glm5next_router.cu:33-93).  NaN scores are never
// chosen, except expert 0 when its score is NaN (the reference scan seeds its
// running best with expert 0).  One wave per token; the row sits in LDS.
constexpr int GLM_MAX_E = 4096;
__global__ __launch_bounds__(64) void k_glm_router_topk(float *__restrict__ logits, const float *__restrict__ bias,
                                                        int32_t *__restrict__ ids, float *__restrict__ weights, int E,
                                                        int K, int gating, int normalize, float scale) {
  __shared__ float row[GLM_MAX_E];
  __shared__ int s_id[64];
  __shared__ float s_w[64];
  const int s = blockIdx.x, lane = threadIdx.x;
  float *lr = logits + (size_t)s * E;
  if (gating == 0) {
    float mx = -__builtin_inff();
    for (int e = lane; e < E; e += 64) {
      row[e] = lr[e];
      mx = fmaxf(mx, row[e]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int e = lane; e < E; e += 64) {
      const float v = exp_f32(row[e] - mx);
      row[e] = v;
      sum += v;
    }
    sum = group_sum<64>(sum);
    const float inv = 1.0f / sum;
    for (int e = lane; e < E; e += 64) row[e] *= inv;
  } else {
    for (int e = lane; e < E; e += 64) {
      const float x = lr[e];
      float v;
      if (gating == 1) {
        v = 1.0f / (1.0f + exp_f32(-x));
      } else if (gating == 2) {
        const float sp = x > 0.0f ? x + log1pf(exp_f32(-x)) : log1pf(exp_f32(x));
        v = sqrtf(sp);
      } else {
        v = x;
      }
      row[e] = v;
    }
  }
  stage_sync();
  const float NEG = -3.402823466e+38f;
  for (int k = 0; k < K; ++k) {
    unsigned long long best = 0;
    for (int e = lane; e < E; e += 64) {
      const float sc = row[e] + (bias ? bias[e] : 0.0f);
      if (sc == sc) {
        const unsigned long long key = rank_key(sc, e);
        best = key > best ? key : best;
      }
    }
    best = wave_max_u64(best);
    const float s0 = row[0] + (bias ? bias[0] : 0.0f);
    const int b = (s0 != s0 || best == 0) ? 0 : (int)(0xffffffffu - (uint32_t)best);
    const float p = row[b];
    stage_sync();
    if (lane == 0) {
      s_id[k] = b;
      s_w[k] = p;
      row[b] = NEG;
    }
    stage_sync();
  }
  for (int e = lane; e < E; e += 64) lr[e] = row[e];
  if (lane == 0) {
    float sum = 0.0f;
    for (int k = 0; k < K; ++k) sum += s_w[k];
    const float inv = 1.0f / fmaxf(sum, 6.103515625e-5f);
    for (int k = 0; k < K; ++k) {
      float v = s_w[k];
      if (normalize) v *= inv;
      if (scale != 0.0f) v *= scale;
      ids[(size_t)s * K + k] = s_id[k];
      weights[(size_t)s * K + k] = v;
    }
  }
}

}  // namespace zm
