// zm_mmq.hpp -- bucketed MUL_MAT_ID for prefill-sized buckets on int8 MFMA.
//
// Per active expert, out[pair][row] = W_e[row] . q8(x[pair]) for the pairs of
// the expert's bucket (the CSR of /root/reference/core/batched_dispatch_pipeline.cpp:1181-1202),
// gate/up optionally fused with SwiGLU (moe_routed_ggml.hpp:166-191).
//
// Tile: one wave computes 16 tokens x 16 weight rows with
// v_mfma_i32_16x16x32_i8, tokens as the A operand and weight rows as the B
// operand, so every lane's four outputs belong to ONE weight row (lane % 16)
// whose scales the lane has decoded itself.  A Q4_K sub-block (32 weights,
// one 6-bit scale and min) is exactly one MFMA K step:
//   isum[t][r] += sc[r][sb] * (q[r] . x[t])_sb            (int32, exact)
//   imin[t][r]  = sum_sb bsum[t][sb] * m[r][sb]           (v_mfma_f32_16x16x4f32;
//                 |terms| < 2^18, sums < 2^24: exact in fp32)
//   f[t][r]    += d_x[t] * (d[r] * isum - dmin[r] * imin)  (ggml's vec_dot_q4_K_q8_K combine)
// The weight nibbles feed the MFMA directly (0..15 as int8): no dequantized
// copy is materialized.  Activations are the planar Q8_K rows of the decode
// path (qs | bsums | d).
#pragma once

#include "zm_kernels.hpp"

namespace zm {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

constexpr int MMQ_TT = 4;  // 16-token tiles per pass over the weights

__device__ __forceinline__ long u2l(uint2 v) { return (long)(((unsigned long)v.y << 32) | v.x); }

template <bool GATEUP>
__global__ __launch_bounds__(256) void k_mmq_q4k(GemvArgs a) {
  int e, p0, p1;
  if (a.dense_S > 0) {
    if (blockIdx.y > 0) return;
    e = 0;
    p0 = 0;
    p1 = a.dense_S;
  } else {
    if ((int)blockIdx.y >= *a.n_active) return;
    e = a.active[blockIdx.y];
    p0 = a.offs[e];
    p1 = a.offs[e + 1];
  }
  constexpr int NM = GATEUP ? 2 : 1;
  constexpr int BB = 144;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * 64 + wave * 16 + n;  // weight row of this lane (B operand, output column)
  const bool rv = row < a.nrows;
  const uint32_t wbytes = (uint32_t)((size_t)a.nrows * a.w_rstride);
  rsrc_t rw[NM];
  rw[0] = make_rsrc(a.w0 + (size_t)e * a.w_estride, wbytes);
  if constexpr (GATEUP) rw[1] = make_rsrc(a.w1 + (size_t)e * a.w_estride, wbytes);
  const int vrow = rv ? row * (int)a.w_rstride : OOR;
  const int Kp = a.dense_S > 0 ? 1 : a.K;

  for (int pc = p0; pc < p1; pc += 16 * MMQ_TT) {
    const int nt = min(MMQ_TT, (p1 - pc + 15) / 16);
    // x row of this lane's A token (pair pc + 16t + n) and of its four output
    // tokens (pairs pc + 16t + 4g + j), per tile
    const uint8_t *xa[MMQ_TT];
    bool va[MMQ_TT];
    const uint8_t *xo[MMQ_TT][4];
    int po[MMQ_TT][4];
#pragma unroll
    for (int t = 0; t < MMQ_TT; ++t) {
      auto xrow_of = [&](int p, bool &ok) {
        ok = p < p1;
        const int pair = a.dense_S > 0 ? (ok ? p : p0) : a.pairs[ok ? p : p0];
        const int tok = pair / Kp, k = pair % Kp;
        return a.xq + (size_t)(tok * a.ne11 + k % a.ne11) * a.xq_rstride;
      };
      xa[t] = xrow_of(pc + 16 * t + n, va[t]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bool ok;
        const int p = pc + 16 * t + 4 * g + j;
        xo[t][j] = xrow_of(p, ok);
        po[t][j] = ok ? (a.dense_S > 0 ? p : a.pairs[p]) : -1;
      }
    }
    float f[NM][MMQ_TT][4];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int t = 0; t < MMQ_TT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) f[m][t][j] = 0.f;

    for (int b = 0; b < a.nb; ++b) {
      // weights of this lane's row, block b: header and the 8-byte qs chunks
      // 32i + 8g (i = 0..3; low nibbles: sub-block 2i, high: 2i+1)
      uint4 hdr[NM];
      uint2 qs[NM][4];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        hdr[m] = bld16(rw[m], vrow + b * BB, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[m][i] = bld8(rw[m], vrow + b * BB + 16 + 32 * i + 8 * g, 0);
      }
      // activations of the pass: A fragments (x bytes 64i + 8g and 64i + 32 + 8g),
      // 32-weight bsums of sub-blocks g and g + 4, d of the output tokens
      uint2 xl[MMQ_TT][4], xh[MMQ_TT][4];
      float bs_a[MMQ_TT][2], xd[MMQ_TT][4];
      const int nb = a.nb;
#pragma unroll
      for (int t = 0; t < MMQ_TT; ++t) {
        if (t < nt) {
          const uint8_t *xq = xa[t] + (size_t)b * QK;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xl[t][i] = va[t] ? ld8(xq + 64 * i + 8 * g) : make_uint2(0, 0);
            xh[t][i] = va[t] ? ld8(xq + 64 * i + 32 + 8 * g) : make_uint2(0, 0);
          }
          const int16_t *bs = reinterpret_cast<const int16_t *>(xa[t] + q8_bs_off(nb)) + b * 16;
          bs_a[t][0] = va[t] ? (float)(bs[2 * g] + bs[2 * g + 1]) : 0.f;
          bs_a[t][1] = va[t] ? (float)(bs[2 * g + 8] + bs[2 * g + 9]) : 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) xd[t][j] = reinterpret_cast<const float *>(xo[t][j] + q8_d_off(nb))[b];
        }
      }
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const uint32_t u0 = hdr[m].y, u1 = hdr[m].z, u2 = hdr[m].w;
        const uint32_t sc_lo = u0 & 0x3f3f3f3fu, mn_lo = u1 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_hi = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
        const float d = h2f((uint16_t)(hdr[m].x & 0xffffu)), dmin = h2f((uint16_t)(hdr[m].x >> 16));
        // B operand of the min product: m[row][sb] for sb = g and g + 4
        const float mb0 = (float)((mn_lo >> (8 * g)) & 0xffu), mb1 = (float)((mn_hi >> (8 * g)) & 0xffu);
#pragma unroll
        for (int t = 0; t < MMQ_TT; ++t) {
          if (t >= nt) continue;
          int isum[4] = {0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint2 q = qs[m][i];
            const long wl = u2l(make_uint2(q.x & 0x0f0f0f0fu, q.y & 0x0f0f0f0fu));
            const long wh = u2l(make_uint2((q.x >> 4) & 0x0f0f0f0fu, (q.y >> 4) & 0x0f0f0f0fu));
            const v4i_t z = {0, 0, 0, 0};
            const v4i_t dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(u2l(xl[t][i]), wl, z, 0, 0, 0);
            const v4i_t dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(u2l(xh[t][i]), wh, z, 0, 0, 0);
            const uint32_t scw = i < 2 ? sc_lo : sc_hi;
            const int s0 = (int)((scw >> (16 * (i & 1))) & 0xffu), s1 = (int)((scw >> (16 * (i & 1) + 8)) & 0xffu);
#pragma unroll
            for (int j = 0; j < 4; ++j) isum[j] += __mul24(s0, dl[j]) + __mul24(s1, dh[j]);
          }
          v4f_t mn = {0.f, 0.f, 0.f, 0.f};
          mn = __builtin_amdgcn_mfma_f32_16x16x4f32(bs_a[t][0], mb0, mn, 0, 0, 0);
          mn = __builtin_amdgcn_mfma_f32_16x16x4f32(bs_a[t][1], mb1, mn, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) f[m][t][j] += xd[t][j] * (d * (float)isum[j] - dmin * mn[j]);
        }
      }
    }
    // lane holds (token pc + 16t + 4g + j, row): store out[tok][k][row]
    if (rv) {
#pragma unroll
      for (int t = 0; t < MMQ_TT; ++t) {
        if (t >= nt) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int pair = po[t][j];
          if (pair < 0) continue;
          const int tok = pair / Kp, k = pair % Kp;
          const float v = GATEUP ? silu_f32(f[0][t][j]) * f[NM - 1][t][j] : f[0][t][j];
          a.out[(size_t)tok * a.out_s + (size_t)k * a.out_k + row] = v;
        }
      }
    }
  }
}

}  // namespace zm
