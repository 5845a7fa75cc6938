// zm_kernels.hpp -- the routed-expert kernels for gfx950 (wave64, CDNA4).
//
//   k_quant_q8K  : f32 rows -> Q8_K (16 lanes per 256-value block)
//   k_router     : gating + (grouped) top-k + weights + slot table, one wave per token
//   k_bucket     : stable counting sort of (token, slot) pairs by expert
//   k_gemv       : bucketed MUL_MAT_ID GEMV over Q8_K activations (decode path)
//   k_combine    : k-ascending weighted sum over the top-k axis (+ shared expert)
//   k_router_gemv: fp32 router logits
#pragma once

#include "zm_device.hpp"

// The non-template kernels below have internal linkage: this header is
// included by more than one translation unit (the decode-kernel instantiation
// units take its device functions only).

namespace zm {

// ============================================================ Q8_K quantization
//
// ggml quantize_row_q8_K (restated in oracle/zm_oracle.c): the signed value of
// largest magnitude (first on ties) gives iscale = -127/max; q = min(127,
// round_half_even(iscale*x)); d = 1/iscale; bsums = sums of 16.
// Lane l of a 16-lane group holds values [16l, 16l+16) of the block, so the
// block's maximum takes four in-row DPP steps and each lane's 16 values are
// exactly one of the block's 16-sums.
struct Q8Out16 {
  uint4 q;     // 16 int8
  float d;
  int bsum;
};

__device__ __forceinline__ Q8Out16 quant_block16(const float (&x)[16], int l16) {
  // largest and smallest value of the block; a NaN drops out of fmaxf/fminf
  // exactly as it drops out of ggml's |x| > amax comparison
  float hi = x[0], lo = x[0];
#pragma unroll
  for (int j = 1; j < 16; ++j) {
    hi = fmaxf(hi, x[j]);
    lo = fminf(lo, x[j]);
  }
  hi = dpp_max_f<DPP_XOR1>(hi);
  lo = dpp_min_f<DPP_XOR1>(lo);
  hi = dpp_max_f<DPP_XOR2>(hi);
  lo = dpp_min_f<DPP_XOR2>(lo);
  hi = dpp_max_f<DPP_HALF_MIRROR>(hi);
  lo = dpp_min_f<DPP_HALF_MIRROR>(lo);
  hi = dpp_max_f<DPP_MIRROR>(hi);
  lo = dpp_min_f<DPP_MIRROR>(lo);
  const float amax = fmaxf(hi, -lo);
  Q8Out16 o;
  if (!(amax > 0.0f)) {  // all zero (or no finite/infinite value at all)
    o.q = make_uint4(0, 0, 0, 0);
    o.d = 0.0f;
    o.bsum = 0;
    return o;
  }
  // the signed value of largest magnitude; when +amax and -amax both occur,
  // the first in block order wins: each lane finds its first, the lowest lane
  // of the 16 with one decides
  float mx = hi > -lo ? hi : lo;
  if (hi == -lo) {
    int key = 64;  // (lane << 1 | negative) of this lane's first hit
#pragma unroll
    for (int j = 15; j >= 0; --j) key = __builtin_fabsf(x[j]) == amax ? (l16 << 1) | (x[j] < 0.f) : key;
    key = min(key, dpp_i<DPP_XOR1>(key));
    key = min(key, dpp_i<DPP_XOR2>(key));
    key = min(key, dpp_i<DPP_HALF_MIRROR>(key));
    key = min(key, dpp_i<DPP_MIRROR>(key));
    mx = (key & 1) ? lo : hi;
  }
  const float iscale = -127.f / mx;
  // ggml's q = min(127, nearest_int(v)) as a byte: nearest_int keeps the low
  // 23 bits of v + 1.5*2^23 less 2^22, so clamping those bits at 2^22 + 127
  // and keeping their low byte gives the same int8 for every input
  uint32_t t[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float v = iscale * x[j] + 12582912.f;
    t[j] = min(__float_as_uint(v) & 0x007fffffu, 0x0040007fu);
  }
  uint32_t w[4];
  int bs = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    w[k] = __builtin_amdgcn_perm(t[4 * k + 1], t[4 * k], 0x0c0c0400u) |
           __builtin_amdgcn_perm(t[4 * k + 3], t[4 * k + 2], 0x04000c0cu);
    bs = __builtin_amdgcn_sdot4((int)w[k], 0x01010101, bs, false);
  }
  o.q = make_uint4(w[0], w[1], w[2], w[3]);
  o.d = 1.0f / iscale;
  o.bsum = bs;
  return o;
}

// one Q8_K block (planar row layout) from the 16 values of this lane
__device__ __forceinline__ void store_q8_16(uint8_t *row, int nb, int blk, const Q8Out16 &o, int l16) {
  *reinterpret_cast<uint4 *>(row + (size_t)blk * QK + 16 * l16) = o.q;
  if (l16 == 0) reinterpret_cast<float *>(row + q8_d_off(nb))[blk] = o.d;
  reinterpret_cast<int16_t *>(row + q8_bs_off(nb))[blk * 16 + l16] = (int16_t)o.bsum;
}

// rows x nb blocks, 16 lanes per block (quant_block16); planar != 0 writes the
// internal planar layout, else ggml block_q8_K
static __global__ __launch_bounds__(256) void k_quant_q8K(const float *__restrict__ x, size_t x_rstride, int nb, int rows,
                                                   uint8_t *__restrict__ y, size_t y_rstride, int planar) {
  const int l16 = threadIdx.x & 15;
  const int gb = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int row = gb / nb, b = gb % nb;
  if (row >= rows) return;
  const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)row * x_rstride + (size_t)b * QK + 16 * l16);
  float v[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 f = src[i];
    v[4 * i] = f.x;
    v[4 * i + 1] = f.y;
    v[4 * i + 2] = f.z;
    v[4 * i + 3] = f.w;
  }
  const Q8Out16 o = quant_block16(v, l16);
  uint8_t *yr = y + (size_t)row * y_rstride;
  if (planar) {
    store_q8_16(yr, nb, b, o, l16);
  } else {
    uint8_t *blk = yr + (size_t)b * 292;
    __builtin_memcpy(blk + 4 + 16 * l16, &o.q, 16);
    if (l16 == 0) __builtin_memcpy(blk, &o.d, 4);
    const int16_t bs = (int16_t)o.bsum;
    __builtin_memcpy(blk + 260 + 2 * l16, &bs, 2);
  }
}

// ============================================================ router
//
// moe_routed::gate_probs / select_ids / route_weights
// (/root/reference/models/graph/moe_routed_ggml.hpp:52-141), with the grouped
// selection of core/moe_router_service.cpp:1409-1440 and the device router of
// kernels/models/glm5next_router.cu:33-93.  Top-k order: descending score,
// lowest expert index first on ties.
struct RouterArgs {
  const float *logits;      // [S][E]
  const float *logit_bias;  // [E] or null: added to logits before gating
  const float *sel_bias;    // [E] or null: added to probs for selection only
  const int32_t *route_map; // [E] or null: global expert -> slot (or -1)
  const float *route_mask;  // [E] or null
  int E, K, gating, n_groups, n_groups_used, weights_norm;
  float weights_scale;
  int32_t *ids;  // [S][K]
  float *weights;
};

__device__ __forceinline__ bool outranks(float sa, int ia, float sb, int ib) {
  return sa > sb || (sa == sb && ia < ib);
}

constexpr int ROUTER_MAX_E = 1024;

// One wave routes one token.  Expert e = lane + 64*i sits in register i of its
// lane (E <= 64*P).  Results: lane k < K holds route k (id after the slot
// table, weight normalised / scaled / masked).  `scr` is E floats of LDS
// private to the wave (used for grouped selection only).
struct WaveRoute {
  int id;
  float w;
};
template <int P>
__device__ __forceinline__ WaveRoute router_wave(const RouterArgs &a, int s, float *scr) {
  const int lane = threadIdx.x & 63;
  const int E = a.E, K = a.K;
  const float NEG_INF = __int_as_float(0xff800000);
  const float *l = a.logits + (size_t)s * E;
  float v[P], sb[P];
  int rm[P];
  float rk[P];
  // every global load of the router goes out first, unconditionally: an absent
  // array is a buffer resource of extent 0 (its loads return 0 and touch no memory)
  const uint32_t ext = (uint32_t)E * 4u;
  const rsrc_t r_l = make_rsrc(l, ext);
  const rsrc_t r_lb = make_rsrc(a.logit_bias, a.logit_bias ? ext : 0u);
  const rsrc_t r_sb = make_rsrc(a.sel_bias, a.sel_bias ? ext : 0u);
  const rsrc_t r_rm = make_rsrc(a.route_map, a.route_map ? ext : 0u);
  const rsrc_t r_rk = make_rsrc(a.route_mask, a.route_map && a.route_mask ? ext : 0u);
  float lb[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int e = lane + 64 * i;
    const int vo = e < E ? 4 * e : OOR;
    v[i] = __uint_as_float(bld4(r_l, vo, 0));
    lb[i] = __uint_as_float(bld4(r_lb, vo, 0));
    sb[i] = __uint_as_float(bld4(r_sb, vo, 0));
    rm[i] = (int)bld4(r_rm, vo, 0);
    rk[i] = __uint_as_float(bld4(r_rk, vo, 0));
  }
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const bool in = lane + 64 * i < E;
    v[i] = !in ? NEG_INF : (a.logit_bias ? v[i] + lb[i] : v[i]);
    rk[i] = a.route_mask ? rk[i] : 1.0f;
  }
  if (a.gating == 0) {
    float mx = v[0];
#pragma unroll
    for (int i = 1; i < P; ++i) mx = fmaxf(mx, v[i]);
    mx = wave_max(mx);
    double sum = 0.0;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      v[i] = lane + 64 * i < E ? exp_f32(v[i] - mx) : 0.0f;
      sum += (double)v[i];
    }
    sum = wave_sum_f64(sum);
    const float inv = (float)(1.0 / sum);
#pragma unroll
    for (int i = 0; i < P; ++i) v[i] = v[i] * inv;
  } else {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const float x = v[i];
      v[i] = a.gating == 1 ? 1.0f / (1.0f + exp_f32(-x)) : sqrtf(x > 0.0f ? x + log1pf(exp_f32(-x)) : log1pf(exp_f32(x)));
    }
  }
  // v = gate probabilities p; selection scores sel = p + sel_bias
  float sel[P];
#pragma unroll
  for (int i = 0; i < P; ++i) sel[i] = a.sel_bias ? v[i] + sb[i] : v[i];
  const int G = a.n_groups;
  if (G > 1 && a.n_groups_used > 0 && a.n_groups_used < G && E % G == 0 && G <= 64) {
    // group score = best + second best selection score of the group; keep the
    // n_groups_used best groups
    const int gs = E / G;
    float gsc = NEG_INF;
    if (gs == 16 || gs == 32 || gs == 64) {
      // a group is gs consecutive lanes of one register: two group-wide key
      // maxima, the first one's lowest lane taken out for the second; a score
      // is recovered from its key (the map is a bijection up to -0 -> +0).
      // Each phase runs over all registers before the next, so the P
      // independent DPP chains interleave.
      auto groups = [&](auto gs_tag) {
        constexpr int GS = decltype(gs_tag)::value;
        const int base = lane & ~(GS - 1);
        const unsigned long long gmask = (GS == 64 ? ~0ull : ((1ull << (GS & 63)) - 1ull)) << base;
        uint32_t k0[P], k1[P];
#pragma unroll
        for (int i = 0; i < P; ++i) k0[i] = lane + 64 * i < E ? score_key(sel[i]) : 0u;
#pragma unroll
        for (int i = 0; i < P; ++i) k1[i] = group_max_u32(k0[i], GS);
#pragma unroll
        for (int i = 0; i < P; ++i) {
          const unsigned long long b1 = __ballot(lane + 64 * i < E && k0[i] == k1[i]) & gmask;
          const bool first = b1 != 0ull && lane == (int)__builtin_ctzll(b1);
          k0[i] = first ? 0u : k0[i];
        }
#pragma unroll
        for (int i = 0; i < P; ++i) k0[i] = group_max_u32(k0[i], GS);
#pragma unroll
        for (int i = 0; i < P; ++i)
          if (lane + 64 * i < E && (lane & (GS - 1)) == 0)
            scr[(lane + 64 * i) / GS] = score_from_key(k1[i]) + score_from_key(k0[i]);
      };
      if (gs == 16) groups(std::integral_constant<int, 16>{});
      else if (gs == 32) groups(std::integral_constant<int, 32>{});
      else groups(std::integral_constant<int, 64>{});
      stage_sync();
      if (lane < G) gsc = scr[lane];
    } else {
      // lane g scans group g
#pragma unroll
      for (int i = 0; i < P; ++i)
        if (lane + 64 * i < E) scr[lane + 64 * i] = sel[i];
      stage_sync();
      if (lane < G) {
        int b1 = -1, b2 = -1;
        float s1 = 0.f, s2 = 0.f;
        for (int j = 0; j < gs; ++j) {
          const int e = lane * gs + j;
          const float x = scr[e];
          if (b1 < 0 || outranks(x, e, s1, b1)) {
            b2 = b1;
            s2 = s1;
            b1 = e;
            s1 = x;
          } else if (b2 < 0 || outranks(x, e, s2, b2)) {
            b2 = e;
            s2 = x;
          }
        }
        gsc = gs >= 2 ? s1 + s2 : s1;
      }
    }
    int r = 0;
    for (int g2 = 0; g2 < G; ++g2) r += outranks(readlane_f(gsc, g2), g2, gsc, lane);
    const unsigned long long keep = __ballot(lane < G && r < a.n_groups_used);
#pragma unroll
    for (int i = 0; i < P; ++i)
      if (!((keep >> ((lane + 64 * i) / gs)) & 1ull)) sel[i] = NEG_INF;
    stage_sync();  // scr is reused by the caller
  }
  // top-K in the order "higher score, then lower expert index"
  uint32_t key[P];
#pragma unroll
  for (int i = 0; i < P; ++i) key[i] = lane + 64 * i < E ? score_key(sel[i]) : 0u;
  uint32_t valid = 0;
#pragma unroll
  for (int i = 0; i < P; ++i) valid |= (lane + 64 * i < E ? 1u : 0u) << i;
  int myid = 0;
  float myw = 0.f, mymask = 1.0f;
  // Fast path (K <= 16): a lower bound L on the K-th largest key is the
  // smallest of NS >= K subset maxima (NS distinct experts are >= it); only
  // the experts with key >= L can be selected.  When at most 64 remain they
  // are compacted in index order into LDS and each is ranked against all of
  // them at once (independent compares instead of K dependent wave-wide
  // rounds); the ranks < K are the routes, in order.
  bool routed = false;
  if (K <= 16) {
    uint32_t lm = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) lm = ((valid >> i) & 1u) && key[i] > lm ? key[i] : lm;
    lm = max(lm, (uint32_t)dpp_i<DPP_XOR1>((int)lm));
    lm = max(lm, (uint32_t)dpp_i<DPP_XOR2>((int)lm));  // maxima of 16 subsets of 4 lanes
    if (K <= 8) {
      lm = max(lm, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)lm));  // 8 subsets of 8 lanes
    } else {
      lm = min(lm, (uint32_t)dpp_i<DPP_HALF_MIRROR>((int)lm));
    }
    lm = min(lm, (uint32_t)dpp_i<DPP_MIRROR>((int)lm));
    const uint32_t L = min(min((uint32_t)__builtin_amdgcn_readlane((int)lm, 0), (uint32_t)__builtin_amdgcn_readlane((int)lm, 16)),
                           min((uint32_t)__builtin_amdgcn_readlane((int)lm, 32), (uint32_t)__builtin_amdgcn_readlane((int)lm, 48)));
    unsigned long long bal[P];
    int C = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      bal[i] = __ballot(((valid >> i) & 1u) && key[i] >= L);
      C += __popcll(bal[i]);
    }
    if (C >= K && C <= 64) {
      uint32_t *ck = reinterpret_cast<uint32_t *>(scr);  // [0,64) keys, [64,128) ids, [128,192) p, [192,256) slot, [256,320) mask
      uint32_t *co = ck + 320;                           // [320,384): routes (id, p, slot, mask) x 16
      int base = 0;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        if ((bal[i] >> lane) & 1ull) {
          const int pos = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal[i] >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)bal[i], 0));
          ck[pos] = key[i];
          ck[64 + pos] = (uint32_t)(lane + 64 * i);
          ck[128 + pos] = __float_as_uint(v[i]);
          ck[192 + pos] = (uint32_t)rm[i];
          ck[256 + pos] = __float_as_uint(rk[i]);
        }
        base += __popcll(bal[i]);
      }
      if (lane >= C) ck[lane] = 0u;  // all 64 key slots defined; padding never outranks
      stage_sync();
      // rank = candidates before this one in (key descending, position
      // ascending) order.  First the larger keys (one compare and one
      // carry-add per candidate, 16 keys read per step); the counts are then
      // 0..C-1 exactly when no key repeats, else the equal keys at earlier
      // positions are added
      int rank = 0;
      uint32_t mk = 0;
      if (lane < C) {
        mk = ck[lane];
        for (int t = 0; t < C; t += 16) {
          uint4 kt[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) kt[q] = *reinterpret_cast<const uint4 *>(ck + t + 4 * q);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t kq[4] = {kt[q].x, kt[q].y, kt[q].z, kt[q].w};
#pragma unroll
            for (int u = 0; u < 4; ++u)
              asm("v_cmp_gt_u32_e32 vcc, %1, %2\n\tv_addc_co_u32_e32 %0, vcc, 0, %0, vcc"
                  : "+v"(rank)
                  : "v"(kq[u]), "v"(mk)
                  : "vcc");
          }
        }
      }
      if (group_sum_i<64>(rank) != C * (C - 1) / 2 && lane < C)
        for (int t = 0; t < lane; ++t) rank += ck[t] == mk;
      if (lane < C && rank < K) {
        co[4 * rank] = ck[64 + lane];
        co[4 * rank + 1] = ck[128 + lane];
        co[4 * rank + 2] = ck[192 + lane];
        co[4 * rank + 3] = ck[256 + lane];
      }
      stage_sync();
      if (lane < K) {
        const int e = (int)co[4 * lane];
        myw = __uint_as_float(co[4 * lane + 1]);
        myid = e;
        if (a.route_map) {
          myid = (int)co[4 * lane + 2];
          mymask = a.route_mask ? __uint_as_float(co[4 * lane + 3]) : (myid >= 0 ? 1.0f : 0.0f);
        }
      }
      stage_sync();  // scr is reused by the caller
      routed = true;
    }
  }
  // General path: K rounds of a wave-wide 32-bit score-key maximum; the winner
  // is the lowest expert index holding it (register i = 0 first, then the
  // lowest lane in the ballot)
  for (int k = 0; !routed && k < K; ++k) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) m = ((valid >> i) & 1u) && key[i] >= m ? key[i] : m;
    const uint32_t best = wave_max_u32(m);
    int e = 0;
#pragma unroll
    for (int i = P - 1; i >= 0; --i) {
      const unsigned long long bal = __ballot(((valid >> i) & 1u) && key[i] == best);
      e = bal ? (int)__builtin_ctzll(bal) + 64 * i : e;
    }
    const int owner = e & 63, iw = e >> 6;
    // the owner lane takes the winner's values out of its registers (selects,
    // not an indexed register read, so the arrays stay in registers)
    float pw = 0.f, rkw = 1.0f;
    int rmw = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool hit = i == iw;
      pw = hit ? v[i] : pw;
      rmw = hit ? rm[i] : rmw;
      rkw = hit ? rk[i] : rkw;
      if (hit && lane == owner) valid &= ~(1u << i);
    }
    pw = readlane_f(pw, owner);
    int id = e;
    float msk = 1.0f;
    if (a.route_map) {
      id = __builtin_amdgcn_readlane(rmw, owner);
      msk = a.route_mask ? readlane_f(rkw, owner) : (id >= 0 ? 1.0f : 0.0f);
    }
    if (lane == k) {
      myid = id;
      myw = pw;
      mymask = msk;
    }
  }
  // weights: norm in k order (double, as ggml's sum_rows), scale, slot mask
  float w = myw;
  if (a.weights_norm) {
    // the lane values are read out first; only the additions are serial
    const double dw = (double)myw;
    double sum = 0.0;
    for (int k = 0; k < K; ++k) sum += __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(dw), k),
                                                         __builtin_amdgcn_readlane(__double2loint(dw), k));
    float fs = (float)sum;
    fs = fs < 6.103515625e-5f ? 6.103515625e-5f : fs;
    w = w / fs;
  }
  if (a.weights_scale != 0.0f && a.weights_scale != 1.0f) w = w * a.weights_scale;
  if (a.route_map) w = w * mymask;
  return WaveRoute{myid, w};
}

// E <= 64*P for the smallest P in {1, 2, 4, 8, 16}, P <= MAXP
template <int MAXP>
__device__ __forceinline__ WaveRoute route_token(const RouterArgs &a, int s, float *scr) {
  if (a.E <= 64) return router_wave<1>(a, s, scr);
  if (a.E <= 128) return router_wave<2>(a, s, scr);
  if (MAXP <= 2 || a.E <= 256) return router_wave<MAXP < 4 ? MAXP : 4>(a, s, scr);
  if (MAXP <= 4 || a.E <= 512) return router_wave<MAXP < 8 ? MAXP : 8>(a, s, scr);
  return router_wave<MAXP>(a, s, scr);
}

// one wave per token, 4 tokens per workgroup
static __global__ __launch_bounds__(256) void k_router(RouterArgs a, int S) {
  __shared__ float scr[4][ROUTER_MAX_E];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int s = blockIdx.x * 4 + wave;
  if (s >= S) return;
  const WaveRoute r = route_token<16>(a, s, scr[wave]);
  if (lane < a.K) {
    a.ids[(size_t)s * a.K + lane] = r.id;
    a.weights[(size_t)s * a.K + lane] = r.w;
  }
}

// ============================================================ bucketing
//
// Stable counting sort of the flat pair ids p = s*K + k by expert, the CSR of
// /root/reference/core/batched_dispatch_pipeline.cpp:1181-1202 (token-major
// inside each bucket).  One workgroup of 1024 threads; pairs are ranked in
// chunks of 1024 with a wave "match" loop (ballot per distinct expert) plus
// per-wave counts, so the order is exactly the sequential one.
constexpr int BUCKET_MAX_E = 512;

// Every thread reads its pairs' expert ids once (pair c * 1024 + tid for chunk
// c, up to BUCKET_CH chunks held in registers; larger inputs re-read ids per
// chunk), so the count, scan and ranking passes wait for memory only once.
constexpr int BUCKET_CH = 8;

static __global__ __launch_bounds__(1024) void k_bucket(const int32_t *__restrict__ ids, int n_pairs, int E,
                                                 int32_t *__restrict__ counts, int32_t *__restrict__ offs,
                                                 int32_t *__restrict__ pairs, int32_t *__restrict__ active,
                                                 int32_t *__restrict__ n_active) {
  __shared__ int cnt[BUCKET_MAX_E];
  __shared__ int base[BUCKET_MAX_E];
  __shared__ int wcnt[16][BUCKET_MAX_E];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nch = (n_pairs + 1023) / 1024;
  int eid[BUCKET_CH];
#pragma unroll
  for (int c = 0; c < BUCKET_CH; ++c) {
    const int i = c * 1024 + tid;
    const int e = i < n_pairs ? ids[i] : -1;
    eid[c] = e >= 0 && e < E ? e : -1;
  }
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int i = c * 1024 + tid;
    int e = -1;
    if (c < BUCKET_CH) {
#pragma unroll
      for (int q = 0; q < BUCKET_CH; ++q) e = q == c ? eid[q] : e;
    } else if (i < n_pairs) {
      e = ids[i];
      e = e >= 0 && e < E ? e : -1;
    }
    if (e >= 0) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (w == 0) {
    // exclusive scan over E (<= 512) by one wave: 8 per lane
    int local[8];
    int acc = 0, nz = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = lane * 8 + j;
      local[j] = e < E ? cnt[e] : 0;
      acc += local[j];
      nz += local[j] > 0;
    }
    int incl = acc, inz = nz;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const int o = __shfl_up(incl, m, 64);
      const int oz = __shfl_up(inz, m, 64);
      if (lane >= m) {
        incl += o;
        inz += oz;
      }
    }
    int run = incl - acc, runz = inz - nz;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = lane * 8 + j;
      if (e < E) {
        offs[e] = run;
        base[e] = run;
        counts[e] = local[j];
        if (local[j] > 0) active[runz++] = e;
        run += local[j];
      }
    }
    if (lane == 63) {
      offs[E] = incl;
      *n_active = inz;
    }
  }
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int nbits = E > 1 ? 32 - __builtin_clz((unsigned)(E - 1)) : 1;  // bits of an expert id
  for (int c = 0; c < nch; ++c) {
    for (int e = lane; e < E; e += 64) wcnt[w][e] = 0;
    const int i = c * 1024 + tid;
    int e = -1;
    if (c < BUCKET_CH) {
#pragma unroll
      for (int q = 0; q < BUCKET_CH; ++q) e = q == c ? eid[q] : e;
    } else if (i < n_pairs) {
      e = ids[i];
      e = e >= 0 && e < E ? e : -1;
    }
    const bool valid = e >= 0;
    __syncthreads();  // (first chunk: also the scan's base[] before it is read)
    // rank among the earlier lanes of this wave with the same expert: the
    // lanes holding the same id are the intersection, over the id's bits, of
    // one ballot per bit (or its complement), so no loop over distinct ids
    uint64_t m = __ballot(valid);
    for (int j = 0; j < nbits; ++j) {
      const uint64_t bj = __ballot(valid && ((e >> j) & 1));
      m &= ((e >> j) & 1) ? bj : ~bj;
    }
    const int rank = __builtin_popcountll(m & lt_mask);
    if (valid && rank == 0) wcnt[w][e] = __builtin_popcountll(m);
    __syncthreads();
    if (valid) {
      int r = base[e] + rank;
      for (int w2 = 0; w2 < w; ++w2) r += wcnt[w2][e];
      pairs[r] = i;
    }
    __syncthreads();
    for (int e2 = tid; e2 < E; e2 += 1024) {
      int add = 0;
      for (int w2 = 0; w2 < 16; ++w2) add += wcnt[w2][e2];
      base[e2] += add;
    }
    __syncthreads();  // wcnt is cleared, and base read, by the next chunk
  }
}

// ============================================================ bucketed GEMV
//
// dst rows of every (token, slot) pair routed to an expert; one workgroup per
// (row tile, active expert).  A wave covers 64/LPR rows per step with LPR
// lanes per row (one 64-weight quarter each, ITER quarters per lane when a
// row has more than 64 quarters).  Activation slices for NP pairs stay in
// registers for the whole tile, so each weight byte is read once per bucket
// chunk of NP pairs.
struct GemvArgs {
  const uint8_t *w0;  // expert 0 of the weight tensor (gate, or the only one)
  const uint8_t *w1;  // up (GATEUP only)
  size_t w_estride, w_rstride;
  int nrows, nb;
  const uint8_t *xq;  // planar Q8_K rows
  size_t xq_rstride;
  int ne11, K;
  const int32_t *n_active, *active, *offs, *pairs;
  int dense_S;  // > 0: expert 0, pairs 0..dense_S-1 (token = pair)
  float *out;
  size_t out_s, out_k;  // in floats
  int tile_rows;
  const uint64_t *grid;   // IQ2_XXS / IQ3_XXS grid or IQ4_XS value table (global), staged into LDS
  const uint64_t *signs;
  // int8-MFMA path: (expert, first pair) work items of up to 32 pairs each
  const int32_t *items, *n_items;
  uint32_t xq_bytes;  // extent of the xq buffer
};

template <int T, int LPR, int ITER, int NP, bool GATEUP>
static __global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  __shared__ uint64_t s_grid[T == T_IQ2_XXS ? 256 : (T == T_IQ3_XXS ? 128 : (T == T_IQ4_XS ? 2 : 1))];
  __shared__ uint64_t s_signs[T == T_IQ2_XXS || T == T_IQ3_XXS ? 128 : 1];
  if constexpr (T == T_IQ2_XXS || T == T_IQ3_XXS) {  // IQ3_XXS: 256 x u32 grid
    for (int i = threadIdx.x; i < (T == T_IQ2_XXS ? 256 : 128); i += 256) s_grid[i] = a.grid[i];
    if (threadIdx.x < 128) s_signs[threadIdx.x] = a.signs[threadIdx.x];
    __syncthreads();
  } else if constexpr (T == T_IQ4_XS) {  // a.grid: the 16-byte value table
    if (threadIdx.x < 2) s_grid[threadIdx.x] = a.grid[threadIdx.x];
    __syncthreads();
  }
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
  constexpr int RPI = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int u0 = lane % LPR, rsub = lane / LPR;
  const int U = a.nb * 4;
  const int row_begin = blockIdx.x * a.tile_rows;
  const int row_end = min(row_begin + a.tile_rows, a.nrows);
  const uint8_t *W0 = a.w0 + (size_t)e * a.w_estride;
  const uint8_t *W1 = GATEUP ? a.w1 + (size_t)e * a.w_estride : nullptr;
  constexpr int BB = block_bytes(T);

  for (int pc = p0; pc < p1; pc += NP) {
    Q8Slice xs[NP][ITER];
    int ptok[NP], pk[NP];
    bool pv[NP];
#pragma unroll
    for (int n = 0; n < NP; ++n) {
      const int p = pc + n;
      pv[n] = p < p1;
      const int pair = a.dense_S > 0 ? (pv[n] ? p : p0) : a.pairs[pv[n] ? p : p0];
      const int Kp = a.dense_S > 0 ? 1 : a.K;
      ptok[n] = pair / Kp;
      pk[n] = pair % Kp;
      const uint8_t *xrow = a.xq + (size_t)(ptok[n] * a.ne11 + pk[n] % a.ne11) * a.xq_rstride;
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int u = u0 + it * LPR;
        if (u < U) load_q8_slice<T>(xrow, a.nb, u >> 2, u & 3, xs[n][it]);
      }
    }
    for (int r0 = row_begin + wave * RPI; r0 < row_end; r0 += 4 * RPI) {
      const int r = r0 + rsub;
      const bool rv = r < row_end;
      float acc0[NP], acc1[NP];
#pragma unroll
      for (int n = 0; n < NP; ++n) acc0[n] = acc1[n] = 0.f;
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int u = u0 + it * LPR;
        if (rv && u < U) {
          const int b = u >> 2, q = u & 3;
          WSlice w0, w1;
          load_w_slice<T>(W0 + (size_t)r * a.w_rstride + (size_t)b * BB, q, w0);
          if constexpr (GATEUP) load_w_slice<T>(W1 + (size_t)r * a.w_rstride + (size_t)b * BB, q, w1);
#pragma unroll
          for (int n = 0; n < NP; ++n) {
            acc0[n] += quarter_dot<T>(w0, q, xs[n][it], s_grid, s_signs);
            if constexpr (GATEUP) acc1[n] += quarter_dot<T>(w1, q, xs[n][it], s_grid, s_signs);
          }
        }
      }
#pragma unroll
      for (int n = 0; n < NP; ++n) {
        acc0[n] = group_sum<LPR>(acc0[n]);
        if constexpr (GATEUP) acc1[n] = group_sum<LPR>(acc1[n]);
      }
      if (rv && u0 == 0) {
#pragma unroll
        for (int n = 0; n < NP; ++n) {
          if (!pv[n]) continue;
          const float v = GATEUP ? silu_f32(acc0[n]) * acc1[n] : acc0[n];
          a.out[(size_t)ptok[n] * a.out_s + (size_t)pk[n] * a.out_k + r] = v;
        }
      }
    }
  }
}

// ============================================================ combine
// ggml_mul(down, weights) then sum_topk (moe_routed_ggml.hpp:198-214):
// out = ((w0*y0 + w1*y1) + w2*y2) + ...   (+ shared, moe_block.hpp:201-202)
// one output per thread: for an output buffer that is not 16-byte aligned
static __global__ __launch_bounds__(256) void k_combine1(const float *__restrict__ y, const float *__restrict__ w,
                                                  const float *__restrict__ shared, int H, int K,
                                                  float *__restrict__ out) {
  const int s = blockIdx.y;
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  const float *ys = y + (size_t)s * K * H;
  float acc = w[(size_t)s * K] * ys[h];
  for (int k = 1; k < K; ++k) acc = acc + w[(size_t)s * K + k] * ys[(size_t)k * H + h];
  if (shared) acc = acc + shared[(size_t)s * H + h];
  out[(size_t)s * H + h] = acc;
}

static __global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y, const float *__restrict__ w,
                                                 const float *__restrict__ shared, int H, int K,
                                                 float *__restrict__ out) {
  // four consecutive outputs per thread (H is a multiple of 256): float4 loads
  // of every route's row, the same k-ascending sum per element
  const int s = blockIdx.y;
  const int h = 4 * (blockIdx.x * 256 + threadIdx.x);
  if (h >= H) return;
  const float *ys = y + (size_t)s * K * H;
  const float *ws = w + (size_t)s * K;
  float4 yk[8];
  const int K0 = K < 8 ? K : 8;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < K0) yk[k] = *reinterpret_cast<const float4 *>(ys + (size_t)k * H + h);
  float4 acc;
  acc.x = ws[0] * yk[0].x;
  acc.y = ws[0] * yk[0].y;
  acc.z = ws[0] * yk[0].z;
  acc.w = ws[0] * yk[0].w;
#pragma unroll
  for (int k = 1; k < 8; ++k)
    if (k < K0) {
      const float wk = ws[k];
      acc.x = acc.x + wk * yk[k].x;
      acc.y = acc.y + wk * yk[k].y;
      acc.z = acc.z + wk * yk[k].z;
      acc.w = acc.w + wk * yk[k].w;
    }
  for (int k = 8; k < K; ++k) {
    const float wk = ws[k];
    const float4 v = *reinterpret_cast<const float4 *>(ys + (size_t)k * H + h);
    acc.x = acc.x + wk * v.x;
    acc.y = acc.y + wk * v.y;
    acc.z = acc.z + wk * v.z;
    acc.w = acc.w + wk * v.w;
  }
  if (shared) {
    const float4 v = *reinterpret_cast<const float4 *>(shared + (size_t)s * H + h);
    acc.x = acc.x + v.x;
    acc.y = acc.y + v.y;
    acc.z = acc.z + v.z;
    acc.w = acc.w + v.w;
  }
  *reinterpret_cast<float4 *>(out + (size_t)s * H + h) = acc;
}

// zero (negative id) or NaN (id >= n_experts) rows of routes the GEMV skips
// (patches/ggml/0002...:50-54; kernels/quant/kquant_matmul.cu:660-663)
static __global__ void k_fill_skipped(const int32_t *__restrict__ ids, size_t id_s, size_t id_k, int n_ids, int S,
                               int n_experts, int O, float *out, size_t out_s, size_t out_k) {
  // pairs are strided over grid y (at most 65535 rows of workgroups)
  for (int pair = blockIdx.y; pair < n_ids * S; pair += gridDim.y) {
    const int s = pair / n_ids, k = pair % n_ids;
    const int e = ids[s * id_s + k * id_k];
    if (e >= 0 && e < n_experts) continue;
    const float v = e < 0 ? 0.0f : __int_as_float(0x7fc00000);
    for (int r = blockIdx.x * 256 + threadIdx.x; r < O; r += gridDim.x * 256) out[s * out_s + k * out_k + r] = v;
  }
}

// ============================================================ fp32 router GEMV
// logits[s][e] = sum_i W[e][i] * x[s][i] (ggml_mul_mat(router, cur), moe_routed_ggml.hpp:55)
static __global__ __launch_bounds__(256) void k_router_gemv(const float *__restrict__ W, const float *__restrict__ x,
                                                     int H, int E, int S, float *__restrict__ logits) {
  __shared__ float part[4][64];
  const int e = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float *wr = W + (size_t)e * H;
  for (int s0 = 0; s0 < S; s0 += 64) {
    // each wave covers a quarter of H for up to 64 tokens... tokens looped
    const int ns = min(64, S - s0);
    for (int si = 0; si < ns; ++si) {
      const float *xr = x + (size_t)(s0 + si) * H;
      float acc = 0.f;
      // the first RG_IT chunks are all requested before the first fma (one
      // memory round trip instead of one per chunk); same summation order
      constexpr int RG_IT = 8;
      const int i0 = (wave * 64 + lane) * 4;
      float4 wv[RG_IT], xv[RG_IT];
#pragma unroll
      for (int k = 0; k < RG_IT; ++k) {
        const int i = i0 + 1024 * k;
        wv[k] = i < H ? *reinterpret_cast<const float4 *>(wr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        xv[k] = i < H ? *reinterpret_cast<const float4 *>(xr + i) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int k = 0; k < RG_IT; ++k) {
        if (i0 + 1024 * k >= H) break;
        acc = __builtin_fmaf(wv[k].x, xv[k].x, acc);
        acc = __builtin_fmaf(wv[k].y, xv[k].y, acc);
        acc = __builtin_fmaf(wv[k].z, xv[k].z, acc);
        acc = __builtin_fmaf(wv[k].w, xv[k].w, acc);
      }
      for (int i = i0 + 1024 * RG_IT; i < H; i += 1024) {
        const float4 w4 = *reinterpret_cast<const float4 *>(wr + i);
        const float4 x4 = *reinterpret_cast<const float4 *>(xr + i);
        acc = __builtin_fmaf(w4.x, x4.x, acc);
        acc = __builtin_fmaf(w4.y, x4.y, acc);
        acc = __builtin_fmaf(w4.z, x4.z, acc);
        acc = __builtin_fmaf(w4.w, x4.w, acc);
      }
      acc = group_sum<64>(acc);
      if (lane == 0) part[wave][si] = acc;
    }
    __syncthreads();
    if (wave == 0 && lane < ns) {
      logits[(size_t)(s0 + lane) * E + e] = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
    }
    __syncthreads();
  }
}

// Batched form (S >= 8): 16 tokens x 16 experts per workgroup on
// v_mfma_f32_16x16x4f32.  The K range is cut into KS = gridDim.z slices (one
// per workgroup, so that enough workgroups stream the router weights) and each
// slice over the 4 waves, summed in LDS in wave order into part[z][s][e];
// k_router_sum adds the slices in order.  Lane (n = lane % 16, g = lane / 16)
// feeds token / expert n with the 4 consecutive values k0 + 4g .. 4g+3 of each
// 16-wide K chunk, one per MFMA.  H % (64 * KS) == 0.
typedef float v4f_rt __attribute__((ext_vector_type(4)));
static __global__ __launch_bounds__(256) void k_router_gemm(const float *__restrict__ W, const float *__restrict__ x, int H,
                                                     int E, int S, float *__restrict__ part) {
  __shared__ float red[4][64][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int e0 = blockIdx.x * 16, s0 = blockIdx.y * 16, z = blockIdx.z, KS = gridDim.z;
  const int e = min(e0 + n, E - 1), s = min(s0 + n, S - 1);
  const float4 *wr = reinterpret_cast<const float4 *>(W + (size_t)e * H) + g;
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)s * H) + g;
  const int kq = H / (64 * KS);  // 16-wide chunks per wave
  const int c0 = (z * 4 + wave) * kq;
  // 8 chunks of loads in flight, two accumulator chains
  v4f_rt acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
  constexpr int U = 8;
  for (int cb = c0; cb < c0 + kq; cb += U) {
    float4 a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(cb + u, c0 + kq - 1);
      a[u] = xr[4 * c];
      b[u] = wr[4 * c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (cb + u >= c0 + kq) break;
      v4f_rt &t = (u & 1) ? acc2 : acc;
      t = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].x, b[u].x, t, 0, 0, 0);
      t = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].y, b[u].y, t, 0, 0, 0);
      t = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].z, b[u].z, t, 0, 0, 0);
      t = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u].w, b[u].w, t, 0, 0, 0);
    }
  }
  acc += acc2;
#pragma unroll
  for (int j = 0; j < 4; ++j) red[wave][lane][j] = acc[j];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ss = s0 + 4 * g + j, ee = e0 + n;  // D lane l, reg j: token 4g + j, expert n
      const float v = (red[0][lane][j] + red[1][lane][j]) + (red[2][lane][j] + red[3][lane][j]);
      if (ss < S && ee < E) part[((size_t)z * S + ss) * E + ee] = v;
    }
  }
}
static __global__ __launch_bounds__(256) void k_router_sum(const float *__restrict__ part, int n, int KS,
                                                    float *__restrict__ logits) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float v = part[i];
  for (int z = 1; z < KS; ++z) v += part[(size_t)z * n + i];
  logits[i] = v;
}

}  // namespace zm
