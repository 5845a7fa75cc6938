// zm_decode.hpp -- one persistent kernel for a whole routed MoE layer at
// decode sizes (S <= 8 tokens): router -> Q8_K(x) -> gate/up + SwiGLU ->
// Q8_K(act) -> down -> weighted top-k sum (+ shared expert), with no kernel
// boundary in between.
//
// Grid: as many 512-thread workgroups as the device holds at once.
//   P0  every workgroup routes all tokens and quantizes x into LDS --
//       redundant, but no grid-wide barrier precedes the first weight request.
//       With a shared expert each wave then requests the weights of its first
//       down rows (P2); without one it requests them when its workgroup's
//       gate/up rows are done, so they stream while the workgroups wait for
//       the act rows and take no bandwidth from the gate/up rows.
//   P1  the shared expert's gate/up rows (which need no routing) and then the
//       routed (pair, row) rows are each cut into one contiguous range per
//       workgroup; the shared range starts as soon as x is quantized, while
//       the routing waves finish.  Waves stream batches of rows
//       (double-buffered) and store the SwiGLU output; the workgroup then
//       counts itself in one of 16 arrival counters and adds its row counts to
//       the counter of every 256-row act block its ranges touch.
//   P2  down rows (token s, row h): each wave takes act blocks of the
//       workgroup's tokens as soon as their counters reach 256 rows,
//       quantizes them into LDS (Q8_K), and after the last one the workgroup
//       computes out[s][h] = sum_k w_k * (W_down[e_k][h] . q8(act_k)) (+ shared).
//       No grid-wide barrier: blocks finished early are quantized while the
//       last gate/up rows are still being computed elsewhere.
// Counters come in two sets used by alternate calls: an epoch word selects the
// set; the other set is zeroed at the end of the call (by the first and last
// workgroups, off the critical path), and workgroup 0 bumps the epoch once
// every workgroup has arrived (all of them have read it by then), so no
// workgroup waits on an atomic's return value.
// The hot loops are straight-line code: a lane or row without work loads and
// stores through an out-of-range buffer offset (loads return zeros, stores are
// dropped), so every load of a batch is issued unconditionally and the
// compiler's wait counts stay exact (a conditionally issued load or store
// forces waits for everything issued after it).
// Cross-workgroup data moves through agent-scope relaxed atomics and sc1
// loads/stores (coherent past the per-XCD L2s); no agent-scope fence (an L2
// write-back + invalidate on gfx950) is issued.  The wait is bounded: on
// expiry the error word is set and the kernel still drains.
#pragma once

#include "zm_blockdot.hpp"
#include "zm_kernels.hpp"

namespace zm {

constexpr int DEC_THREADS = 512;
constexpr int DEC_WAVES = DEC_THREADS / 64;
constexpr int DEC_MAX_S = 8;
constexpr int DEC_MAX_PAIRS = 128;  // S * K
constexpr int DEC_LDS_Q8 = 65536;   // Q8_K staging: x rows in P0/P1, act rows in P2
constexpr int DEC_NCNT = 16;        // arrival counters per set (one 64-byte line each) to spread the atomics
constexpr int DEC_CNT_STRIDE = 16;  // words between counters
constexpr int DEC_MAX_ABLK = 1024;  // act blocks (256 gate/up rows each) tracked per call
constexpr int DEC_BCNT_STRIDE = 32; // words between block counters (one 128-byte line each)
constexpr int DEC_BLK_BASE = DEC_CNT_STRIDE * (1 + 2 * DEC_NCNT);
constexpr int DEC_SYNC_WORDS = DEC_BLK_BASE + 2 * DEC_MAX_ABLK * DEC_BCNT_STRIDE;
constexpr int DEC_MAX_E = 512;      // router experts handled in the fused kernel

struct DecodeArgs {
  RouterArgs r;  // logits, biases, slot table; r.ids / r.weights: optional global outputs
  const float *x;
  float *out;
  int H, F, K, S, nbH, nbF;
  const uint8_t *wg, *wu, *wd;
  size_t g_rstride, g_estride, d_rstride, d_estride;
  int Fs, nbFs;
  const uint8_t *sg, *su, *sd;
  size_t sg_rstride, sd_rstride;
  uint32_t wg_bytes, wd_bytes, sg_bytes, sd_bytes;  // buffer-resource extents (< 2 GiB)
  float *act;
  // [0] epoch, [1] error, [DEC_CNT_STRIDE*(1+NCNT*set+i)] arrival counter i of
  // set 0/1, [DEC_BLK_BASE + DEC_BCNT_STRIDE*(DEC_MAX_ABLK*set + b)] rows of act
  // block b stored
  uint32_t *sync;
  const uint64_t *grid, *signs;
  int spin_limit;
  uint64_t *trace;  // optional: 8 timestamps per workgroup
};

// q = j / d, r = j % d for 0 <= j < 2^24 via a float reciprocal and one
// select-based correction (exact in that range); no division sequence, no branch.
__device__ __forceinline__ void divmod24(int j, int d, float inv, int &q, int &r) {
  q = (int)((float)j * inv);
  r = j - q * d;
  q += (int)(r >= d) - (int)(r < 0);
  r = j - q * d;
}

template <class V>
__device__ __forceinline__ V ld_co(const V *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class V>
__device__ __forceinline__ void st_co(V *p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// this wave's coherent stores have completed (vmcnt(0)) before what follows
__device__ __forceinline__ void stores_done() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt left at their maxima
}
__device__ __forceinline__ void after_wait() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup"); }
// LDS hand-over between the waves of a workgroup: this wave's LDS accesses
// complete (release, LDS only: no wait for its global loads), then lane 0 adds
// v to the counter; the waiter spins on the counter and acquires
__device__ __forceinline__ void lds_signal(int *c, int v) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if (__lane_id() == 0) __hip_atomic_fetch_add(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_wait(int *c, int v) {
  while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < v) __builtin_amdgcn_s_sleep(1);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// one f32 through a buffer resource with sc1 (coherent past the L2); an
// out-of-range offset drops the store
__device__ __forceinline__ void bst_co(rsrc_t r, int vo, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, vo, 0, 16);
}
__device__ __forceinline__ void bst(rsrc_t r, int vo, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, vo, 0, 0);
}
// phase timestamps are kept in registers and written at the end of the kernel,
// so that no trace store sits in the in-order memory counter of a later wait
#define ZM_TRACE(slot)                           \
  do {                                           \
    if (a.trace) trace_t[(slot)] = wall_clock64(); \
  } while (0)

// Q8_K block (16 lanes) into an LDS activation row (q8l layout)
__device__ __forceinline__ void store_q8_16l(uint8_t *row, int nb, int blk, const Q8Out16 &o, int l16) {
  *reinterpret_cast<uint4 *>(row + (size_t)blk * Q8L_BLK + 16 * l16) = o.q;
  if (l16 == 0) reinterpret_cast<float *>(row + q8l_d_off(nb))[blk] = o.d;
  reinterpret_cast<int16_t *>(row + q8l_bs_off(nb))[blk * 16 + l16] = (int16_t)o.bsum;
}

// gate/up row kind for the P1 streaming loop: weight type and routed/shared
template <int T, bool SHARED, int L>
struct RowsTag {
  static constexpr int value = T;
  static constexpr bool shared = SHARED;
  static constexpr int lanes = L;  // lanes per row (one unit each)
};

template <int TG, int TD, int TS, int L1, int IR, int IS>
__global__ __launch_bounds__(DEC_THREADS) void k_moe_decode(DecodeArgs a) {
  __shared__ int s_ids[DEC_MAX_PAIRS];
  __shared__ float s_w[DEC_MAX_PAIRS];
  __shared__ int s_cidx[DEC_MAX_PAIRS];  // pair -> compact routed index (or -1)
  __shared__ int s_vp[DEC_MAX_PAIRS];    // compact index -> pair
  __shared__ int s_goff[DEC_MAX_PAIRS];  // compact index -> gate/up expert byte offset
  __shared__ int s_gtok[DEC_MAX_PAIRS];  // compact index -> token
  __shared__ int s_doff[DEC_MAX_PAIRS];  // pair -> down expert byte offset (or -1)
  __shared__ int s_nvp;
  __shared__ int s_xq_done;  // waves done quantizing x (shared-expert rows start on it)
  __shared__ int s_err;
  __shared__ uint32_t s_stale;
  __shared__ __attribute__((aligned(16))) uint8_t s_q8[DEC_LDS_Q8];
  __shared__ float4 s_stage[DEC_WAVES][256];  // per wave: router scratch, then the act transpose
  constexpr bool kIQ2 = TG == T_IQ2_XXS || TD == T_IQ2_XXS || TS == T_IQ2_XXS;
  constexpr bool kIQ4 = TG == T_IQ4_XS || TD == T_IQ4_XS || TS == T_IQ4_XS;
  constexpr bool kIQ3 = TG == T_IQ3_XXS || TD == T_IQ3_XXS || TS == T_IQ3_XXS;
  static_assert((int)kIQ2 + (int)kIQ3 + (int)kIQ4 <= 1, "one lookup table per layer");
  // the shared rows start before the table-filling waves (the routing waves
  // among them) are counted, so a shared expert never reads a lookup table
  static_assert(TS != T_IQ2_XXS && TS != T_IQ3_XXS && TS != T_IQ4_XS, "shared expert type without a lookup table");
  // the lookup tables first in LDS (largest alignment first): their addresses
  // fit the 16-bit offset field of the LDS reads, so an index becomes an
  // address in one or two instructions
  __shared__ __attribute__((aligned(kIQ2 || kIQ3 ? 4096 : 8))) uint64_t s_grid[kIQ2 ? 256 : (kIQ3 ? 128 : (kIQ4 ? 2 : 1))];
  __shared__ __attribute__((aligned(kIQ2 || kIQ3 ? 2048 : 8))) uint64_t s_signs[kIQ2 || kIQ3 ? 128 : 1];
  __shared__ int s_step;  // next dynamically assigned routed gate/up step
  static_assert(IS == 0 || TS != 0, "shared iterations need a shared type");
  static_assert(L1 == 16 || L1 == 32 || L1 == 20, "lanes per routed gate/up row");
  constexpr int L2 = 32;  // lanes per down row (2 rows per wave step)
  constexpr int NS = IS > 0 ? IS : 1;

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int G = gridDim.x, g = blockIdx.x;
  const int S = a.S, K = a.K, H = a.H, F = a.F;
  const size_t q8x = q8l_row_bytes(a.nbH);
  const size_t q8F = q8l_row_bytes(a.nbF);
  const size_t q8Fs = a.Fs > 0 ? q8l_row_bytes(a.nbFs) : 0;
  uint64_t trace_t[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  ZM_TRACE(0);
  if (tid == 0) s_step = 0;  // published by the first workgroup barrier
  if constexpr (TS != 0) {
    // the x-quantization counter starts at zero before any wave counts itself:
    // an LDS store and a plain barrier (no memory fence, so no wave waits for
    // its global loads here)
    if (tid == 0) s_xq_done = 0;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
  }
  // The epoch word selects this call's counter set (the other set is cleared
  // at the end, for the next call).  An earlier call's wait expired (error
  // word set): its counters are in an unknown state, so none of them is
  // trusted.  The error word is read by one thread and acted on after the
  // first workgroup barrier (a uniform decision): every workgroup writes NaN
  // to its output rows and leaves.  zm_moe_status reports the error and resets
  // the sync words; calls then run normally.  Both words are requested here
  // and consumed later, so no wave waits for them before its first loads.
  const uint32_t epoch_v = ld_co(&a.sync[0]);
  uint32_t stale_v = 0;
  if (tid == 0) stale_v = ld_co(&a.sync[1]);

  // ---------------------------------------------------------------- P0: route, quantize x
  // Wave w < S routes token w; the other waves quantize x (16 lanes per
  // block, 4 blocks per wave and round), each loading its next group of blocks
  // while it quantizes one.  With S = DEC_WAVES every wave routes, then
  // quantizes.  The lookup tables are loaded up front by the non-routing
  // threads (thread index rotated past the routing waves) and stored to LDS
  // after routing, so their latency overlaps the router's.
  if (tid == 0) s_err = 0;
  const int nxb = S * a.nbH;
  const int l16 = lane & 15;
  const int nwk = S < DEC_WAVES ? DEC_WAVES - S : DEC_WAVES;  // x-quant workers
  const int wi = wave >= S ? wave - S : (S < DEC_WAVES ? nwk + wave : wave);  // worker index (>= nwk: none)
  const int jt = (tid - 64 * S) & (DEC_THREADS - 1);
  uint64_t tab_g = 0, tab_s = 0;
  if constexpr (kIQ2) {
    if (jt < 256) tab_g = a.grid[jt];
    if (jt < 128) tab_s = a.signs[jt];
  } else if constexpr (kIQ3) {  // a.grid: the IQ3_XXS grid (256 x u32)
    if (jt < 128) tab_g = a.grid[jt];
    if (jt < 128) tab_s = a.signs[jt];
  } else if constexpr (kIQ4) {  // a.grid: the IQ4_XS value table
    if (jt < 2) tab_g = a.grid[jt];
  }
  auto xload = [&](int grp, float4 (&v)[4]) {
    const int bb = grp * 4 + (lane >> 4);
    if (grp * 4 < nxb && bb < nxb) {  // x rows are contiguous (H = nbH * QK): block bb at bb * QK
      const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)bb * QK + 16 * l16);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = src[i];
    }
  };
  float4 xcur[4] = {};
  // with more groups than workers the first group is requested at the top of
  // the kernel (c4: 81 -> 80 us); with one group or less per worker it is
  // requested in the quantization loop (measured: the early request made c2
  // 0.3 us slower)
  const bool xearly = (nxb + 3) / 4 > nwk;
  if (xearly && wave >= S) xload(wi, xcur);
  if (wave < S) {
    const WaveRoute r = route_token<8>(a.r, wave, reinterpret_cast<float *>(s_stage[wave]));
    if (lane < K) {
      s_ids[wave * K + lane] = r.id;
      s_w[wave * K + lane] = r.w;
      if (g == 0 && a.r.ids) {
        a.r.ids[wave * K + lane] = r.id;
        a.r.weights[wave * K + lane] = r.w;
      }
    }
    if (S == 1 || !a.r.route_map) {
      // one token, or no slot table (every route valid, so token w's pairs
      // are compact indices wK .. wK + K - 1): each routing wave compacts its
      // own pairs (see below), which saves a workgroup barrier
      const bool ok = lane < K && r.id >= 0;
      const unsigned long long m = __ballot(ok);
      const int c = wave * K + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
      const int p = wave * K + lane;
      if (lane < K) {
        s_cidx[p] = ok ? c : -1;
        s_doff[p] = ok ? r.id * (int)a.d_estride : -1;
      }
      if (ok) {
        s_vp[c] = p;
        s_goff[c] = r.id * (int)a.g_estride;
        s_gtok[c] = wave;
      }
      if (tid == 0) s_nvp = S == 1 ? __popcll(m) : S * K;
    }
  }
  if constexpr (kIQ2) {
    if (jt < 256) s_grid[jt] = tab_g;
    if (jt < 128) s_signs[jt] = tab_s;
  } else if constexpr (kIQ3) {
    if (jt < 128) s_grid[jt] = tab_g;
    if (jt < 128) s_signs[jt] = tab_s;
  } else if constexpr (kIQ4) {
    if (jt < 2) s_grid[jt] = tab_g;
  }
  ZM_TRACE(6);
  if (wi < nwk) {
    if (!xearly || wave < S) xload(wi, xcur);
    // this lane's block (token s, block b) of each group, stepped by the
    // 4 * nwk blocks between a worker's groups (one division, up front)
    const int bb0 = wi * 4 + (lane >> 4), ds = 4 * nwk / a.nbH, db = 4 * nwk % a.nbH;
    int s = bb0 / a.nbH, b = bb0 % a.nbH;
    for (int grp = wi; grp * 4 < nxb; grp += nwk) {
      float4 xnext[4] = {};
      xload(grp + nwk, xnext);
      if (s < S) {
        float xv[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xv[4 * i] = xcur[i].x;
          xv[4 * i + 1] = xcur[i].y;
          xv[4 * i + 2] = xcur[i].z;
          xv[4 * i + 3] = xcur[i].w;
        }
        store_q8_16l(s_q8 + (size_t)s * q8x, a.nbH, b, quant_block16(xv, l16), l16);
      }
      s += ds;
      b += db;
      if (b >= a.nbH) {
        b -= a.nbH;
        ++s;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) xcur[i] = xnext[i];
    }
  }
  ZM_TRACE(7);
  // P1 rows: L lanes per row (L1 for routed rows, 64 for shared rows), 64/L
  // rows per wave step; lane li = lane % L takes unit li of the row (one
  // super-block, or half of one for Q4_K).  Steps go through two register
  // buffers: step st+1 is in flight while step st computes.  act holds the S *
  // Fs shared rows (token, row n) first, then the routed rows (route c, row n).
  const int Tsh = TS != 0 ? S * a.Fs : 0;  // Fs = 0 exactly when there is no shared expert
  const rsrc_t ract = make_rsrc(a.act, (uint32_t)(S * K * F + Tsh) * 4u);
  const float invF = 1.0f / (float)F, invFs = a.Fs > 0 ? 1.0f / (float)a.Fs : 0.f;
  auto stream_rows = [&](auto ttag, int r0, int r1) {
    // rows [r0, r1) of the kind's own row space; routed rows sit after the
    // S * Fs shared rows in act
    constexpr int TT = decltype(ttag)::value;
    constexpr bool SH = decltype(ttag)::shared;
    constexpr int LL = decltype(ttag)::lanes;
    // LL = 20: rows of 20 units (IQ2_XXS at H = 5120) as 16 + 4 lanes, three
    // rows per step: main lanes 16r .. 16r + 15 take units 0..15 of row r,
    // tail lanes 48 + 4r .. +3 units 16..19 (lanes 60..63 idle), so 60 of
    // 64 lanes work where 32-lane rows would leave 12 of every 32 idle
    constexpr bool TAIL = LL == 20;
    constexpr int R1 = TAIL ? 3 : 64 / LL;
    const int li1 = TAIL ? (lane < 48 ? (lane & 15) : 16 + (lane & 3)) : lane % LL;
    const int rg1 = TAIL ? (lane < 48 ? (lane >> 4) : ((lane - 48) >> 2)) : lane / LL;
    constexpr int UP = unit_per_block<TT>();
    constexpr int BT = block_bytes(TT);
    const int U1 = a.nbH * UP;
    const rsrc_t rgt = SH ? make_rsrc(a.sg, a.sg_bytes) : make_rsrc(a.wg, a.wg_bytes);
    const rsrc_t rut = SH ? make_rsrc(a.su, a.sg_bytes) : make_rsrc(a.wu, a.wg_bytes);
    const bool uok = li1 < U1;
    const int blk = min(li1 / UP, a.nbH - 1), part = li1 % UP;
    const int nst_all = (r1 - r0 + R1 - 1) / R1;
    // Wave w starts with step w.  With many steps per wave (routed rows only)
    // the further steps come from an LDS counter when the wave issues its
    // loads: with a fixed stride the two waves of a SIMD drift apart (the
    // older one is issued first) and the late one finishes alone, without a
    // second wave to hide its latency (c4: first and last wave of a workgroup
    // 11 us apart, 3 us with the counter).  With few steps per wave the fixed
    // stride is kept (c5 was 0.9 us slower with the counter).
    const bool dyn = !SH && nst_all >= 6 * DEC_WAVES;
    // The shared rows (streamed before the routing barrier) go to the
    // x-quantization workers only: a routing wave that took one would request
    // it after routing and hold up the barrier by a full load round trip (c5:
    // routing done 5.2 us, barrier 7.4 us).
    const int kw = SH ? (wi < nwk ? wi : nst_all) : wave;
    const int kstride = SH ? nwk : DEC_WAVES;
    auto grab = [&](int kprev) {
      if (!dyn) return kprev + kstride;
      int v = 0;
      if (lane == 0) v = __hip_atomic_fetch_add(&s_step, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      return DEC_WAVES + __builtin_amdgcn_readfirstlane(v);
    };
    // step k -> this lane's (valid, row j, token, weight-row byte offset)
    auto row1 = [&](int k, bool &valid, int &j, int &tok, int &roff) {
      j = r0 + R1 * k + rg1;
      valid = k < nst_all && j < r1 && rg1 < R1;
      j = valid ? j : r0;
      int q, n;
      if constexpr (SH) {
        divmod24(j, a.Fs, invFs, q, n);
        tok = q;
        roff = (int)__umul24((uint32_t)n, (uint32_t)a.sg_rstride);
      } else {
        divmod24(j, F, invF, q, n);
        tok = s_gtok[q];
        roff = s_goff[q] + (int)__umul24((uint32_t)n, (uint32_t)a.g_rstride);
      }
    };
    // a step's row (valid, j, token) is worked out once, when its loads are issued
    struct RowInfo {
      bool valid;
      int j, tok;
    };
    auto issue = [&](int st, Unit<TT> (&bw)[2], RowInfo &ri) {
      int roff;
      row1(st, ri.valid, ri.j, ri.tok, roff);
      const int vo = (ri.valid && uok) ? roff + blk * BT : OOR;
      load_unit<TT>(rgt, vo, part, bw[0]);
      load_unit<TT>(rut, vo, part, bw[1]);
    };
    auto compute = [&](const Unit<TT> (&bw)[2], const RowInfo &ri) {
      const bool valid = ri.valid;
      const int j = ri.j, tok = ri.tok;
      float o[2];
      unit_dots<TT, 2>(bw, part, xblk(s_q8 + (size_t)tok * q8x, a.nbH, blk), s_grid, s_signs, o);
      float ag, au;
      if constexpr (TAIL) {
        // row r = main 16-sum (lanes 16r..) + tail 4-sum (lanes 48 + 4r..),
        // read out by the row's writer lane
        const float g16 = group_sum<16>(o[0]), u16 = group_sum<16>(o[1]);
        const float g4 = group_sum<4>(o[0]), u4 = group_sum<4>(o[1]);
        float tg[3], tu[3];
#pragma unroll
        for (int rr = 0; rr < 3; ++rr) {
          tg[rr] = readlane_f(g16, 16 * rr) + readlane_f(g4, 48 + 4 * rr);
          tu[rr] = readlane_f(u16, 16 * rr) + readlane_f(u4, 48 + 4 * rr);
        }
        ag = rg1 == 0 ? tg[0] : (rg1 == 1 ? tg[1] : tg[2]);
        au = rg1 == 0 ? tu[0] : (rg1 == 1 ? tu[1] : tu[2]);
      } else {
        ag = group_sum<LL>(o[0]);
        au = group_sum<LL>(o[1]);
      }
      bst_co(ract, (li1 == 0 && valid) ? 4 * (SH ? j : Tsh + j) : OOR, silu_f32(ag) * au);
    };
    // sched_barrier keeps every load of a step ahead of the math that waits
    // on the previous one (vmcnt is in order: an interleaved wait drains the
    // queue); steps past the end load and store nothing
    Unit<TT> A[2], B[2];
    RowInfo ra, rb;
    int ka = kw;
    if (ka < nst_all) issue(ka, A, ra);
    while (ka < nst_all) {
      const int kb = grab(ka);
      issue(kb, B, rb);
      __builtin_amdgcn_sched_barrier(0);
      compute(A, ra);
      __builtin_amdgcn_sched_barrier(0);
      if (kb >= nst_all) break;  // B empty: no dots on zeros
      ka = grab(kb);
      issue(ka, A, ra);
      __builtin_amdgcn_sched_barrier(0);
      compute(B, rb);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // shared-expert rows need no routing: every wave starts its share of this
  // workgroup's shared rows once all of x is quantized (the waves that had
  // quantization work count themselves in LDS), so they stream while the
  // routing waves finish
  const int sh0 = (int)((long)Tsh * g / G), sh1 = (int)((long)Tsh * (g + 1) / G);
  if constexpr (TS != 0) {
    const int nqw = min(nwk, (nxb + 3) / 4);  // waves with x-quantization work
    if (wi < nqw) lds_signal(&s_xq_done, 1);  // this wave's x blocks are in LDS
    lds_wait(&s_xq_done, nqw);
    stream_rows(RowsTag<TS, true, 64>{}, sh0, sh1);
  }
  if (tid == 0) s_stale = stale_v;
  __syncthreads();
  if (s_stale != 0u) {
    const int T2e = S * H;
    const int v0 = (int)((long)T2e * g / G), v1 = (int)((long)T2e * (g + 1) / G);
    for (int j = v0 + tid; j < v1; j += DEC_THREADS) a.out[j] = __builtin_nanf("");
    return;
  }
  const bool compact = S > 1 && a.r.route_map;
  if (compact && wave == 0) {
    // compact the routed pairs (id >= 0) in pair order: ballot + prefix count
    int n = 0;
    for (int p0 = 0; p0 < S * K; p0 += 64) {
      const int p = p0 + lane;
      const bool ok = p < S * K && s_ids[p] >= 0;
      const unsigned long long m = __ballot(ok);
      const int c = n + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
      if (p < S * K) {
        s_cidx[p] = ok ? c : -1;
        s_vp[p] = 0;
      }
      n += __popcll(m);
    }
    stage_sync();
    for (int p0 = 0; p0 < S * K; p0 += 64) {
      const int p = p0 + lane;
      if (p < S * K) {
        // per-pair offsets worked out once: the per-row address math then
        // needs only 24-bit multiplies (row < 2^14, row stride < 2^24)
        const int id = s_ids[p];
        s_doff[p] = id >= 0 ? id * (int)a.d_estride : -1;
        if (s_cidx[p] >= 0) {
          s_vp[s_cidx[p]] = p;
          s_goff[s_cidx[p]] = id * (int)a.g_estride;
          s_gtok[s_cidx[p]] = p / K;
        }
      }
    }
    if (lane == 0) s_nvp = n;
  }
  if (compact) __syncthreads();
  ZM_TRACE(1);
  const int nvp = s_nvp;
  const int T1r = nvp * F;

  // ---------------------------------------------------------------- P2 set-up: down rows
  // L2 = 32 lanes per down row, 2 rows per wave step; step st of this wave
  // covers rows u0 + 2*(wave + DEC_WAVES*st) + lane / 32.  Lane li = lane % 32
  // takes units li + 32*it of the row: IR routed iterations over K*nbF*UPD
  // units (route, block, part), IS shared iterations over nbFs*UPS units.  The
  // first step of every wave is requested after the gate/up rows (below).
  const int li2 = lane % L2, rg2 = lane / L2;
  const int T2 = S * H;
  const int u0 = (int)((long)T2 * g / G), u1 = (int)((long)T2 * (g + 1) / G);
  const int nst2_all = (u1 - u0 + (64 / L2) - 1) / (64 / L2);
  const int nst2 = nst2_all > wave ? (nst2_all - wave + DEC_WAVES - 1) / DEC_WAVES : 0;
  const float invH = 1.0f / (float)H;
  // IQ2_XXS down rows in half blocks: c4's 8 x 6 blocks per row split into 96
  // units over 32 lanes (three full iterations instead of two with half the
  // lanes idle in the second)
  constexpr bool H2 = TD == T_IQ2_XXS;
  constexpr int UPD = H2 ? 2 : unit_per_block<TD>();
  constexpr int UPS = TS ? unit_per_block<TS>() : 1;
  constexpr int BD = block_bytes(TD);
  constexpr int BSD = TS ? block_bytes(TS) : 1;
  const int URd = K * a.nbF * UPD, URb = a.nbF * UPD, USd = a.nbFs * UPS;
  const rsrc_t rd = make_rsrc(a.wd, a.wd_bytes), rsd = make_rsrc(a.sd, a.sd_bytes);
  const rsrc_t rout = make_rsrc(a.out, (uint32_t)T2 * 4u);
  // row of step st for this lane -> (valid, token, row h); invalid rows map to a valid one
  auto row2 = [&](int st, bool &valid, int &s, int &h) {
    const int j = u0 + (64 / L2) * (wave + DEC_WAVES * st) + rg2;
    valid = st < nst2 && j < u1;
    divmod24(valid ? j : min(u0, T2 - 1), H, invH, s, h);
  };
  auto load_step2 = [&](int st, Unit<TD> (&wr)[IR], Unit<TS ? TS : TD> (&ws)[NS]) {
    bool valid;
    int s, h;
    row2(st, valid, s, h);
#pragma unroll
    for (int it = 0; it < IR; ++it) {
      const int u = li2 + L2 * it;
      const int k = u / URb, rem = u - k * URb;
      const int eoff = s_doff[s * K + min(k, K - 1)];
      const bool ok = valid && u < URd && eoff >= 0;
      if constexpr (H2)
        load_unit_half(rd, ok ? eoff + (int)__umul24((uint32_t)h, (uint32_t)a.d_rstride) + (rem / UPD) * BD : OOR,
                       rem % UPD, wr[it]);
      else
        load_unit<TD>(rd, ok ? eoff + (int)__umul24((uint32_t)h, (uint32_t)a.d_rstride) + (rem / UPD) * BD : OOR,
                      rem % UPD, wr[it]);
    }
    if constexpr (IS > 0) {
#pragma unroll
      for (int it = 0; it < IS; ++it) {
        const int u = li2 + L2 * it;
        const bool ok = valid && u < USd;
        load_unit<TS>(rsd, ok ? (int)__umul24((uint32_t)h, (uint32_t)a.sd_rstride) + (u / UPS) * BSD : OOR, u % UPS, ws[it]);
      }
    }
  };
  Unit<TD> c2r[IR];
  Unit<TS ? TS : TD> c2s[NS];
  // Q3_K, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS and IQ4_XS down units of the first
  // step are expanded while the workgroup waits for the act rows (their
  // loads have landed by then), so that only the v_dot4s and scale
  // multiply-adds of that step follow the wait
  constexpr bool kExpQ3 = TD == T_Q3_K, kExpIQ2 = TD == T_IQ2_XXS, kExpQ4 = TD == T_Q4_K, kExpQ6 = TD == T_Q6_K;
  constexpr bool kExpIQ3 = TD == T_IQ3_XXS, kExpIQ4 = TD == T_IQ4_XS;
  constexpr bool kExp = kExpQ3 || kExpIQ2 || kExpQ4 || kExpQ6 || kExpIQ3 || kExpIQ4;
  // units expanded (the rest stay raw: register budget; Q6_K's larger raw
  // units leave room for one of three, IQ4_XS's kernel for one)
  constexpr int NE = (kExpQ6 && IR >= 3) || kExpIQ4 ? 1 : (IR < 2 ? IR : 2);
  std::conditional_t<kExpQ3, Q3Exp,
                     std::conditional_t<kExpIQ2, IQ2Exp,
                                        std::conditional_t<kExpQ4, Q4Exp, std::conditional_t<kExpQ6, Q6Exp,
                                                           std::conditional_t<kExpIQ3, IQ3Exp,
                                                                              std::conditional_t<kExpIQ4, IQ4Exp, NoExp>>>>>>
      ex[NE];
  auto expand_step0 = [&]() {
    if constexpr (kExp) {
#pragma unroll
      for (int it = 0; it < NE; ++it) {
        const int u = li2 + L2 * it;
        const int rem = u - (u / URb) * URb;
        if constexpr (kExpQ3)
          q3_expand(c2r[it], rem % UPD, ex[it]);
        else if constexpr (kExpQ4)
          q4_expand(c2r[it], rem % UPD, ex[it]);
        else if constexpr (kExpQ6)
          q6_expand(c2r[it], ex[it]);
        else if constexpr (kExpIQ3)
          iq3_expand(c2r[it], s_grid, s_signs, ex[it]);
        else if constexpr (kExpIQ4)
          iq4_expand(c2r[it], rem % UPD, s_grid, ex[it]);
        else
          iq2_expand(c2r[it], s_grid, s_signs, ex[it]);
      }
    }
  };
  // ---------------------------------------------------------------- P1: routed gate/up rows
  // rows [t0, t1) of the routed row space (route c, row n); the shared rows
  // were streamed before the routing barrier
  const int t0 = (int)((long)T1r * g / G), t1 = (int)((long)T1r * (g + 1) / G);
  stream_rows(RowsTag<TG, false, L1>{}, t0, t1);
  stores_done();
  // The first down step is requested once this workgroup's act stores are
  // acknowledged (stores_done waits for every load and store of the wave), so
  // the down weights stream while the workgroups wait for the act rows.
  // Requested before the gate/up rows they took HBM bandwidth from the rows
  // every workgroup waits for: c2 first gate/up data 8.4 -> 5.2 us after the
  // start, layer 25.9 -> 25.1 us; with a shared expert (c5) 31.4 -> 31.0 us
  // since its shared rows no longer hold up the routing barrier.
  load_step2(0, c2r, c2s);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  ZM_TRACE(2);
  const uint32_t epoch = __builtin_amdgcn_readfirstlane(epoch_v);
  uint32_t *const cnt = a.sync + DEC_CNT_STRIDE * (1 + DEC_NCNT * (int)(epoch & 1u));
  uint32_t *const bcnt = a.sync + DEC_BLK_BASE + DEC_BCNT_STRIDE * DEC_MAX_ABLK * (int)(epoch & 1u);
  // arrival (for the epoch) and rows per act block: row j belongs to block j / 256
  if (tid == 0) atomicAdd(&cnt[DEC_CNT_STRIDE * (g % DEC_NCNT)], 1u);
  {
    // act rows stored: the routed range [Tsh + t0, Tsh + t1) (threads 1..) and
    // the shared range [sh0, sh1) (threads 65..)
    const int r0 = tid < 64 ? Tsh + t0 : sh0, r1 = tid < 64 ? Tsh + t1 : sh1, i = (tid & 63) - 1;
    if (r1 > r0 && tid < 128 && i >= 0 && i <= ((r1 - 1) >> 8) - (r0 >> 8)) {
      const int b = (r0 >> 8) + i;
      atomicAdd(&bcnt[DEC_BCNT_STRIDE * b], (uint32_t)(min(r1, (b + 1) << 8) - max(r0, b << 8)));
    }
  }
  // Clear the other counter set for the next call: its last users were the
  // previous call's workgroups, all finished.  Issued here by wave 0, behind
  // its atomics (at the start these stores sat in the memory counter ahead of
  // the router's loads; at the end their acknowledgements delayed the exit).
  {
    uint32_t *const other = a.sync + DEC_BLK_BASE + DEC_BCNT_STRIDE * DEC_MAX_ABLK * (int)((epoch + 1u) & 1u);
    for (int i = g + G * tid; tid < 64 && i < DEC_MAX_ABLK; i += G * 64) st_co(other + DEC_BCNT_STRIDE * i, 0u);
    if (g == G - 1 && tid < DEC_NCNT)
      st_co(a.sync + DEC_CNT_STRIDE * (1 + DEC_NCNT * (int)((epoch + 1u) & 1u) + tid), 0u);
  }
  ZM_TRACE(3);

  // act rows of this workgroup's tokens (at most two) -> Q8_K in LDS; the rows
  // of skipped routes become zero blocks, so every LDS value read later is finite
  const int s_lo = u1 > u0 ? u0 / H : 0;
  const int s_hi = u1 > u0 ? (u1 - 1) / H : -1;
  const size_t tok_bytes = (size_t)K * q8F + q8Fs;
  if (!s_err) {
    const int nb_tok = K * a.nbF + (a.Fs > 0 ? a.nbFs : 0);
    const int nb_all = (s_hi - s_lo + 1) * nb_tok;
    // block bi -> act byte offset (OOR for a skipped route), LDS row, blocks in
    // that row, block index
    auto info = [&](int bi, int &aoff, uint8_t *&row, int &nb, int &blk) {
      const int ts = bi / nb_tok, r = bi - ts * nb_tok;
      const int s = s_lo + ts;
      if (r < K * a.nbF) {
        const int k = r / a.nbF;
        blk = r - k * a.nbF;
        nb = a.nbF;
        const int c = s_cidx[s * K + k];
        aoff = c < 0 ? OOR : (Tsh + c * F + blk * QK) * 4;
        row = s_q8 + (size_t)ts * tok_bytes + (size_t)k * q8F;
      } else {
        blk = r - K * a.nbF;
        nb = a.nbFs;
        aoff = (s * a.Fs + blk * QK) * 4;
        row = s_q8 + (size_t)ts * tok_bytes + (size_t)K * q8F;
      }
    };
    // Each wave takes 4 blocks per round, QR rounds at a time: it waits until
    // the counters of those blocks show all 256 rows stored (lane i < 4*QR
    // polls one), then issues coalesced 16-byte sc1 loads for all of them (lane
    // l holds floats 4l..4l+3 of block k), transposes each round through this
    // wave's LDS stage to 16 lanes per block and runs quant_block16.  The wait
    // is bounded: on expiry the error word is set and the kernel still drains.
    constexpr int QR = kExp ? 2 : 3;  // 2 with expanded units in registers (c2: its 48 blocks in one round)
    const int kq = lane >> 4;
    bool expanded = false;  // wave-uniform
    const int Tshb = Tsh >> 8;  // act blocks of the shared rows (Fs is a multiple of 256)
    for (int base = wave * 4; base < nb_all; base += DEC_WAVES * 4 * QR) {
      // act offsets of this round's blocks (wave-uniform), worked out before
      // the wait: the divisions and slot-table reads are ~2 us of scalar code
      int aoffs[QR][4];
#pragma unroll
      for (int r = 0; r < QR; ++r) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          int aoff, nb, blk;
          uint8_t *row;
          const int bi = base + r * DEC_WAVES * 4 + k;
          info(min(bi, nb_all - 1), aoff, row, nb, blk);
          aoffs[r][k] = bi >= nb_all ? OOR : aoff;
        }
      }
      // and where this lane's block of each round goes in LDS: row offset
      // (< 64 KiB) | block << 16 | blocks in the row << 24, or ~0u past the end
      uint32_t sinfo[QR];
#pragma unroll
      for (int r = 0; r < QR; ++r) {
        const int bi = base + r * DEC_WAVES * 4 + kq;
        int aoff, nb, blk;
        uint8_t *row;
        info(min(bi, nb_all - 1), aoff, row, nb, blk);
        sinfo[r] = bi < nb_all ? (uint32_t)(row - s_q8) | (uint32_t)blk << 16 | (uint32_t)nb << 24 : ~0u;
      }
      {
        int bid = -1;
        const int bi = base + (lane >> 2) * DEC_WAVES * 4 + (lane & 3);
        if (lane < 4 * QR && bi < nb_all) {
          const int ts = bi / nb_tok, r = bi - ts * nb_tok;
          const int s = s_lo + ts;
          if (r < K * a.nbF) {
            const int k = r / a.nbF;
            const int c = s_cidx[s * K + k];
            bid = c < 0 ? -1 : Tshb + c * a.nbF + (r - k * a.nbF);
          } else {
            bid = s * a.nbFs + (r - K * a.nbF);
          }
        }
        int spins = 0;
        // the first poll is requested before the first-step expansion, whose
        // VALU work then overlaps the poll's round trip
        uint32_t pv = bid < 0 ? (uint32_t)QK : ld_co(&bcnt[DEC_BCNT_STRIDE * bid]);
        if (!expanded) {
          expand_step0();
          expanded = true;
        }
        while (true) {
          const bool ready = bid < 0 || pv >= (uint32_t)QK;
          // a negative limit (a host-forced give-up) expires on the first poll
          if (__ballot(!ready) == 0ull && a.spin_limit >= 0) break;
          __builtin_amdgcn_s_sleep(1);
          if (++spins > a.spin_limit) {
            if (lane == 0) {
              atomicOr(&a.sync[1], 1u);
              s_err = 1;
            }
            break;
          }
          pv = bid < 0 ? (uint32_t)QK : ld_co(&bcnt[DEC_BCNT_STRIDE * bid]);
        }
        after_wait();
      }
      float4 ld[QR][4];
#pragma unroll
      for (int r = 0; r < QR; ++r) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int vo = aoffs[r][k] == OOR ? OOR : aoffs[r][k] + 16 * lane;
          const auto v4 = __builtin_amdgcn_raw_buffer_load_b128(ract, vo, 0, 16);
          ld[r][k] = make_float4(__uint_as_float(v4[0]), __uint_as_float(v4[1]), __uint_as_float(v4[2]),
                                 __uint_as_float(v4[3]));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < QR; ++r) {
        if (base + r * DEC_WAVES * 4 >= nb_all) break;
#pragma unroll
        for (int k = 0; k < 4; ++k) s_stage[wave][k * 64 + lane] = ld[r][k];
        stage_sync();
        float xv16[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 f = s_stage[wave][kq * 64 + 4 * l16 + i];
          xv16[4 * i] = f.x;
          xv16[4 * i + 1] = f.y;
          xv16[4 * i + 2] = f.z;
          xv16[4 * i + 3] = f.w;
        }
        stage_sync();
        if (sinfo[r] != ~0u)  // a zero block for a skipped route
          store_q8_16l(s_q8 + (sinfo[r] & 0xffffu), (int)(sinfo[r] >> 24), (int)((sinfo[r] >> 16) & 0xffu),
                       quant_block16(xv16, l16), l16);
      }
    }
    if (!expanded) expand_step0();  // a wave without act blocks to fetch
  }
  __syncthreads();
  ZM_TRACE(4);
  // workgroup 0 reads the arrival counters now, so that the read is back by
  // the end of the down rows (all workgroups have arrived by then in practice:
  // their arrivals precede the act blocks this workgroup has just waited for)
  int arrived = 0;
  if (g == 0 && wave == 0) {
    const int c = lane < DEC_NCNT ? (int)ld_co(&cnt[DEC_CNT_STRIDE * lane]) : 0;
    arrived = __builtin_amdgcn_readlane(group_sum_i<16>(c), 0);
  }

  if (s_err) {
    // this call's wait expired: its output rows are marked, not left stale
    for (int j = u0 + tid; j < u1; j += DEC_THREADS) bst(rout, 4 * j, __builtin_nanf(""));
  } else {
    // one down step; FIRST (the first step of a layer with an expanded down
    // type) dots the units expanded during the act wait, so the raw units are
    // dead until the next step's loads
    auto down_step = [&](int st, auto first_tag) {
      constexpr bool FIRST = decltype(first_tag)::value;
      bool valid;
      int s, h;
      row2(st, valid, s, h);
      const uint8_t *tb = s_q8 + (size_t)(s - s_lo) * tok_bytes;
      float acc = 0.f;
#pragma unroll
      for (int it = 0; it < IR; ++it) {
        const int u = li2 + L2 * it;
        const int k = min(u / URb, K - 1), rem = u - (u / URb) * URb;
        const float wk = u < URd ? s_w[s * K + k] : 0.0f;
        float o[1];
        const XBlk xb = xblk(tb + (size_t)k * q8F, a.nbF, min(rem / UPD, a.nbF - 1));
        if (kExp && FIRST && it < NE) {  // (it is a constant after unrolling)
          o[0] = exp_dot(ex[it < NE ? it : 0], rem % UPD, xb);
        } else {
          const Unit<TD> one[1] = {c2r[it]};
          unit_dots<TD, 1, H2>(one, rem % UPD, xb, s_grid, s_signs, o);
        }
        acc += wk * o[0];
      }
      if constexpr (IS > 0) {
#pragma unroll
        for (int it = 0; it < IS; ++it) {
          const int u = li2 + L2 * it;
          float o[1];
          const Unit<TS ? TS : TD> one[1] = {c2s[it]};
          unit_dots<TS ? TS : TD, 1>(one, u % UPS, xblk(tb + (size_t)K * q8F, a.nbFs, min(u / UPS, a.nbFs - 1)),
                                     s_grid, s_signs, o);
          acc += o[0];
        }
      }
      acc = group_sum<L2>(acc);
      bst(rout, (li2 == 0 && valid) ? 4 * (s * H + h) : OOR, acc);
      __builtin_amdgcn_sched_barrier(0);
      if (st + 1 < nst2) load_step2(st + 1, c2r, c2s);  // (the unpacking of a unit costs VALU even when out of range)
      __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (kExp) {
      if (nst2 > 0) down_step(0, std::true_type{});
      for (int st = 1; st < nst2; ++st) down_step(st, std::false_type{});
    } else {
      for (int st = 0; st < nst2; ++st) down_step(st, std::false_type{});
    }
  }
  ZM_TRACE(5);
  // workgroup 0 retires the epoch once every workgroup has arrived (each read
  // the epoch before arriving); after an expired wait the epoch stays (the host
  // resets the sync words)
  if (g == 0 && wave == 0) {
    int spins = 0;
    bool ok = true;
    while (arrived < G) {
      const int c = lane < DEC_NCNT ? (int)ld_co(&cnt[DEC_CNT_STRIDE * lane]) : 0;
      const int total = __builtin_amdgcn_readlane(group_sum_i<16>(c), 0);
      if (total >= G) break;
      __builtin_amdgcn_s_sleep(1);
      if (++spins > a.spin_limit) {
        ok = false;
        if (lane == 0) atomicOr(&a.sync[1], 1u);
        break;
      }
    }
    if (ok && lane == 0 && !s_err) st_co(&a.sync[0], epoch + 1u);
  }
  // slot 7 from the first x-quantization worker (the one with the most
  // groups), the others from thread 0
  if (a.trace && tid == 0) {
#pragma unroll
    for (int i = 0; i < 7; ++i) a.trace[(size_t)g * 8 + i] = trace_t[i];
  }
  if (a.trace && tid == 64 * (S < DEC_WAVES ? S : 0)) a.trace[(size_t)g * 8 + 7] = trace_t[7];
}

#undef ZM_TRACE

using DecFn = void (*)(DecodeArgs);

template <int TG, int TD, int TS, int L1>
DecFn dec_pick2(int ir, int is) {
  if (is != (TS ? 1 : 0)) return nullptr;
  constexpr int IS = TS ? 1 : 0;
  if (ir <= 2) return k_moe_decode<TG, TD, TS, L1, 2, IS>;
  if (ir <= 3) return k_moe_decode<TG, TD, TS, L1, 3, IS>;
  return nullptr;
}

// L1: lanes per routed gate/up row (16 or 32, one unit each; shared rows use
// 64); IR / IS: 32-lane iterations over the routed / shared units of a down row
template <int TG, int TD, int TS>
DecFn dec_pick(int l1, int ir, int is) {
  if constexpr (TG == T_IQ2_XXS)
    if (l1 == 20) return dec_pick2<TG, TD, TS, 20>(ir, is);
  if (l1 == 16) return dec_pick2<TG, TD, TS, 16>(ir, is);
  if (l1 == 32) return dec_pick2<TG, TD, TS, 32>(ir, is);
  return nullptr;
}

// The instantiated decode kernels, split over two translation units so they
// compile in parallel (zm_dec_a.hip, zm_dec_b.hip); nullptr when the layer's
// (gate, down, shared) types or unit counts have no instantiation.
DecFn find_decode_a(int tg, int td, int ts, int l1, int ir, int is);
DecFn find_decode_b(int tg, int td, int ts, int l1, int ir, int is);

}  // namespace zm
