// zm_decode.hpp -- one persistent kernel for a whole routed MoE layer at
// decode sizes (S <= 8 tokens): router -> Q8_K(x) -> gate/up + SwiGLU ->
// Q8_K(act) -> down -> weighted top-k sum (+ shared expert), with no kernel
// boundary in between.
//
// Grid: as many 512-thread workgroups as the device holds at once.
//   P0  every workgroup routes all tokens and quantizes x into LDS --
//       redundant, but no grid-wide barrier precedes the first weight request.
//       Each wave then requests the weights of its first down rows (P2), so
//       they stream while gate/up computes and while the workgroups wait.
//   P1  the (pair, row) space of gate/up rows is cut into one contiguous range
//       per workgroup; waves stream batches of rows (double-buffered) and store
//       the SwiGLU output; the workgroup then adds its row count to one of 16
//       rows-done counters.
//   P2  down rows (token s, row h): the workgroup waits until the counters sum
//       to all rows, quantizes the act rows of its tokens into LDS (Q8_K) and
//       computes out[s][h] = sum_k w_k * (W_down[e_k][h] . q8(act_k)) (+ shared).
//   Exit: the last workgroup to leave zeroes the sync words for the next call.
// The hot loops carry no lane-divergent branches: a lane without work loads
// through an out-of-range buffer offset, which returns zeros, so its dot is 0.
// Cross-workgroup data moves through agent-scope relaxed atomic loads/stores
// (sc1: coherent past the per-XCD L2s) and one counter; no agent-scope fence
// (an L2 write-back + invalidate on gfx950) is issued.  The wait is bounded:
// on expiry the error word is set and the kernel still drains.
#pragma once

#include "zm_kernels.hpp"

namespace zm {

constexpr int DEC_THREADS = 512;
constexpr int DEC_WAVES = DEC_THREADS / 64;
constexpr int DEC_MAX_S = 8;
constexpr int DEC_MAX_PAIRS = 128;  // S * K
constexpr int DEC_LDS_Q8 = 65536;   // Q8_K staging: x rows in P0/P1, act rows in P2
constexpr int DEC_NCNT = 16;        // rows-done counters (one 64-byte line each) to spread the atomics
constexpr int DEC_CNT_STRIDE = 16;  // words between counters
constexpr int DEC_SYNC_WORDS = DEC_CNT_STRIDE * (1 + DEC_NCNT);
// lane offset past every buffer extent (all < 2^31): such a load returns zeros
constexpr int OOR = (int)0x80000000u;

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
  uint32_t wg_bytes, wd_bytes, sg_bytes, sd_bytes;  // buffer-resource extents (< 4 GiB)
  float *act;
  uint32_t *sync;  // [0] workgroups exited, [1] error, [DEC_CNT_STRIDE*(1+i)] rows-done counter i
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
#define ZM_TRACE(slot)                                                         \
  do {                                                                         \
    if (a.trace && tid == 0) a.trace[(size_t)g * 8 + (slot)] = wall_clock64(); \
  } while (0)

template <int TG, int TD, int TS, int IT1, int ITR, int ITS>
__global__ __launch_bounds__(DEC_THREADS) void k_moe_decode(DecodeArgs a) {
  __shared__ int s_ids[DEC_MAX_PAIRS];
  __shared__ float s_w[DEC_MAX_PAIRS];
  __shared__ int s_cidx[DEC_MAX_PAIRS];  // pair -> compact routed index (or -1)
  __shared__ int s_vp[DEC_MAX_PAIRS];    // compact index -> pair
  __shared__ int s_nvp;
  __shared__ int s_err;
  __shared__ __attribute__((aligned(16))) uint8_t s_q8[DEC_LDS_Q8];
  __shared__ float4 s_stage[DEC_WAVES][256];  // per-wave transpose of 4 act blocks
  constexpr bool kIQ2 = TG == T_IQ2_XXS || TD == T_IQ2_XXS || TS == T_IQ2_XXS;
  __shared__ uint64_t s_grid[kIQ2 ? 256 : 1];
  __shared__ uint64_t s_signs[kIQ2 ? 128 : 1];
  static_assert(ITS == 0 || TS != 0, "shared iterations need a shared type");
  constexpr int NS = ITS > 0 ? ITS : 1;

  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6);
  const int q4 = lane & 3;  // quarter of a super-block this lane handles (every unit count is a multiple of 4)
  const int G = gridDim.x, g = blockIdx.x;
  const int S = a.S, K = a.K, H = a.H, F = a.F;
  const size_t q8x = q8_row_bytes(a.nbH);
  const size_t q8F = q8_row_bytes(a.nbF);
  const size_t q8Fs = a.Fs > 0 ? q8_row_bytes(a.nbFs) : 0;
  ZM_TRACE(0);

  // ---------------------------------------------------------------- P0: route, quantize x
  // Wave w < S routes token w (its loads go out first); the other waves
  // quantize x (16 lanes per block, 4 blocks per wave and round), then the
  // routing waves join them.
  if (tid == 0) s_err = 0;
  const int nxb = S * a.nbH;
  const int l16 = lane & 15;
  const int wi = wave >= S ? wave - S : wave + DEC_WAVES - S;  // x-quant worker index
  float xv[16];
  auto load_x = [&](int grp) {
    const int bb = grp * 4 + (lane >> 4);
    if (bb < nxb) {
      const int s = bb / a.nbH, b = bb % a.nbH;
      const float4 *src = reinterpret_cast<const float4 *>(a.x + (size_t)s * H + (size_t)b * QK + 16 * l16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 f = src[i];
        xv[4 * i] = f.x;
        xv[4 * i + 1] = f.y;
        xv[4 * i + 2] = f.z;
        xv[4 * i + 3] = f.w;
      }
    }
  };
  if (wave < S) {
    const WaveRoute r = route_token(a.r, wave, reinterpret_cast<float *>(s_stage[wave]));
    if (lane < K) {
      s_ids[wave * K + lane] = r.id;
      s_w[wave * K + lane] = r.w;
      if (g == 0 && a.r.ids) {
        a.r.ids[wave * K + lane] = r.id;
        a.r.weights[wave * K + lane] = r.w;
      }
    }
  }
  if constexpr (kIQ2) {
    for (int i = tid; i < 256; i += DEC_THREADS) s_grid[i] = a.grid[i];
    for (int i = tid; i < 128; i += DEC_THREADS) s_signs[i] = a.signs[i];
  }
  ZM_TRACE(6);
  for (int grp = wi; grp * 4 < nxb; grp += DEC_WAVES) {
    load_x(grp);
    const int bb = grp * 4 + (lane >> 4);
    if (bb < nxb) {
      const int s = bb / a.nbH, b = bb % a.nbH;
      store_q8_16(s_q8 + (size_t)s * q8x, a.nbH, b, quant_block16(xv, l16), l16);
    }
  }
  ZM_TRACE(7);
  __syncthreads();
  if (wave == 0) {
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
      if (p < S * K && s_cidx[p] >= 0) s_vp[s_cidx[p]] = p;
    }
    if (lane == 0) s_nvp = n;
  }
  __syncthreads();
  ZM_TRACE(1);
  const int nvp = s_nvp;
  const int T1r = nvp * F;
  const int T1 = T1r + S * a.Fs;

  // ---------------------------------------------------------------- P2 set-up: down rows
  // Lane unit v = lane + 64*it of a down row: the ITR routed iterations cover
  // K*U2 quarters (route v / U2, quarter v % U2), the ITS shared iterations the
  // shared expert's U2s quarters.  Lane offsets depend on the token only.  The
  // first rows of every wave are requested now, before any gate/up work.
  const int T2 = S * H;
  const int u0 = (int)((long)T2 * g / G), u1 = (int)((long)T2 * (g + 1) / G);
  const float invH = 1.0f / (float)H;
  const int U2 = 4 * a.nbF, U2s = 4 * a.nbFs;
  constexpr int BD = block_bytes(TD);
  constexpr int BSD = TS ? block_bytes(TS) : 1;
  const rsrc_t rd = make_rsrc(a.wd, a.wd_bytes), rsd = make_rsrc(a.sd, a.sd_bytes);
  int vo_r[ITR], vo_s[NS];
  int vo_tok = -1;
  auto lane_offsets = [&](int s) {
#pragma unroll
    for (int it = 0; it < ITR; ++it) {
      const int v = lane + 64 * it;
      const int k = v / U2, u = v - k * U2;
      const int e = s_ids[s * K + min(k, K - 1)];
      vo_r[it] = (k < K && e >= 0) ? e * (int)a.d_estride + (u >> 2) * BD : OOR;
    }
#pragma unroll
    for (int it = 0; it < ITS; ++it) {
      const int u = lane + 64 * it;
      vo_s[it] = u < U2s ? (u >> 2) * BSD : OOR;
    }
    vo_tok = s;
  };
  auto load_row = [&](int j, WSlice(&wr)[ITR], WSlice(&ws)[NS]) {
    int s, h;
    divmod24(j, H, invH, s, h);
    s = uniform(s);
    h = uniform(h);
    if (s != vo_tok) lane_offsets(s);
    const int so = uniform(h * (int)a.d_rstride);
#pragma unroll
    for (int it = 0; it < ITR; ++it) load_w_slice_b<TD>(rd, vo_r[it], so, q4, wr[it]);
    if constexpr (ITS > 0) {
      const int sos = uniform(h * (int)a.sd_rstride);
#pragma unroll
      for (int it = 0; it < ITS; ++it) load_w_slice_b<TS>(rsd, vo_s[it], sos, q4, ws[it]);
    }
  };
  // two rows in flight when they fit in registers, else one
  constexpr bool P2DB = ITR + ITS <= 3;
  WSlice c0r[ITR], c0s[NS];
  WSlice c1r[P2DB ? ITR : 1], c1s[P2DB ? NS : 1];
  const int jw = u0 + wave;
  if (jw < u1) load_row(jw, c0r, c0s);
  if constexpr (P2DB)
    if (jw + DEC_WAVES < u1) load_row(jw + DEC_WAVES, c1r, c1s);
  __builtin_amdgcn_sched_barrier(0);

  // ---------------------------------------------------------------- P1: gate/up rows
  // Row i of this wave is j = t0 + wave + DEC_WAVES*i.  Rows go in batches of RB
  // with two register buffers: batch b+1 is in flight while batch b computes.
  const int t0 = (int)((long)T1 * g / G), t1 = (int)((long)T1 * (g + 1) / G);
  const int U1 = 4 * a.nbH;
  const float invF = 1.0f / (float)F, invFs = a.Fs > 0 ? 1.0f / (float)a.Fs : 0.f;
  {
    constexpr int BG = block_bytes(TG);
    constexpr int BS = TS ? block_bytes(TS) : 1;
    constexpr int SLICE_DW = TG == T_Q2_K ? 7 : (TG == T_Q4_K ? 12 : (TG == T_IQ2_XXS ? 5 : 12));
    constexpr int RB0 = 80 / (2 * 2 * SLICE_DW * IT1);
    constexpr int RB = RB0 < 1 ? 1 : (RB0 > 4 ? 4 : RB0);
    const int nrw = t1 - t0 > wave ? (t1 - t0 - wave + DEC_WAVES - 1) / DEC_WAVES : 0;
    const rsrc_t rg = make_rsrc(a.wg, a.wg_bytes), ru = make_rsrc(a.wu, a.wg_bytes);
    const rsrc_t rsg = make_rsrc(a.sg, a.sg_bytes), rsu = make_rsrc(a.su, a.sg_bytes);
    // lane offsets inside a row (routed / shared block sizes; OOR past the row)
    // and the activation block (clamped: idle lanes read real, finite data)
    int vo1[IT1], vo1s[IT1], xb1[IT1];
#pragma unroll
    for (int it = 0; it < IT1; ++it) {
      const int u = lane + 64 * it;
      vo1[it] = u < U1 ? (u >> 2) * BG : OOR;
      vo1s[it] = u < U1 ? (u >> 2) * BS : OOR;
      xb1[it] = min(u >> 2, a.nbH - 1);
    }
    auto issue = [&](int i0, WSlice(&bg)[RB][IT1], WSlice(&bu)[RB][IT1]) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int i = i0 + r;
        if (i >= nrw) break;
        const int j = t0 + wave + DEC_WAVES * i;
        if (j < T1r) {
          int c, n;
          divmod24(j, F, invF, c, n);
          const int e = uniform(s_ids[s_vp[uniform(c)]]);
          const int so = uniform(e * (int)a.g_estride + uniform(n) * (int)a.g_rstride);
#pragma unroll
          for (int it = 0; it < IT1; ++it) {
            load_w_slice_b<TG>(rg, vo1[it], so, q4, bg[r][it]);
            load_w_slice_b<TG>(ru, vo1[it], so, q4, bu[r][it]);
          }
        } else if constexpr (TS != 0) {
          int ts_, n;
          divmod24(j - T1r, a.Fs, invFs, ts_, n);
          const int so = uniform(uniform(n) * (int)a.sg_rstride);
#pragma unroll
          for (int it = 0; it < IT1; ++it) {
            load_w_slice_b<TS>(rsg, vo1s[it], so, q4, bg[r][it]);
            load_w_slice_b<TS>(rsu, vo1s[it], so, q4, bu[r][it]);
          }
        }
      }
    };
    // the token's activation slices stay in registers while the token does not change
    Q8Slice xsc[IT1];
    int xs_key = -1;
    auto compute = [&](int i0, WSlice(&bg)[RB][IT1], WSlice(&bu)[RB][IT1]) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int i = i0 + r;
        if (i >= nrw) break;
        const int j = t0 + wave + DEC_WAVES * i;
        const bool shared_row = j >= T1r;
        int q_, r_;
        divmod24(shared_row ? j - T1r : j, shared_row ? a.Fs : F, shared_row ? invFs : invF, q_, r_);
        const int tok = uniform(shared_row ? q_ : s_vp[q_] / K);
        const int key = shared_row ? tok + DEC_MAX_S : tok;
        if (key != xs_key) {
          xs_key = key;
          const uint8_t *xrow = s_q8 + (size_t)tok * q8x;
#pragma unroll
          for (int it = 0; it < IT1; ++it) {
            if (!shared_row)
              load_q8_slice<TG>(xrow, a.nbH, xb1[it], q4, xsc[it]);
            else if constexpr (TS != 0)
              load_q8_slice<TS>(xrow, a.nbH, xb1[it], q4, xsc[it]);
          }
        }
        float ag = 0.f, au = 0.f;
        if (!shared_row) {
#pragma unroll
          for (int it = 0; it < IT1; ++it) {
            ag += quarter_dot<TG>(bg[r][it], q4, xsc[it], s_grid, s_signs);
            au += quarter_dot<TG>(bu[r][it], q4, xsc[it], s_grid, s_signs);
          }
        } else if constexpr (TS != 0) {
#pragma unroll
          for (int it = 0; it < IT1; ++it) {
            ag += quarter_dot<TS>(bg[r][it], q4, xsc[it], s_grid, s_signs);
            au += quarter_dot<TS>(bu[r][it], q4, xsc[it], s_grid, s_signs);
          }
        }
        ag = group_sum<64>(ag);
        au = group_sum<64>(au);
        if (lane == 0) st_co(a.act + j, silu_f32(ag) * au);
      }
    };
    // sched_barrier keeps every load of a batch ahead of the math that waits on
    // the previous one (vmcnt is in order: an interleaved wait drains the queue)
    WSlice g0[RB][IT1], v0[RB][IT1], g1[RB][IT1], v1[RB][IT1];
    if (nrw > 0) issue(0, g0, v0);
    for (int i0 = 0; i0 < nrw; i0 += 2 * RB) {
      if (i0 + RB < nrw) issue(i0 + RB, g1, v1);
      __builtin_amdgcn_sched_barrier(0);
      compute(i0, g0, v0);
      if (i0 + RB < nrw) {
        if (i0 + 2 * RB < nrw) issue(i0 + 2 * RB, g0, v0);
        __builtin_amdgcn_sched_barrier(0);
        compute(i0 + RB, g1, v1);
      }
    }
  }
  stores_done();
  __syncthreads();
  ZM_TRACE(2);
  if (tid == 0 && t1 > t0) atomicAdd(&a.sync[DEC_CNT_STRIDE * (1 + g % DEC_NCNT)], (uint32_t)(t1 - t0));

  // ---------------------------------------------------------------- P2: wait, quantize act, down rows
  // lanes 0..15 of wave 0 poll one counter each and sum them
  if (wave == 0) {
    const uint32_t target = (uint32_t)T1;
    int spins = 0;
    while (true) {
      const int c = lane < DEC_NCNT ? (int)ld_co(&a.sync[DEC_CNT_STRIDE * (1 + lane)]) : 0;
      const uint32_t total = (uint32_t)__builtin_amdgcn_readlane(group_sum_i<16>(c), 0);
      if (total >= target) break;
      __builtin_amdgcn_s_sleep(1);
      if (++spins > a.spin_limit) {
        if (lane == 0) {
          atomicOr(&a.sync[1], 1u);
          s_err = 1;
        }
        break;
      }
    }
  }
  __syncthreads();
  after_wait();
  ZM_TRACE(3);

  // act rows of this workgroup's tokens (at most two) -> Q8_K in LDS; the rows
  // of skipped routes become zero blocks, so every LDS value read later is finite
  const int s_lo = u1 > u0 ? u0 / H : 0;
  const int s_hi = u1 > u0 ? (u1 - 1) / H : -1;
  const size_t tok_bytes = (size_t)K * q8F + q8Fs;
  if (!s_err) {
    const int nb_tok = K * a.nbF + (a.Fs > 0 ? a.nbFs : 0);
    const int nb_all = (s_hi - s_lo + 1) * nb_tok;
    // block bi -> act byte offset (OOR: skipped route or past the end), LDS row,
    // blocks in that row, block index
    auto info = [&](int bi, int &aoff, uint8_t *&row, int &nb, int &blk) {
      const int ts = bi / nb_tok, r = bi - ts * nb_tok;
      const int s = s_lo + ts;
      if (r < K * a.nbF) {
        const int k = r / a.nbF;
        blk = r - k * a.nbF;
        nb = a.nbF;
        const int c = s_cidx[s * K + k];
        aoff = c < 0 ? OOR : (c * F + blk * QK) * 4;
        row = s_q8 + (size_t)ts * tok_bytes + (size_t)k * q8F;
      } else {
        blk = r - K * a.nbF;
        nb = a.nbFs;
        aoff = (T1r + s * a.Fs + blk * QK) * 4;
        row = s_q8 + (size_t)ts * tok_bytes + (size_t)K * q8F;
      }
    };
    // Each wave takes 4 blocks per round: coalesced 16-byte sc1 loads (lane l
    // holds floats 4l..4l+3 of block k), a transpose through this wave's LDS
    // stage to 16 lanes per block, then quant_block16.  QR rounds of loads are
    // in flight together.
    constexpr int QR = 3;
    const rsrc_t ract = make_rsrc(a.act, (uint32_t)T1 * 4u);
    const int kq = lane >> 4;
    for (int base = wave * 4; base < nb_all; base += DEC_WAVES * 4 * QR) {
      float4 ld[QR][4];
#pragma unroll
      for (int r = 0; r < QR; ++r) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          int aoff, nb, blk;
          uint8_t *row;
          const int bi = base + r * DEC_WAVES * 4 + k;
          info(min(bi, nb_all - 1), aoff, row, nb, blk);
          const int vo = (bi >= nb_all || aoff == OOR) ? OOR : aoff + 16 * lane;
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
        const int bi = base + r * DEC_WAVES * 4 + kq;
        if (bi < nb_all) {
          int aoff, nb, blk;
          uint8_t *row;
          info(bi, aoff, row, nb, blk);
          store_q8_16(row, nb, blk, quant_block16(xv16, l16), l16);  // a zero block for a skipped route
        }
      }
    }
  }
  __syncthreads();
  ZM_TRACE(4);

  if (!s_err) {
    int cur_s = -1;
    Q8Slice qr[ITR], qsh[NS];
    float wgt[ITR];
    auto compute_row = [&](int j, WSlice(&cr)[ITR], WSlice(&cs)[NS]) {
      int s, h;
      divmod24(j, H, invH, s, h);
      s = uniform(s);
      h = uniform(h);
      if (s != cur_s) {
        cur_s = s;
        const uint8_t *tb = s_q8 + (size_t)(s - s_lo) * tok_bytes;
#pragma unroll
        for (int it = 0; it < ITR; ++it) {
          const int v = lane + 64 * it;
          const int kr = v / U2, u = v - kr * U2, k = min(kr, K - 1);
          load_q8_slice<TD>(tb + (size_t)k * q8F, a.nbF, u >> 2, q4, qr[it]);
          wgt[it] = kr < K ? s_w[s * K + k] : 0.0f;
        }
#pragma unroll
        for (int it = 0; it < ITS; ++it) {
          const int u = lane + 64 * it;
          load_q8_slice<TS>(tb + (size_t)K * q8F, a.nbFs, min(u >> 2, a.nbFs - 1), q4, qsh[it]);
        }
      }
      float acc = 0.f;
#pragma unroll
      for (int it = 0; it < ITR; ++it) acc += wgt[it] * quarter_dot<TD>(cr[it], q4, qr[it], s_grid, s_signs);
#pragma unroll
      for (int it = 0; it < ITS; ++it) acc += quarter_dot<TS>(cs[it], q4, qsh[it], s_grid, s_signs);
      acc = group_sum<64>(acc);
      if (lane == 0) a.out[(size_t)s * H + h] = acc;
    };
    if constexpr (P2DB) {
      for (int j = jw; j < u1; j += 2 * DEC_WAVES) {
        compute_row(j, c0r, c0s);
        if (j + 2 * DEC_WAVES < u1) load_row(j + 2 * DEC_WAVES, c0r, c0s);
        __builtin_amdgcn_sched_barrier(0);
        if (j + DEC_WAVES < u1) {
          compute_row(j + DEC_WAVES, c1r, c1s);
          if (j + 3 * DEC_WAVES < u1) load_row(j + 3 * DEC_WAVES, c1r, c1s);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else {
      for (int j = jw; j < u1; j += DEC_WAVES) {
        compute_row(j, c0r, c0s);
        if (j + DEC_WAVES < u1) load_row(j + DEC_WAVES, c0r, c0s);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  ZM_TRACE(5);

  // ---------------------------------------------------------------- exit: the last workgroup zeroes the sync words
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = atomicAdd(&a.sync[0], 1u);
    if (old == (uint32_t)G - 1) {
      for (int i = 0; i < DEC_NCNT; ++i) st_co(&a.sync[DEC_CNT_STRIDE * (1 + i)], 0u);
      st_co(&a.sync[0], 0u);
    }
  }
}

#undef ZM_TRACE

}  // namespace zm
