// zm_decode.hpp -- one persistent kernel for a whole routed MoE layer at
// decode sizes (S <= 8 tokens): router -> Q8_K(x) -> gate/up + SwiGLU ->
// Q8_K(act) -> down -> weighted top-k sum (+ shared expert), with no kernel
// boundary in between.
//
// Launch: cooperative (all workgroups co-resident), 512 threads each.
//   P0  every workgroup routes all tokens (one wave) and quantizes x into LDS
//       (other waves) -- redundant but a few hundred cycles, and it avoids a
//       grid-wide barrier before the first weight byte is requested.
//   P1  the (pair, row) space of gate/up rows is cut into one contiguous
//       range per workgroup; waves stream two rows at a time and write the
//       SwiGLU output.  Each 256-row act block has a completion counter; the
//       workgroup whose rows complete a block quantizes it to Q8_K and bumps
//       `done`.
//   P2  down rows: each wave first issues the weight loads of its first row,
//       then waits for `done` to reach the block count, then computes
//       out[s][h] = sum_k w_k * (W_down[e_k][h] . q8(act_k)) (+ shared).
//   Exit: the last workgroup to leave resets the counters to zero, so the
//       sync words are zero again for the next launch on the stream.
// Waits are bounded (spin limit): on expiry the error word is set and the
// kernel still drains, so no launch can hang the device.
#pragma once

#include "zm_kernels.hpp"

namespace zm {

constexpr int DEC_THREADS = 512;
constexpr int DEC_WAVES = DEC_THREADS / 64;
constexpr int DEC_MAX_S = 8;
constexpr int DEC_MAX_PAIRS = 128;        // S * K
constexpr int DEC_MAX_XQ_BLOCKS = 128;    // S * H / 256
constexpr int DEC_MAX_TOUCH = 16;         // act blocks one workgroup's P1 range may touch

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
  float *act;
  uint8_t *aq;
  uint32_t *sync;  // [0] done, [1] exit, [2] error, [3] unused, [4..] act block counters
  const uint64_t *grid, *signs;
  int spin_limit;
};

__device__ __forceinline__ uint32_t ld_acq(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int T>
__device__ __forceinline__ void load_q8_lds_slice(const uint8_t *row, int nb, int u, Q8Slice &s) {
  load_q8_slice<T>(row, nb, u >> 2, u & 3, s);
}

template <int TG, int TD, int TS, int IT1, int IT2>
__global__ __launch_bounds__(DEC_THREADS) void k_moe_decode(DecodeArgs a) {
  __shared__ float s_p[ROUTER_MAX_E];
  __shared__ float s_sel[ROUTER_MAX_E];
  __shared__ float s_gs[64];
  __shared__ int s_ids[DEC_MAX_PAIRS];
  __shared__ float s_w[DEC_MAX_PAIRS];
  __shared__ int s_cidx[DEC_MAX_PAIRS];   // pair -> compact routed index (or -1)
  __shared__ int s_vp[DEC_MAX_PAIRS];     // compact index -> pair
  __shared__ int s_nvp;
  __shared__ int s_quant[DEC_MAX_TOUCH];
  __shared__ int s_nquant;
  __shared__ int s_err;
  __shared__ __attribute__((aligned(16))) uint8_t s_xq[DEC_MAX_XQ_BLOCKS * 292];
  __shared__ uint64_t s_grid[(TG == T_IQ2_XXS || TD == T_IQ2_XXS || TS == T_IQ2_XXS) ? 256 : 1];
  __shared__ uint64_t s_signs[(TG == T_IQ2_XXS || TD == T_IQ2_XXS || TS == T_IQ2_XXS) ? 128 : 1];
  constexpr bool kIQ2 = TG == T_IQ2_XXS || TD == T_IQ2_XXS || TS == T_IQ2_XXS;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = gridDim.x, g = blockIdx.x;
  const int S = a.S, K = a.K, H = a.H, F = a.F;
  const size_t q8x = q8_row_bytes(a.nbH);
  const size_t q8F = q8_row_bytes(a.nbF);
  const size_t q8Fs = a.Fs > 0 ? q8_row_bytes(a.nbFs) : 0;

  // ---------------------------------------------------------------- P0
  if constexpr (kIQ2) {
    for (int i = tid; i < 256; i += DEC_THREADS) s_grid[i] = a.grid[i];
    for (int i = tid; i < 128; i += DEC_THREADS) s_signs[i] = a.signs[i];
  }
  if (tid == 0) s_err = 0;
  if (wave == 0) {
    for (int s = 0; s < S; ++s) {
      int id;
      float w;
      router_token(a.r, s, lane, s_p, s_sel, s_gs, id, w);
      if (lane < K) {
        s_ids[s * K + lane] = id;
        s_w[s * K + lane] = w;
        if (g == 0 && a.r.ids) {
          a.r.ids[s * K + lane] = id;
          a.r.weights[s * K + lane] = w;
        }
      }
      wave_sync();
    }
    if (lane == 0) {
      int n = 0;
      for (int p = 0; p < S * K; ++p) {
        if (s_ids[p] >= 0) {
          s_cidx[p] = n;
          s_vp[n++] = p;
        } else {
          s_cidx[p] = -1;
        }
      }
      s_nvp = n;
    }
  } else {
    const int nblk = S * a.nbH;
    for (int bi = wave - 1; bi < nblk; bi += DEC_WAVES - 1) {
      const int s = bi / a.nbH, b = bi % a.nbH;
      const float4 v = *reinterpret_cast<const float4 *>(a.x + (size_t)s * H + (size_t)b * QK + 4 * lane);
      const Q8Out o = quant_block_wave(v, lane);
      uint8_t *row = s_xq + (size_t)s * q8x;
      const uint32_t packed = (uint32_t)(uint8_t)o.q[0] | ((uint32_t)(uint8_t)o.q[1] << 8) |
                              ((uint32_t)(uint8_t)o.q[2] << 16) | ((uint32_t)(uint8_t)o.q[3] << 24);
      *reinterpret_cast<uint32_t *>(row + (size_t)b * QK + 4 * lane) = packed;
      if (lane == 0) reinterpret_cast<float *>(row + q8_d_off(a.nbH))[b] = o.d;
      if ((lane & 3) == 0) reinterpret_cast<int16_t *>(row + q8_bs_off(a.nbH))[b * 16 + (lane >> 2)] = (int16_t)o.bsum16;
    }
  }
  __syncthreads();
  const int nvp = s_nvp;

  // ---------------------------------------------------------------- P1: gate/up rows
  const long T1r = (long)nvp * F;
  const long T1 = T1r + (long)S * a.Fs;
  const long t0 = T1 * g / G, t1 = T1 * (g + 1) / G;
  const int U1 = 4 * a.nbH;
  {
    constexpr int BG = block_bytes(TG);
    constexpr int BS = TS ? block_bytes(TS) : 1;
    for (long j0 = t0 + wave; j0 < t1; j0 += 2 * DEC_WAVES) {
      WSlice wgs[2][IT1], wus[2][IT1];
      bool rv[2];
      bool shared_row[2];
      int tok[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const long j = j0 + (long)r * DEC_WAVES;
        rv[r] = j < t1;
        shared_row[r] = j >= T1r;
        const uint8_t *gp, *up;
        if (!shared_row[r]) {
          const int c = (int)(j / F), n = (int)(j % F);
          const int p = s_vp[rv[r] ? c : 0];
          tok[r] = p / K;
          const size_t off = (size_t)s_ids[p] * a.g_estride + (size_t)n * a.g_rstride;
          gp = a.wg + off;
          up = a.wu + off;
        } else {
          const long js = j - T1r;
          tok[r] = (int)(js / a.Fs);
          const int n = (int)(js % a.Fs);
          gp = a.sg + (size_t)n * a.sg_rstride;
          up = a.su + (size_t)n * a.sg_rstride;
        }
#pragma unroll
        for (int it = 0; it < IT1; ++it) {
          const int u = lane + 64 * it;
          if (rv[r] && u < U1) {
            if (!shared_row[r]) {
              load_w_slice<TG>(gp + (size_t)(u >> 2) * BG, u & 3, wgs[r][it]);
              load_w_slice<TG>(up + (size_t)(u >> 2) * BG, u & 3, wus[r][it]);
            } else if constexpr (TS != 0) {
              load_w_slice<TS>(gp + (size_t)(u >> 2) * BS, u & 3, wgs[r][it]);
              load_w_slice<TS>(up + (size_t)(u >> 2) * BS, u & 3, wus[r][it]);
            }
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        float ag = 0.f, au = 0.f;
#pragma unroll
        for (int it = 0; it < IT1; ++it) {
          const int u = lane + 64 * it;
          if (rv[r] && u < U1) {
            Q8Slice xs;
            const uint8_t *xrow = s_xq + (size_t)tok[r] * q8x;
            if (!shared_row[r]) {
              load_q8_lds_slice<TG>(xrow, a.nbH, u, xs);
              ag += quarter_dot<TG>(wgs[r][it], u & 3, xs, s_grid, s_signs);
              au += quarter_dot<TG>(wus[r][it], u & 3, xs, s_grid, s_signs);
            } else if constexpr (TS != 0) {
              load_q8_lds_slice<TS>(xrow, a.nbH, u, xs);
              ag += quarter_dot<TS>(wgs[r][it], u & 3, xs, s_grid, s_signs);
              au += quarter_dot<TS>(wus[r][it], u & 3, xs, s_grid, s_signs);
            }
          }
        }
        ag = group_sum<64>(ag);
        au = group_sum<64>(au);
        if (lane == 0 && rv[r]) a.act[j0 + (long)r * DEC_WAVES] = silu_f32(ag) * au;
      }
    }
  }
  __threadfence();
  __syncthreads();
  // completion counters of the 256-row act blocks this workgroup touched
  if (tid == 0) s_nquant = 0;
  __syncthreads();
  if (t1 > t0) {
    const long b0 = t0 / QK, b1 = (t1 - 1) / QK;
    if (tid <= b1 - b0 && tid < DEC_MAX_TOUCH) {
      const long b = b0 + tid;
      const long lo = t0 > b * QK ? t0 : b * QK;
      const long hi = t1 < (b + 1) * QK ? t1 : (b + 1) * QK;
      const uint32_t cnt = (uint32_t)(hi - lo);
      const uint32_t old = atomicAdd(&a.sync[4 + b], cnt);
      if (old + cnt == QK) s_quant[atomicAdd(&s_nquant, 1)] = (int)b;
    }
  }
  __syncthreads();
  for (int i = wave; i < s_nquant; i += DEC_WAVES) {
    __threadfence();
    const long b = s_quant[i];
    const float4 v = reinterpret_cast<const float4 *>(a.act + b * QK)[lane];
    const Q8Out o = quant_block_wave(v, lane);
    uint8_t *row;
    int blk, nb;
    if (b < T1r / QK) {
      const int c = (int)(b / a.nbF);
      blk = (int)(b % a.nbF);
      nb = a.nbF;
      row = a.aq + (size_t)c * q8F;
    } else {
      const long bs = b - T1r / QK;
      const int s = (int)(bs / a.nbFs);
      blk = (int)(bs % a.nbFs);
      nb = a.nbFs;
      row = a.aq + (size_t)S * K * q8F + (size_t)s * q8Fs;
    }
    const uint32_t packed = (uint32_t)(uint8_t)o.q[0] | ((uint32_t)(uint8_t)o.q[1] << 8) |
                            ((uint32_t)(uint8_t)o.q[2] << 16) | ((uint32_t)(uint8_t)o.q[3] << 24);
    *reinterpret_cast<uint32_t *>(row + (size_t)blk * QK + 4 * lane) = packed;
    if (lane == 0) reinterpret_cast<float *>(row + q8_d_off(nb))[blk] = o.d;
    if ((lane & 3) == 0) reinterpret_cast<int16_t *>(row + q8_bs_off(nb))[blk * 16 + (lane >> 2)] = (int16_t)o.bsum16;
    __threadfence();
    if (lane == 0) atomicAdd(&a.sync[0], 1u);
  }

  // ---------------------------------------------------------------- P2: down rows
  const long T2 = (long)S * H;
  const long u0 = T2 * g / G, u1 = T2 * (g + 1) / G;
  const int U2 = 4 * a.nbF, U2s = 4 * a.nbFs;
  const int V = K * U2 + (a.Fs > 0 ? U2s : 0);
  constexpr int BD = block_bytes(TD);
  constexpr int BSD = TS ? block_bytes(TS) : 1;

  auto load_row = [&](long j, WSlice (&ws)[IT2]) {
    const int s = (int)(j / H), h = (int)(j % H);
#pragma unroll
    for (int it = 0; it < IT2; ++it) {
      const int v = lane + 64 * it;
      if (v < K * U2) {
        const int k = v / U2, u = v % U2;
        const int e = s_ids[s * K + k];
        if (e >= 0)
          load_w_slice<TD>(a.wd + (size_t)e * a.d_estride + (size_t)h * a.d_rstride + (size_t)(u >> 2) * BD, u & 3,
                           ws[it]);
      } else if constexpr (TS != 0) {
        if (v < V) {
          const int u = v - K * U2;
          load_w_slice<TS>(a.sd + (size_t)h * a.sd_rstride + (size_t)(u >> 2) * BSD, u & 3, ws[it]);
        }
      }
    }
  };

  WSlice cur[IT2];
  long j = u0 + wave;
  if (j < u1) load_row(j, cur);

  // wait for every act block to be quantized
  if (tid == 0) {
    const uint32_t target = (uint32_t)(T1 / QK);
    int spins = 0;
    while (ld_acq(&a.sync[0]) < target) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins > a.spin_limit) {
        atomicOr(&a.sync[2], 1u);
        s_err = 1;
        break;
      }
    }
    __threadfence();
  }
  __syncthreads();
  __threadfence();

  if (!s_err) {
    int cur_s = -1;
    Q8Slice qs[IT2];
    float wr[IT2];
    for (; j < u1; j += DEC_WAVES) {
      WSlice nxt[IT2];
      const long jn = j + DEC_WAVES;
      if (jn < u1) load_row(jn, nxt);
      const int s = (int)(j / H), h = (int)(j % H);
      if (s != cur_s) {
        cur_s = s;
#pragma unroll
        for (int it = 0; it < IT2; ++it) {
          const int v = lane + 64 * it;
          wr[it] = 0.f;
          if (v < K * U2) {
            const int k = v / U2, u = v % U2;
            const int c = s_cidx[s * K + k];
            if (c >= 0) {
              load_q8_slice<TD>(a.aq + (size_t)c * q8F, a.nbF, u >> 2, u & 3, qs[it]);
              wr[it] = s_w[s * K + k];
            }
          } else if constexpr (TS != 0) {
            if (v < V) {
              const int u = v - K * U2;
              load_q8_slice<TS>(a.aq + (size_t)S * K * q8F + (size_t)s * q8Fs, a.nbFs, u >> 2, u & 3, qs[it]);
              wr[it] = 1.0f;
            }
          }
        }
      }
      float acc = 0.f;
#pragma unroll
      for (int it = 0; it < IT2; ++it) {
        const int v = lane + 64 * it;
        if (v < K * U2) {
          const int k = v / U2, u = v % U2;
          if (s_ids[s * K + k] >= 0) acc += wr[it] * quarter_dot<TD>(cur[it], u & 3, qs[it], s_grid, s_signs);
        } else if constexpr (TS != 0) {
          if (v < V) {
            const int u = v - K * U2;
            acc += quarter_dot<TS>(cur[it], u & 3, qs[it], s_grid, s_signs);
          }
        }
      }
      acc = group_sum<64>(acc);
      if (lane == 0) a.out[(size_t)s * H + h] = acc;
#pragma unroll
      for (int it = 0; it < IT2; ++it) cur[it] = nxt[it];
    }
  }

  // ---------------------------------------------------------------- exit: last workgroup resets the counters
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    const uint32_t old = atomicAdd(&a.sync[1], 1u);
    if (old == (uint32_t)G - 1) {
      const long nblk = T1 / QK;
      for (long b = 0; b < nblk; ++b) __hip_atomic_store(&a.sync[4 + b], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.sync[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.sync[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __threadfence();
    }
  }
}

}  // namespace zm
