// zm_mmq.hpp -- bucketed MUL_MAT_ID for prefill-sized buckets on int8 MFMA.
//
// Per active expert, out[pair][row] = W_e[row] . q8(x[pair]) for the pairs of
// the expert's bucket (the CSR of /root/reference/core/batched_dispatch_pipeline.cpp:1181-1202),
// gate/up optionally fused with SwiGLU (moe_routed_ggml.hpp:166-191).
//
// Tile: one wave computes 16 tokens x 16 weight rows with
// v_mfma_i32_16x16x64_i8, tokens as the A operand and weight rows as the B
// operand, so every lane's four outputs belong to ONE weight row (lane % 16)
// and every lane's 16 B-operand bytes to one 32-weight sub-block of that row,
// whose 6-bit scale sc = 8*hi + lo the lane has decoded itself.  The scale is
// folded into the weights: the lane multiplies its nibbles by lo and by hi
// (products <= 105, int8), and two MFMA chains accumulate over the block:
//   isum[t][r] = D_lo + 8 * D_hi = sum_sb sc[r][sb] * (q[r] . x[t])_sb  (int32, exact)
//   mn[t][r]   = sum_sb bsum[t][sb] * (-dmin[r] * m[r][sb])   (v_mfma_f32_16x16x4f32;
//                -dmin * m is exact in fp32, so mn is -dmin * imin to fp32 rounding)
//   f[t][r]   += d_x[t] * (d[r] * isum + mn)  (ggml's vec_dot_q4_K_q8_K combine)
// Q4_K / Q5_K K order of a 64-weight chunk i (qs group i, bytes 32i..32i+31,
// holding sub-block 2i in its low nibbles and 2i + 1 in its high nibbles):
// k-group g holds bytes 8g..8g+7 of the group, low nibbles then high nibbles,
// i.e. weights 64i + 8g .. +7 and 64i + 32 + 8g .. +7, so every qs byte is
// loaded by one lane only (Q5_K: the fifth bits are bits 2i, 2i + 1 of the
// lane's qh bytes 8g..8g+7); the activation operand is read in the same order
// (two 8-byte LDS reads).  The weight unpacking is done once per block for all
// token tiles of the work item.  No dequantized weight copy is materialized.
// Activations reach LDS by direct buffer-to-LDS loads (no register staging),
// token rows XOR-swizzled in 16-byte chunks by the token index.
//
// IQ2_XXS / IQ3_XXS (grid values up to 43 / 62 with per-8-weight signs, and a
// (2 ls + 1) <= 31 scale per 32-weight sub-block) dot each sub-block on its own
// v_mfma_i32_16x16x32_i8 (K = the sub-block; lane group g holds its 8-weight
// group g): signed grid bytes from the LDS-staged grid and sign masks, scales
// per lane on the integer results.
//
// IQ4_XS (a 16-entry value table, up to |127|, and a 6-bit signed scale per
// 32-weight sub-block) dots each 64-weight chunk as its two sub-blocks on
// v_mfma_i32_16x16x64_i8 with half of B zeroed, values looked up from the
// table in registers; the scales apply per lane as for Q6_K, no min term.
//
// Q5_K adds the fifth bit of each value as a third chain: the bit (0/1) times
// the whole 6-bit scale (<= 63) is int8 too, and isum = D_lo + 8 D_hi + 16 D_5.
//
// Q2_K uses v_mfma_i32_16x16x64_i8 with the 4-bit sub-block scale folded into
// the weights (q * sc <= 45 fits int8): lane (row n, k-group g) of 64-weight
// chunk c = 2h + jp holds bit-plane j = 2jp + (g >> 1) of qs bytes
// 32h + 16(g & 1) .. +15, i.e. weights 64c + 16g .. +15 of sub-block
// 8h + 2j + (g & 1), each byte multiplied by that sub-block's scale; one MFMA
// chain over the 4 chunks gives isum = sum_sb sc * (q . x)_sb exactly, the
// mins term sum_sb (-dmin * m) * bsum16 goes through four v_mfma_f32_16x16x4f32
// (K = 16 sub-blocks), and f += d_x * (d * isum + mn) (ggml's vec_dot_q2_K_q8_K).  Activations are the planar Q8_K rows of the decode
// path (qs | bsums | d).
//
// Q6_K (a 6-bit value and a signed 8-bit scale per 16-weight sub-block: the
// product does not fit int8) keeps the scales out of the weights and uses
// v_mfma_i32_16x16x32_i8, whose K = 32 spans two sub-blocks (lane groups 0-1
// and 2-3): each pair of sub-blocks is issued twice with the other half of
// the B operand zeroed, giving one exact 16x16 integer dot per sub-block,
// scaled per lane (a lane's outputs share one weight row) and summed:
//   isum[t][r] = sum_sb sc[r][sb] * (q[r] . x[t])_sb            (q = 0..63)
//   off[t][r]  = sum_sb sc[r][sb] * bsum16[t][sb]               (v_mfma_f32_16x16x4f32, exact)
//   f[t][r]   += d_x[t] * d[r] * (isum - 32 * off)   (the value is q - 32; ggml's vec_dot_q6_K_q8_K)
// Lane (row n, group g) of sub-block pair p holds weights 32p + 8g .. +7:
// low (p & 3 < 2) or high nibbles of ql bytes 64(p >> 2) + 32(p & 1) + 8g .. +7,
// top bits 2(p & 3) of qh bytes 32(p >> 2) + 8g .. +7.
#pragma once

#include "zm_kernels.hpp"

namespace zm {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));
typedef unsigned short v2u16_t __attribute__((ext_vector_type(2)));
typedef short v2i16_t __attribute__((ext_vector_type(2)));
typedef unsigned v4u_t __attribute__((ext_vector_type(4)));

// buffer-to-LDS loads (lane L's `bytes` land at lds + bytes * L; out-of-range
// lanes write zeros) issued as inline asm: the compiler's wait insertion does not
// track them, so the reads of the other LDS buffer are not held behind them.
// The caller waits for them itself (vmcnt(0)) before the barrier that publishes
// the buffer.
__device__ __forceinline__ v4u_t dma_rsrc(const void *p, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return v4u_t{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is written by the asm and by nothing else here
__device__ __forceinline__ void dma_lds16(v4u_t rs, uint32_t lds, int vo) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(vo), "s"(rs)
               : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4(v4u_t rs, uint32_t lds, int vo) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(vo), "s"(rs)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// four packed bytes times a small factor, bytewise (every product < 256: no
// carry crosses a byte): one packed 16-bit multiply
__device__ __forceinline__ uint32_t mul_bytes(uint32_t packed, uint32_t f) {
  const v2u16_t p = __builtin_bit_cast(v2u16_t, packed);
  const v2u16_t m = {(unsigned short)f, (unsigned short)f};
  return __builtin_bit_cast(uint32_t, p * m);
}

constexpr int MMQ_TOK = 32;            // pairs per work item of the 2-tile kernels (item count bound)


// Work items: every active expert's bucket cut into runs of `tok` pairs,
// item = expert | (first pair offset within the bucket) << 12.  One workgroup.
__global__ __launch_bounds__(1024) void k_mmq_items(const int32_t *__restrict__ n_active,
                                                    const int32_t *__restrict__ active,
                                                    const int32_t *__restrict__ offs, int32_t *__restrict__ items,
                                                    int32_t *__restrict__ n_items, int tok) {
  __shared__ int s_n[1024];
  const int na = *n_active;
  int total = 0;
  for (int base = 0; base < na; base += 1024) {
    const int i = base + (int)threadIdx.x;
    const int e = i < na ? active[i] : 0;
    const int np = i < na ? (offs[e + 1] - offs[e] + tok - 1) / tok : 0;
    s_n[threadIdx.x] = np;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {  // inclusive scan
      const int v = threadIdx.x >= (unsigned)d ? s_n[threadIdx.x - d] : 0;
      __syncthreads();
      s_n[threadIdx.x] += v;
      __syncthreads();
    }
    const int start = total + s_n[threadIdx.x] - np;
    for (int q = 0; q < np; ++q) items[start + q] = e | ((q * tok) << 12);
    total += s_n[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) *n_items = total;
}

// The same work items, largest first: full runs of `tok` pairs, then every
// expert's remaining run in descending order of its 16-pair tiles, so the
// short items fill the tail of the launch.  The order of items with the same
// size is not fixed; no result depends on it (every item writes its own pairs).
// Needs n_active <= 1024 and tok <= 256.
__global__ __launch_bounds__(1024) void k_mmq_items_lpt(const int32_t *__restrict__ n_active,
                                                        const int32_t *__restrict__ active,
                                                        const int32_t *__restrict__ offs, int32_t *__restrict__ items,
                                                        int32_t *__restrict__ n_items, int tok) {
  constexpr int NK = 18;  // size classes: 1..16 tiles of a partial run, 17 = full run
  __shared__ int hist[NK], cur[NK];
  const int tid = threadIdx.x;
  if (tid < NK) hist[tid] = 0;
  __syncthreads();
  const int na = *n_active;
  const int tt = tok / 16;
  int e = 0, nfull = 0, rem = 0, key = 0;
  if (tid < na) {
    e = active[tid];
    const int cnt = offs[e + 1] - offs[e];
    nfull = cnt / tok;
    rem = cnt - nfull * tok;
    key = (rem + 15) / 16;  // 0: no partial run
    if (nfull) atomicAdd(&hist[NK - 1], nfull);
    if (key) atomicAdd(&hist[key], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int k = NK - 1; k >= 1; --k) {
      cur[k] = run;
      run += (k == NK - 1 || k <= tt) ? hist[k] : 0;
    }
    *n_items = run;
  }
  __syncthreads();
  if (tid < na) {
    if (nfull) {
      const int p = atomicAdd(&cur[NK - 1], nfull);
      for (int q = 0; q < nfull; ++q) items[p + q] = e | ((q * tok) << 12);
    }
    if (key) items[atomicAdd(&cur[key], 1)] = e | ((nfull * tok) << 12);
  }
}

// One work item (up to 16*TT pairs of one bucket) against 64 weight rows
// (4 waves x 16 rows).  The activation block of the item is staged in LDS
// (double buffered over the K blocks; each thread holds the next block's share
// in registers while the current block computes); the weights of block b+1
// are requested while block b computes.
template <int T>
struct MmqW;
template <>
struct MmqW<T_Q4_K> {  // d, dmin, scales | this lane's 8 bytes of each 32-byte qs group
  uint4 hdr;
  uint2 qs[4];
};
template <>
struct MmqW<T_Q5_K> {  // d, dmin, scales | this lane's 8 bytes of qh and of each 32-byte qs group
  uint4 hdr;
  uint2 qh;
  uint2 qs[4];
};
template <>
struct MmqW<T_Q2_K> {  // scales | this lane's 2 x 16 bytes of qs | d, dmin
  uint4 sc;
  uint4 qs[2];
  uint32_t dd;
};
template <>
struct MmqW<T_IQ2_XXS> {  // d | all 64 bytes of qs (grid-index and sign+scale words per sub-block)
  uint32_t d;
  uint4 q[4];
};
template <>
struct MmqW<T_IQ3_XXS> {  // d | 64 grid-index bytes | 8 scale+sign words
  uint32_t d;
  uint4 gi[4];
  uint4 sas[2];
};
template <>
struct MmqW<T_IQ4_XS> {  // d, scales_h, scales_l | this lane's 16 qs bytes of each chunk
  uint2 hdr;
  uint4 qs[4];
};
template <>
struct MmqW<T_Q6_K> {  // this lane's 4 x 8 bytes of ql, 2 x 8 bytes of qh | scales | d
  uint2 ql[4];
  uint2 qh[2];
  uint4 sc;
  uint32_t d;
};

template <int T, bool GATEUP, int TT, int NW = 4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(T == T_Q4_K && !GATEUP && TT <= 4 && NW == 4 ? 4 : 1))) void k_mmq(GemvArgs a) {
  constexpr int TOK = 16 * TT;  // pairs per work item
  constexpr int NT = 64 * NW;   // threads: NW waves of 16 weight rows each
  static_assert(T == T_Q4_K || T == T_Q5_K || T == T_Q2_K || T == T_Q6_K || T == T_IQ4_XS || T == T_IQ2_XXS ||
                    T == T_IQ3_XXS,
                "MFMA prefill types");
  constexpr bool kGrid = T == T_IQ2_XXS || T == T_IQ3_XXS;
  // the lookup tables first in LDS (largest alignment first), so their
  // addresses fold into the LDS reads' offset field
  __shared__ __attribute__((aligned(kGrid ? 4096 : 8))) uint64_t s_grid[kGrid ? (T == T_IQ2_XXS ? 256 : 128) : 1];  // IQ3_XXS: 256 x u32
  __shared__ __attribute__((aligned(kGrid ? 2048 : 8))) uint64_t s_signs[kGrid ? 128 : 1];
  constexpr bool K45 = T == T_Q4_K || T == T_Q5_K;
  // The activation blocks reach LDS by direct buffer-to-LDS loads (no register
  // staging); a token's row is 256 bytes with its 16-byte chunks XOR-swizzled
  // by the token index (chunk c of token t at c ^ (t & 15)), so the 16 tokens
  // of an MFMA A operand read 16 different bank groups; the raw int16 16-sums
  // are kept (and added pairwise where 32-sums are used)
  __shared__ __attribute__((aligned(16))) uint8_t s_xq[2][TOK][QK];
  __shared__ __attribute__((aligned(16))) int16_t s_bs16[2][TOK][16];
  __shared__ __attribute__((aligned(16))) float s_xd[2][TOK];
  __shared__ int s_xoff[TOK];      // byte offset of each pair's activation row (OOR: none)
  __shared__ int s_pair[TOK];
  int e, pc, p1;
  if (a.dense_S > 0) {
    e = 0;
    pc = blockIdx.y * TOK;
    p1 = a.dense_S;
    if (pc >= p1) return;
  } else {
    if ((int)blockIdx.y >= *a.n_items) return;
    const int it = a.items[blockIdx.y];
    e = it & 0xfff;
    pc = a.offs[e] + (it >> 12);
    p1 = a.offs[e + 1];
  }
  constexpr int NM = GATEUP ? 2 : 1;
  constexpr int BB = block_bytes(T);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row = blockIdx.x * (16 * NW) + wave * 16 + n;  // weight row of this lane (B operand, output column)
  const bool rv = row < a.nrows;
  const uint32_t wbytes = (uint32_t)((size_t)a.nrows * a.w_rstride);
  rsrc_t rw[NM];
  rw[0] = make_rsrc(a.w0 + (size_t)e * a.w_estride, wbytes);
  if constexpr (GATEUP) rw[1] = make_rsrc(a.w1 + (size_t)e * a.w_estride, wbytes);
  const v4u_t rxd = dma_rsrc(a.xq, a.xq_bytes);
  const int vrow = rv ? row * (int)a.w_rstride : OOR;
  const int Kp = a.dense_S > 0 ? 1 : a.K;
  const int nb = a.nb;
  const int nt = min(TT, (p1 - pc + 15) / 16);
  uint32_t tab[4] = {0, 0, 0, 0};  // IQ4_XS value table (a.grid), wave-uniform
  if constexpr (T == T_IQ4_XS) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      tab[2 * i] = (uint32_t)a.grid[i];
      tab[2 * i + 1] = (uint32_t)(a.grid[i] >> 32);
    }
  }

  if constexpr (kGrid) {
    for (int i = tid; i < (T == T_IQ2_XXS ? 256 : 128); i += NT) s_grid[i] = a.grid[i];
    if (tid < 128) s_signs[tid] = a.signs[tid];
  }
  if (tid < TOK) {
    const int p = pc + tid;
    const bool ok = p < p1;
    const int pair = ok ? (a.dense_S > 0 ? p : a.pairs[p]) : -1;
    s_pair[tid] = pair;
    s_xoff[tid] = ok ? (int)(((pair / Kp) * a.ne11 + (pair % Kp) % a.ne11) * a.xq_rstride) : OOR;
  }
  __syncthreads();

  using WBlk = MmqW<T>;
  auto load_w = [&](int b, WBlk (&w)[NM]) {
    const int vo = b < nb ? vrow + b * BB : OOR;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      if constexpr (T == T_Q4_K) {
        w[m].hdr = bld16(rw[m], vo, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[m].qs[i] = bld8(rw[m], vo + 16 + 32 * i + 8 * g, 0);
      } else if constexpr (T == T_Q5_K) {
        w[m].hdr = bld16(rw[m], vo, 0);
        w[m].qh = bld8(rw[m], vo + 16 + 8 * g, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[m].qs[i] = bld8(rw[m], vo + 48 + 32 * i + 8 * g, 0);
      } else if constexpr (T == T_IQ2_XXS) {
        w[m].d = bld2(rw[m], vo, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[m].q[i] = bld16(rw[m], vo + 2 + 16 * i, 0);
      } else if constexpr (T == T_IQ3_XXS) {
        w[m].d = bld2(rw[m], vo, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[m].gi[i] = bld16(rw[m], vo + 2 + 16 * i, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) w[m].sas[i] = bld16(rw[m], vo + 66 + 16 * i, 0);
      } else if constexpr (T == T_IQ4_XS) {
        w[m].hdr = bld8(rw[m], vo, 0);
#pragma unroll
        for (int c = 0; c < 4; ++c) w[m].qs[c] = bld16(rw[m], vo + 8 + 32 * c + 16 * (g >> 1), 0);
      } else if constexpr (T == T_Q6_K) {
#pragma unroll
        for (int i = 0; i < 4; ++i) w[m].ql[i] = bld8(rw[m], vo + 64 * (i >> 1) + 32 * (i & 1) + 8 * g, 0);
#pragma unroll
        for (int h = 0; h < 2; ++h) w[m].qh[h] = bld8(rw[m], vo + 128 + 32 * h + 8 * g, 0);
        w[m].sc = bld16(rw[m], vo + 192, 0);
        w[m].d = bld2(rw[m], vo + 208, 0);
      } else {
        w[m].sc = bld16(rw[m], vo, 0);
#pragma unroll
        for (int h = 0; h < 2; ++h) w[m].qs[h] = bld16(rw[m], vo + 16 + 32 * h + 16 * (g & 1), 0);
        w[m].dd = bld4(rw[m], vo + 80, 0);
      }
    }
  };
  // direct loads of block b's activations into buffer buf: the qs of
  // TOK tokens (1 KB = 4 tokens per wave instruction), their 16 bsums (32 B per
  // token) and d; out-of-range lanes write zeros
  auto dma_x = [&](int b, int buf) {
    {
      const bool bv = b < nb;
      constexpr int QI = TOK / 4 / NW;  // qs instructions per wave
      static_assert(TOK % (4 * NW) == 0, "qs instructions per wave");
#pragma unroll
      for (int i = 0; i < QI; ++i) {
        const int t0 = 4 * (QI * wave + i);
        const int t = t0 + (lane >> 4), c = (lane & 15) ^ (t & 15);
        const int o = s_xoff[t];
        dma_lds16(rxd, lds_addr(&s_xq[buf][t0][0]), (bv && o != OOR) ? o + b * QK + 16 * c : OOR);
      }
      for (int i = wave; 32 * i < TOK; i += NW) {  // bsums: 2 lanes per token
        const int t = 32 * i + (lane >> 1);
        if (t >= TOK) break;  // lanes past the tile write nothing
        const int o = s_xoff[t];
        dma_lds16(rxd, lds_addr(&s_bs16[buf][32 * i][0]),
                  (bv && o != OOR) ? o + (int)q8_bs_off(nb) + b * 32 + 16 * (lane & 1) : OOR);
      }
      for (int i = wave; 64 * i < TOK; i += NW) {  // d: one float per token
        const int t = 64 * i + lane;
        if (t >= TOK) break;
        const int o = s_xoff[t];
        dma_lds4(rxd, lds_addr(&s_xd[buf][64 * i]), (bv && o != OOR) ? o + (int)q8_d_off(nb) + 4 * b : OOR);
      }
    }
  };

  // reads of the staged activations: logical 16-byte chunk c (or its 8-byte
  // half h) of token tok, and its raw 16-sum j / 32-sum j (16-sums 2j, 2j + 1)
  auto xq16 = [&](int buf, int tok, int c) {
    return *reinterpret_cast<const v4i_t *>(&s_xq[buf][tok][16 * (c ^ (tok & 15))]);
  };
  auto xq8 = [&](int buf, int tok, int c, int h) {
    return *reinterpret_cast<const uint2 *>(&s_xq[buf][tok][16 * (c ^ (tok & 15)) + 8 * h]);
  };
  auto bsum16 = [&](int buf, int tok, int j) { return (int)s_bs16[buf][tok][j]; };
  auto bsum32 = [&](int buf, int tok, int j) {
    const int w = reinterpret_cast<const int *>(&s_bs16[buf][tok][0])[j];
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2i16_t, w), v2i16_t{1, 1}, 0, false);
  };

  // per (matrix, token tile, output): f += d_x * (d * isum + mn), as
  // two fmas (the tile epilogue is most of the per-tile VALU work)
  float f[NM][TT][4];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) f[m][t][j] = 0.f;

  // one block of the K loop from the weights in wcur and activation buffer buf
  auto step = [&](int buf, const WBlk(&wcur)[NM]) {
    if constexpr (K45) {
      // both matrices' operands first, then one pass over the token tiles: the
      // activation operand (and the bsums of the min product) is read from LDS
      // once per tile for gate and up together
      constexpr int N5 = T == T_Q5_K ? 4 : 1;
      v4i_t bl[NM][4], bh[NM][4], b5[NM][N5];
      float dd[NM], dm[NM], mb0[NM], mb1[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        const uint32_t u0 = wcur[m].hdr.y, u1 = wcur[m].hdr.z, u2 = wcur[m].hdr.w;
        const uint32_t sc_lo = u0 & 0x3f3f3f3fu, mn_lo = u1 & 0x3f3f3f3fu;
        const uint32_t sc_hi = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn_hi = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
        dd[m] = h2f((uint16_t)(wcur[m].hdr.x & 0xffffu));
        dm[m] = h2f((uint16_t)(wcur[m].hdr.x >> 16));
        // B operand of the min product: m[row][sb] for sb = g and g + 4
        // with -dmin folded in (exact: an f16 times a 6-bit integer), so the
        // product comes out as the whole min term
        mb0[m] = -dm[m] * (float)((mn_lo >> (8 * g)) & 0xffu);
        mb1[m] = -dm[m] * (float)((mn_hi >> (8 * g)) & 0xffu);
        // scale-folded weights of the 4 chunks: lane's sub-block 2i + (g >> 1),
        // sc = 8 * hi + lo; Q5_K: the fifth bit (bit 2i + (g >> 1) of the lane's
        // qh bytes) is a third chain with the whole scale, isum = D_lo + 8 D_hi + 16 D_5
        {
          // chunk i = qs group i (sub-blocks 2i, 2i + 1): the lane's 8 bytes
          // 8g .. 8g + 7 give 8 weights of each sub-block, low nibbles then
          // high nibbles (the activation operand is read in the same order);
          // Q5_K: their fifth bits are bits 2i, 2i + 1 of the lane's 8 qh bytes
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t scw = (i < 2 ? sc_lo : sc_hi) >> (16 * (i & 1));
            const uint32_t s0 = scw & 0xffu, s1 = (scw >> 8) & 0xffu;
            const uint2 q = wcur[m].qs[i];
            const uint32_t n0 = q.x & 0x0f0f0f0fu, n1 = q.y & 0x0f0f0f0fu;
            const uint32_t n2 = (q.x >> 4) & 0x0f0f0f0fu, n3 = (q.y >> 4) & 0x0f0f0f0fu;
            bl[m][i] = v4i_t{(int)mul_bytes(n0, s0 & 7u), (int)mul_bytes(n1, s0 & 7u), (int)mul_bytes(n2, s1 & 7u),
                             (int)mul_bytes(n3, s1 & 7u)};
            bh[m][i] = v4i_t{(int)mul_bytes(n0, s0 >> 3), (int)mul_bytes(n1, s0 >> 3), (int)mul_bytes(n2, s1 >> 3),
                             (int)mul_bytes(n3, s1 >> 3)};
            if constexpr (T == T_Q5_K) {
              const uint2 h = wcur[m].qh;
              b5[m][i] = v4i_t{(int)mul_bytes((h.x >> (2 * i)) & 0x01010101u, s0),
                               (int)mul_bytes((h.y >> (2 * i)) & 0x01010101u, s0),
                               (int)mul_bytes((h.x >> (2 * i + 1)) & 0x01010101u, s1),
                               (int)mul_bytes((h.y >> (2 * i + 1)) & 0x01010101u, s1)};
            }
          }
        }
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= nt) continue;
        const int tok = 16 * t + n;
        v4i_t xa[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // activations 64i + 8g .. +7 and 64i + 32 + 8g .. +7 (logical 16-byte
          // chunks 4i + g/2 and 4i + 2 + g/2, half g & 1)
          const uint2 lo8 = xq8(buf, tok, 4 * i + (g >> 1), g & 1);
          const uint2 hi8 = xq8(buf, tok, 4 * i + 2 + (g >> 1), g & 1);
          xa[i] = v4i_t{(int)lo8.x, (int)lo8.y, (int)hi8.x, (int)hi8.y};
        }
        // 32-sums of sub-blocks g and g + 4
        const float bs0 = (float)bsum32(buf, tok, g), bs1 = (float)bsum32(buf, tok, g + 4);
        float xdj[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) xdj[j] = s_xd[buf][16 * t + 4 * g + j];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          v4i_t dlo = {0, 0, 0, 0}, dhi = {0, 0, 0, 0}, d5 = {0, 0, 0, 0};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dlo = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i], bl[m][i], dlo, 0, 0, 0);
            dhi = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i], bh[m][i], dhi, 0, 0, 0);
            if constexpr (T == T_Q5_K) d5 = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i], b5[m][i], d5, 0, 0, 0);
          }
          v4f_t mn = {0.f, 0.f, 0.f, 0.f};
          mn = __builtin_amdgcn_mfma_f32_16x16x4f32(bs0, mb0[m], mn, 0, 0, 0);
          mn = __builtin_amdgcn_mfma_f32_16x16x4f32(bs1, mb1[m], mn, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            f[m][t][j] = __builtin_fmaf(xdj[j], __builtin_fmaf(dd[m], (float)(dlo[j] + 8 * dhi[j] + 16 * d5[j]), mn[j]), f[m][t][j]);
        }
      }
    } else if constexpr (kGrid) {
      // one v_mfma_i32_16x16x32_i8 per 32-weight sub-block (K = the sub-block):
      // lane group g holds 8-weight group l = g of every sub-block, grid values
      // with their signs applied (conditional byte negate); the scale (2 ls + 1)
      // multiplies the sub-block's integer dot per lane, the 1/8 (IQ2_XXS) or
      // 1/4 (IQ3_XXS) is folded into d
      long B[NM][8];
      int S[NM][8];
      float DD[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        constexpr float kf = T == T_IQ2_XXS ? 0.125f : 0.25f;
        DD[m] = kf * h2f((uint16_t)(wcur[m].d & 0xffffu));
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) {
          uint32_t glo, ghi, aux;
          if constexpr (T == T_IQ2_XXS) {
            // sub-block sb: words 2sb (grid indices), 2sb + 1 (signs, scale)
            const uint32_t aux0 = u4_get(wcur[m].q[sb >> 1], 2 * (sb & 1));
            aux = u4_get(wcur[m].q[sb >> 1], 2 * (sb & 1) + 1);
            const uint64_t gg = s_grid[(aux0 >> (8 * g)) & 0xffu];
            glo = (uint32_t)gg;
            ghi = (uint32_t)(gg >> 32);
          } else {
            // sub-block sb: grid-index bytes 8sb + 2g, +1 (two 4-value entries), word sb
            const uint32_t iw = u4_get(wcur[m].gi[sb >> 1], 2 * (sb & 1) + (g >> 1));
            aux = u4_get(wcur[m].sas[sb >> 2], sb & 3);
            const uint32_t *g3 = reinterpret_cast<const uint32_t *>(s_grid);
            glo = g3[(iw >> (16 * (g & 1))) & 0xffu];
            ghi = g3[(iw >> (16 * (g & 1) + 8)) & 0xffu];
          }
          const uint64_t mm = s_signs[(aux >> (7 * g)) & 127u];
          const uint32_t mlo = (uint32_t)mm, mhi = (uint32_t)(mm >> 32);
          const uint32_t v0 = sign_bytes(glo, mlo), v1 = sign_bytes(ghi, mhi);
          B[m][sb] = (long)(((uint64_t)v1 << 32) | v0);
          S[m][sb] = 2 * (int)(aux >> 28) + 1;
        }
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= nt) continue;
        const int tok = 16 * t + n;
        float xdj[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) xdj[j] = s_xd[buf][16 * t + 4 * g + j];
        long xa[8];
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) xa[sb] = __builtin_bit_cast(long, xq8(buf, tok, 2 * sb + (g >> 1), g & 1));
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          int isum[4] = {0, 0, 0, 0};
#pragma unroll
          for (int sb = 0; sb < 8; ++sb) {
            const v4i_t z = {0, 0, 0, 0};
            const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa[sb], B[m][sb], z, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) isum[j] = __mul24(S[m][sb], d[j]) + isum[j];
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) f[m][t][j] = __builtin_fmaf(xdj[j], DD[m] * (float)isum[j], f[m][t][j]);
        }
      }
    } else if constexpr (T == T_IQ4_XS) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const float d = h2f((uint16_t)(wcur[m].hdr.x & 0xffffu));
      // chunk c = sub-blocks 2c (lane groups 0-1) and 2c + 1 (groups 2-3); group
      // g takes the low (g even) or high nibbles of its sub-block's 16 qs bytes,
      // through the value table; each chunk is issued twice, the other
      // sub-block's half of B zeroed
      const uint32_t keep0 = g < 2 ? 0xffffffffu : 0u;
      const int ns = 4 * (g & 1);
      v4i_t b0[4], b1[4];
      int s0[4], s1[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 q = wcur[m].qs[c];
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t v = lut16((qw[k] >> ns) & 0x0f0f0f0fu, tab[0], tab[1], tab[2], tab[3]);
          b0[c][k] = (int)(v & keep0);
          b1[c][k] = (int)(v & ~keep0);
        }
        s0[c] = iq4_scale(wcur[m].hdr.x, wcur[m].hdr.y, 2 * c);
        s1[c] = iq4_scale(wcur[m].hdr.x, wcur[m].hdr.y, 2 * c + 1);
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= nt) continue;
        const int tok = 16 * t + n;
        int isum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const v4i_t xa = xq16(buf, tok, 4 * c + g);
          const v4i_t z = {0, 0, 0, 0};
          const v4i_t d0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, b0[c], z, 0, 0, 0);
          const v4i_t d1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa, b1[c], z, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) isum[j] = __mul24(s0[c], d0[j]) + __mul24(s1[c], d1[j]) + isum[j];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) f[m][t][j] = __builtin_fmaf(s_xd[buf][16 * t + 4 * g + j], d * (float)isum[j], f[m][t][j]);
      }
    }
    } else if constexpr (T == T_Q6_K) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const float d = h2f((uint16_t)(wcur[m].d & 0xffffu));
      const uint32_t scb[4] = {wcur[m].sc.x, wcur[m].sc.y, wcur[m].sc.z, wcur[m].sc.w};
      // B operand of the offset product: sc[row][sb] for sb = 4i + g
      float mb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) mb[i] = (float)(int)(int8_t)(scb[i] >> (8 * g));
      // 6-bit values of the 8 sub-block pairs, each issued with the lane's half
      // (groups 0-1: sub-block 2p, groups 2-3: 2p + 1) and zeros in the other
      const uint32_t keep0 = g < 2 ? 0xffffffffu : 0u;
      long b0[8], b1[8];
      int s0[8], s1[8];
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int h = p >> 2, G = p & 3;
        const uint2 q = wcur[m].ql[2 * h + (p & 1)];
        const uint2 hb = wcur[m].qh[h];
        const uint32_t lx = G < 2 ? (q.x & 0x0f0f0f0fu) : ((q.x >> 4) & 0x0f0f0f0fu);
        const uint32_t ly = G < 2 ? (q.y & 0x0f0f0f0fu) : ((q.y >> 4) & 0x0f0f0f0fu);
        const uint32_t vx = lx | (((hb.x >> (2 * G)) & 0x03030303u) << 4);
        const uint32_t vy = ly | (((hb.y >> (2 * G)) & 0x03030303u) << 4);
        b0[p] = (long)(((uint64_t)(vy & keep0) << 32) | (vx & keep0));
        b1[p] = (long)(((uint64_t)(vy & ~keep0) << 32) | (vx & ~keep0));
        s0[p] = (int)(int8_t)(scb[p >> 1] >> (16 * (p & 1)));
        s1[p] = (int)(int8_t)(scb[p >> 1] >> (16 * (p & 1) + 8));
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= nt) continue;
        const int tok = 16 * t + n;
        int isum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const long xa = __builtin_bit_cast(long, xq8(buf, tok, 2 * p + (g >> 1), g & 1));
          const v4i_t z = {0, 0, 0, 0};
          const v4i_t d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, b0[p], z, 0, 0, 0);
          const v4i_t d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xa, b1[p], z, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) isum[j] = __mul24(s0[p], d0[j]) + __mul24(s1[p], d1[j]) + isum[j];
        }
        v4f_t off = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          off = __builtin_amdgcn_mfma_f32_16x16x4f32((float)bsum16(buf, tok, 4 * i + g), mb[i], off, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          f[m][t][j] = __builtin_fmaf(s_xd[buf][16 * t + 4 * g + j], d * (float)(isum[j] - 32 * (int)off[j]), f[m][t][j]);
      }
    }
    } else {
      // Q2_K: both matrices' operands first, then one pass over the token tiles
      // (the activation tile and its bsums read once for gate and up)
      v4i_t bq[NM][4];
      float dd[NM], dm[NM], mb[NM][4];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        dd[m] = h2f((uint16_t)(wcur[m].dd & 0xffffu));
        dm[m] = h2f((uint16_t)(wcur[m].dd >> 16));
        const uint32_t scb[4] = {wcur[m].sc.x, wcur[m].sc.y, wcur[m].sc.z, wcur[m].sc.w};
        // B operand of the min product: m[row][sb] for sb = 4i + g
#pragma unroll
        for (int i = 0; i < 4; ++i) mb[m][i] = -dm[m] * (float)((scb[i] >> (8 * g + 4)) & 15u);  // -dmin folded in (exact)
        // scale-folded weights of the 4 chunks c = 2h + jp: plane j = 2jp + (g >> 1),
        // sub-block 8h + 2j + (g & 1)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int h = c >> 1, jp = c & 1;
          const int j = 2 * jp + (g >> 1);
          const int sb = 8 * h + 2 * j + (g & 1);
          const uint32_t sc = (scb[sb >> 2] >> (8 * (sb & 3))) & 15u;
          const uint4 q = wcur[m].qs[h];
          const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) bq[m][c][k] = (int)mul_bytes((qw[k] >> (2 * j)) & 0x03030303u, sc);
        }
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (t >= nt) continue;
        const int tok = 16 * t + n;
        v4i_t xa[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) xa[c] = xq16(buf, tok, 4 * c + g);
        float bs[4], xdj[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) bs[i] = (float)bsum16(buf, tok, 4 * i + g);
#pragma unroll
        for (int j = 0; j < 4; ++j) xdj[j] = s_xd[buf][16 * t + 4 * g + j];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          v4i_t isum = {0, 0, 0, 0};
#pragma unroll
          for (int c = 0; c < 4; ++c) isum = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[c], bq[m][c], isum, 0, 0, 0);
          v4f_t mn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; ++i) mn = __builtin_amdgcn_mfma_f32_16x16x4f32(bs[i], mb[m][i], mn, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            f[m][t][j] = __builtin_fmaf(xdj[j], __builtin_fmaf(dd[m], (float)isum[j], mn[j]), f[m][t][j]);
        }
      }
    }
  };
  // one block ahead: each step issues block b + 1's activations and weights and
  // waits for all of it at its end.  The loop is unrolled by two, so the two
  // weight register sets and activation buffers alternate without copies.
  WBlk w0[NM], w1[NM];
  load_w(0, w0);
  dma_x(0, 0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct loads have landed
  __syncthreads();
  for (int b = 0;; b += 2) {
    dma_x(b + 1, 1);  // buffer 1's readers finished at the last barrier
    load_w(b + 1, w1);
    step(0, w0);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (b + 1 >= nb) break;
    dma_x(b + 2, 0);
    load_w(b + 2, w0);
    step(1, w1);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (b + 2 >= nb) break;
  }
  // lane holds (pair pc + 16t + 4g + j, row): store out[tok][k][row]
  if (rv) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (t >= nt) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pair = s_pair[16 * t + 4 * g + j];
        if (pair < 0) continue;
        const int tok = pair / Kp, k = pair % Kp;
        const float v = GATEUP ? silu_f32(f[0][t][j]) * f[NM - 1][t][j] : f[0][t][j];
        a.out[(size_t)tok * a.out_s + (size_t)k * a.out_k + row] = v;
      }
    }
  }
}

}  // namespace zm
