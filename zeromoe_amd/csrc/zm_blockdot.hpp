// zm_blockdot.hpp -- whole-super-block int8 dots for the fused decode kernel.
//
// One lane holds one "unit" of a weight row in registers: a whole super-block
// (Q2_K, IQ2_XXS) or half of one (Q3_K, Q4_K, Q5_K, Q6_K, IQ3_XXS, IQ4_XS; the
// IQ2_XXS half is used for down rows), and reads the matching Q8_K
// block of the activation row from LDS (planar layout: qs | bsums | d).  A
// unit's integer dot is the ggml per-block integer sum (kquant layouts of
// /root/reference/kernels/quant/kquant_matmul.cu:35-200, iq2_matmul.cu:27-91);
// the float combine is d_x * (d * isum - dmin * imin) as in ggml's
// vec_dot_*_q8_K.  Several weight units (gate and up) share one pass over the
// activation, and per-sub-block scales are applied once per 16 or 32 weights,
// so the VALU cost is close to one mask and one v_dot4 per 4 weights.
//
// Bit-plane trick (Q2_K, Q3_K): the 2-bit value of plane j is masked in place
// (x & (3 << 2j) per byte), so v_dot4 yields 4^j times the plane's dot; the
// sums are kept per plane and shifted back exactly at the end.  v_dot4 reads
// signed bytes, so a field in bit 7 is first moved down (plane 3 is used as
// (x >> 2) & 0x30, scale 16); Q3_K's high bit joins its plane as the bit above.
#pragma once

#include "zm_device.hpp"

namespace zm {

template <int T>
__host__ __device__ constexpr int unit_per_block() {
  return T == T_Q3_K || T == T_Q4_K || T == T_Q5_K || T == T_Q6_K || T == T_IQ4_XS || T == T_IQ3_XXS ? 2 : 1;
}

// types with a whole-block unit (the fused decode kernel's dot)
template <int T>
__host__ __device__ constexpr bool has_unit() {
  return T == T_Q2_K || T == T_Q3_K || T == T_Q4_K || T == T_Q5_K || T == T_Q6_K || T == T_IQ2_XXS ||
         T == T_IQ3_XXS || T == T_IQ4_XS;
}

template <int T>
struct Unit;
template <>
struct Unit<T_Q2_K> {  // scales[16] | qs[64] | d, dmin
  uint4 sc;
  uint4 q[4];
  uint32_t dd;
};
template <>
struct Unit<T_Q3_K> {  // half h: all of hmask[32] | qs[32h, +32) | scales[12] | d
  uint4 hm[2];
  uint4 q[2];
  uint32_t sc[3];
  uint32_t d;
};
template <>
struct Unit<T_Q4_K> {  // d, dmin, scales[12] | half of qs[128]
  uint4 hdr;
  uint4 q[4];
};
template <>
struct Unit<T_Q5_K> {  // d, dmin, scales[12] | all of qh[32] | half of qs[128]
  uint4 hdr;
  uint4 qh[2];
  uint4 q[4];
};
template <>
struct Unit<T_Q6_K> {  // half h: ql[64h, +64) | qh[32h, +32) | scales[8h, +8) | d
  uint32_t ql[16];
  uint32_t qh[8];
  uint32_t sc[2];
  uint32_t d;
};
template <>
struct Unit<T_IQ3_XXS> {  // d | half of the grid indices (4 sub-blocks) | their scale+sign words
  uint32_t d;
  uint32_t gi[8];
  uint4 sas;
};
template <>
struct Unit<T_IQ4_XS> {  // d, scales_h, scales_l | half of qs[128] (4 sub-blocks)
  uint2 hdr;
  uint4 q[4];
};
template <>
struct Unit<T_IQ2_XXS> {  // d | qs u16[32]
  uint32_t d;
  uint4 q[4];
};

// N dwords from byte offset vo (vo even): dword-aligned loads shifted into
// place, since 16-byte loads that are not dword aligned stream ~35% slower.
// The extra dword read past the N (only when vo is not dword aligned) must lie
// inside the resource: callers keep at least 2 more bytes of the block after
// the region.
template <int N>
__device__ __forceinline__ void load_dwords_shifted(rsrc_t r, int vo, uint32_t (&o)[N]) {
  const int sh = vo & 3, base = vo - sh;
  uint32_t w[N + 1];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    const uint4 v = bld16(r, base + 16 * i, 0);
    w[4 * i] = v.x;
    w[4 * i + 1] = v.y;
    w[4 * i + 2] = v.z;
    w[4 * i + 3] = v.w;
  }
#pragma unroll
  for (int i = 4 * (N / 4); i < N; ++i) w[i] = bld4(r, base + 4 * i, 0);
  w[N] = bld4(r, sh ? base + 4 * N : OOR, 0);
#pragma unroll
  for (int k = 0; k < N; ++k) o[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], (uint32_t)sh);
}

// vo: byte offset of the super-block in the resource (an out-of-range offset
// loads zeros); part: which half for Q4_K, Q5_K and Q6_K
template <int T>
__device__ __forceinline__ void load_unit(rsrc_t r, int vo, int part, Unit<T> &u) {
  if constexpr (T == T_Q2_K) {
    u.sc = bld16(r, vo, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) u.q[i] = bld16(r, vo + 16 + 16 * i, 0);
    u.dd = bld4(r, vo + 80, 0);
  } else if constexpr (T == T_Q3_K) {
    // 110-byte blocks start 2 bytes off a dword every other block, and 16-byte
    // loads that are not dword aligned stream ~35% slower: each region (hmask,
    // the half's qs, scales) is loaded dword-aligned with one dword more and
    // shifted into place
    const int sh = vo & 3, base = vo - sh;
    auto region8 = [&](int off, uint4 &a, uint4 &b) {  // 8 dwords at vo + off
      const uint4 v0 = bld16(r, base + off, 0), v1 = bld16(r, base + off + 16, 0);
      const uint32_t v2 = bld4(r, sh ? base + off + 32 : OOR, 0);  // inside the block when shifted
      const uint32_t w[9] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2};
      uint32_t o[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], (uint32_t)sh);
      a = make_uint4(o[0], o[1], o[2], o[3]);
      b = make_uint4(o[4], o[5], o[6], o[7]);
    };
    region8(0, u.hm[0], u.hm[1]);
    region8(32 + 32 * part, u.q[0], u.q[1]);
    const auto sv = __builtin_amdgcn_raw_buffer_load_b96(r, base + 96, 0, 0);
    const uint32_t s3 = bld4(r, sh ? base + 108 : OOR, 0);
    u.sc[0] = __builtin_amdgcn_alignbyte(sv[1], sv[0], (uint32_t)sh);
    u.sc[1] = __builtin_amdgcn_alignbyte(sv[2], sv[1], (uint32_t)sh);
    u.sc[2] = __builtin_amdgcn_alignbyte(s3, sv[2], (uint32_t)sh);
    u.d = bld2(r, vo + 108, 0);
  } else if constexpr (T == T_Q4_K) {
    u.hdr = bld16(r, vo, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) u.q[i] = bld16(r, vo + 16 + 64 * part + 16 * i, 0);
  } else if constexpr (T == T_Q5_K) {  // 176-byte blocks stay 16-byte aligned
    u.hdr = bld16(r, vo, 0);
    u.qh[0] = bld16(r, vo + 16, 0);
    u.qh[1] = bld16(r, vo + 32, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) u.q[i] = bld16(r, vo + 48 + 64 * part + 16 * i, 0);
  } else if constexpr (T == T_IQ3_XXS) {  // 98-byte blocks: the index region is loaded dword-aligned
    u.d = bld2(r, vo, 0);
    load_dwords_shifted<8>(r, vo + 2 + 32 * part, u.gi);
    u.sas = bld16(r, vo + 66 + 16 * part, 0);  // ends the block: no shifted over-read past it
  } else if constexpr (T == T_IQ4_XS) {  // 136-byte blocks stay 8-byte aligned
    u.hdr = bld8(r, vo, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) u.q[i] = bld16(r, vo + 8 + 64 * part + 16 * i, 0);
  } else if constexpr (T == T_Q6_K) {  // 210-byte blocks: every other one starts 2 bytes off a dword
    load_dwords_shifted<16>(r, vo + 64 * part, u.ql);
    load_dwords_shifted<8>(r, vo + 128 + 32 * part, u.qh);
    load_dwords_shifted<2>(r, vo + 192 + 8 * part, u.sc);
    u.d = bld2(r, vo + 208, 0);
  } else {
    u.d = bld2(r, vo, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) u.q[i] = bld16(r, vo + 2 + 16 * i, 0);
  }
}

// half `part` of an IQ2_XXS block (d, sub-blocks 4 part .. 4 part + 3) into q[0..1]
__device__ __forceinline__ void load_unit_half(rsrc_t r, int vo, int part, Unit<T_IQ2_XXS> &u) {
  u.d = bld2(r, vo, 0);
  u.q[0] = bld16(r, vo + 2 + 32 * part, 0);
  u.q[1] = bld16(r, vo + 18 + 32 * part, 0);
  u.q[2] = make_uint4(0u, 0u, 0u, 0u);
  u.q[3] = make_uint4(0u, 0u, 0u, 0u);
}

__device__ __forceinline__ uint32_t u4c(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}
__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b, int c) {
  typedef short short2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2_t, a), __builtin_bit_cast(short2_t, b), c, false);
}
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

// Activation rows in LDS: qs blocks at a 272-byte stride (so the 16 lanes of
// a row, one block each, read 16 different bank groups instead of one), then
// bsums (16 int16 per block), then d (f32 per block); rows padded to 16 bytes.
constexpr int Q8L_BLK = 272;
__host__ __device__ constexpr size_t q8l_row_bytes(int nb) { return ((size_t)nb * (Q8L_BLK + 36) + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t q8l_bs_off(int nb) { return (size_t)nb * Q8L_BLK; }
__host__ __device__ constexpr size_t q8l_d_off(int nb) { return (size_t)nb * (Q8L_BLK + 32); }

// One activation block: qs (256 int8), bsums (16 int16), d.
struct XBlk {
  const uint4 *q;   // 16 x uint4
  const uint4 *bs;  // 2 x uint4
  float d;
};
// block of an LDS activation row
__device__ __forceinline__ XBlk xblk(const uint8_t *row, int nb, int blk) {
  XBlk x;
  x.q = reinterpret_cast<const uint4 *>(row + (size_t)blk * Q8L_BLK);
  x.bs = reinterpret_cast<const uint4 *>(row + q8l_bs_off(nb) + (size_t)blk * 32);
  x.d = reinterpret_cast<const float *>(row + q8l_d_off(nb))[blk];
  return x;
}
// block of a planar row in global memory (q8_row_bytes layout)
__device__ __forceinline__ XBlk xblk_planar(const uint8_t *row, int nb, int blk) {
  XBlk x;
  x.q = reinterpret_cast<const uint4 *>(row + (size_t)blk * QK);
  x.bs = reinterpret_cast<const uint4 *>(row + q8_bs_off(nb) + (size_t)blk * 32);
  x.d = reinterpret_cast<const float *>(row + q8_d_off(nb))[blk];
  return x;
}

// Integer parts of weight unit w[n] against activation block x, as ggml's
// per-block sums: Q2_K/Q4_K isum = sum sc*dot, imin = sum m*bsum; Q3_K isum
// with q3 = q2 - 4*(bit clear), imin = 0; IQ2_XXS isum = sum (2ls+1)*dot.
// HALF (IQ2_XXS only): w holds half `part` of the block (sub-blocks 4 part ..
// 4 part + 3 in q[0..1]), as the down rows of the fused decode kernel use it
template <int T, int NW, bool HALF = false>
__device__ __forceinline__ void unit_ints(const Unit<T> (&w)[NW], int part, const XBlk &x, const uint64_t *lds_grid,
                                          const uint64_t *lds_signs, int (&ri)[NW], int (&rm)[NW]) {
  if constexpr (T == T_Q2_K) {
    // qs dword 8h+k holds plane j = weights 128h + 32j + 4k..+3 (sub-block 8h + 2j + k/4)
    int acc[NW][4];
#pragma unroll
    for (int n = 0; n < NW; ++n)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[n][j] = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // plane j of byte b, in place (scale 4^j), plane 3 moved to bits 4-5 (scale 16)
        auto pl = [&](uint32_t b) { return j < 3 ? (b & (0x03030303u << (2 * j))) : ((b >> 2) & 0x30303030u); };
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const uint4 xv = x.q[8 * h + 2 * j + kk];
          const int sb = 8 * h + 2 * j + kk;
#pragma unroll
          for (int n = 0; n < NW; ++n) {
            const uint4 q = w[n].q[2 * h + kk];
            int s = dot4(pl(q.x), xv.x, 0);
            s = dot4(pl(q.y), xv.y, s);
            s = dot4(pl(q.z), xv.z, s);
            s = dot4(pl(q.w), xv.w, s);
            const int sc = (int)((u4c(w[n].sc, sb >> 2) >> (8 * (sb & 3))) & 15u);
            acc[n][j] = mad24(sc, s, acc[n][j]);
          }
        }
      }
    const uint4 b0 = x.bs[0], b1 = x.bs[1];
    const uint32_t bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      const int isum = acc[n][0] + (acc[n][1] >> 2) + ((acc[n][2] + acc[n][3]) >> 4);
      int imin = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t mm = (u4c(w[n].sc, c) >> 4) & 0x0f0f0f0fu;  // mins of sub-blocks 4c..4c+3
        imin = sdot2(__builtin_amdgcn_perm(0u, mm, 0x0c010c00u), bs[2 * c], imin);
        imin = sdot2(__builtin_amdgcn_perm(0u, mm, 0x0c030c02u), bs[2 * c + 1], imin);
      }
      ri[n] = isum;
      rm[n] = imin;
    }
  } else if constexpr (T == T_Q3_K) {
    // q3 = q2 + 4 * hbit - 4; hmask byte l (l = 4k + i) holds bit 4h + j of
    // weight 128h + 32j + l.  Plane j is kept in place (bits 2j..2j+1, scale
    // 4^j; plane 3 moved to bits 4-5, scale 16) with its high bit moved next to
    // it (bit 2j + 2, or 6 for plane 3), so one v_dot4 per 4 weights gives
    // 4^j * (q2 + 4 * hbit) . x; the -4 goes through the 16-weight bsums.
    int accq[NW][4], soff[NW];
    uint32_t s4[NW][4];
#pragma unroll
    for (int n = 0; n < NW; ++n) {
#pragma unroll
      for (int j = 0; j < 4; ++j) accq[n][j] = 0;
      soff[n] = 0;
      // 6-bit scales as bytes (ggml's aux[] unpacking), xor 32: a 6-bit signed field is sc - 32
      const uint32_t a0 = w[n].sc[0], a1 = w[n].sc[1], a2 = w[n].sc[2];
      s4[n][0] = ((a0 & 0x0f0f0f0fu) | ((a2 & 0x03030303u) << 4)) ^ 0x20202020u;
      s4[n][1] = ((a1 & 0x0f0f0f0fu) | (((a2 >> 2) & 0x03030303u) << 4)) ^ 0x20202020u;
      s4[n][2] = (((a0 >> 4) & 0x0f0f0f0fu) | (((a2 >> 4) & 0x03030303u) << 4)) ^ 0x20202020u;
      s4[n][3] = (((a1 >> 4) & 0x0f0f0f0fu) | (((a2 >> 6) & 0x03030303u) << 4)) ^ 0x20202020u;
    }
    // half h = part: sub-blocks 8h .. 8h + 7, hmask bits 4h + j (moved down to j)
    const int h = part;
    const uint4 bh = x.bs[h];
    const uint32_t bsw[4] = {bh.x, bh.y, bh.z, bh.w};
    uint4 hmh[NW][2];
    uint32_t sh4[NW][2];
#pragma unroll
    for (int n = 0; n < NW; ++n) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const uint4 m = w[n].hm[kk];
        const uint32_t c = 4u * (uint32_t)h;
        hmh[n][kk] = make_uint4(m.x >> c, m.y >> c, m.z >> c, m.w >> c);
      }
      sh4[n][0] = h ? s4[n][2] : s4[n][0];
      sh4[n][1] = h ? s4[n][3] : s4[n][1];
    }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = j < 3 ? 2 * j + 2 : 6, sft = t - j;
        auto val = [&](uint32_t b, uint32_t m) {
          const uint32_t pl = j < 3 ? (b & (0x03030303u << (2 * j))) : ((b >> 2) & 0x30303030u);
          const uint32_t hs = sft >= 0 ? (m << sft) : (m >> -sft);
          return pl | (hs & (0x01010101u << t));
        };
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const uint4 xv = x.q[8 * h + 2 * j + kk];
          const int sb = 2 * j + kk;  // sub-block 8h + sb
          const int bs = (int)(int16_t)(bsw[sb >> 1] >> (16 * (sb & 1)));
#pragma unroll
          for (int n = 0; n < NW; ++n) {
            const uint4 q = w[n].q[kk];
            const uint4 hm = hmh[n][kk];
            int sq = dot4(val(q.x, hm.x), xv.x, 0);
            sq = dot4(val(q.y, hm.y), xv.y, sq);
            sq = dot4(val(q.z, hm.z), xv.z, sq);
            sq = dot4(val(q.w, hm.w), xv.w, sq);
            const int sc = __builtin_amdgcn_sbfe((int)sh4[n][sb >> 2], 8 * (sb & 3), 6);
            accq[n][j] = mad24(sc, sq, accq[n][j]);
            soff[n] = mad24(sc, bs, soff[n]);
          }
        }
      }
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      ri[n] = accq[n][0] + (accq[n][1] >> 2) + ((accq[n][2] + accq[n][3]) >> 4) - 4 * soff[n];
      rm[n] = 0;
    }
  } else if constexpr (T == T_Q4_K) {
    // part p: sub-blocks 4p..4p+3; qs bytes 32i..32i+31 of group i = 2p + g hold
    // sub-block 2i in the low nibbles and 2i+1 in the high nibbles
    const uint4 b = x.bs[part];  // bsums of sub-blocks 4p..4p+3 (two 16-sums each)
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      const uint32_t u0 = w[n].hdr.y, u1 = w[n].hdr.z, u2 = w[n].hdr.w;
      const uint32_t scv = part == 0 ? (u0 & 0x3f3f3f3fu) : ((u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4));
      const uint32_t mv =
          part == 0 ? (u1 & 0x3f3f3f3fu) : (((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4));
      int isum = 0, imin = 0;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int i = 2 * part + g;
        int slo = 0, shi = 0;
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          const uint4 qv = w[n].q[2 * g + mm];
          const uint4 xl = x.q[4 * i + mm], xh = x.q[4 * i + 2 + mm];
          slo = dot4(qv.x & 0x0f0f0f0fu, xl.x, slo);
          slo = dot4(qv.y & 0x0f0f0f0fu, xl.y, slo);
          slo = dot4(qv.z & 0x0f0f0f0fu, xl.z, slo);
          slo = dot4(qv.w & 0x0f0f0f0fu, xl.w, slo);
          shi = dot4((qv.x >> 4) & 0x0f0f0f0fu, xh.x, shi);
          shi = dot4((qv.y >> 4) & 0x0f0f0f0fu, xh.y, shi);
          shi = dot4((qv.z >> 4) & 0x0f0f0f0fu, xh.z, shi);
          shi = dot4((qv.w >> 4) & 0x0f0f0f0fu, xh.w, shi);
        }
        isum = mad24((int)((scv >> (16 * g)) & 0xffu), slo, isum);
        isum = mad24((int)((scv >> (16 * g + 8)) & 0xffu), shi, isum);
      }
      // min of local sub-block l times both 16-sums of that sub-block: (m, m) . (bs_lo, bs_hi)
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c000c00u), b.x, imin);
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c010c01u), b.y, imin);
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c020c02u), b.z, imin);
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c030c03u), b.w, imin);
      ri[n] = isum;
      rm[n] = imin;
    }
  } else if constexpr (T == T_Q5_K) {
    // Q4_K's structure; bit 2i / 2i+1 of qh byte l is bit 4 of the low / high
    // nibble value of qs byte 32i + l
    const uint4 b = x.bs[part];
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      const uint32_t u0 = w[n].hdr.y, u1 = w[n].hdr.z, u2 = w[n].hdr.w;
      const uint32_t scv = part == 0 ? (u0 & 0x3f3f3f3fu) : ((u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4));
      const uint32_t mv =
          part == 0 ? (u1 & 0x3f3f3f3fu) : (((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4));
      int isum = 0, imin = 0;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int i = 2 * part + g;
        int slo = 0, shi = 0;
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          const uint4 qv = w[n].q[2 * g + mm];
          const uint4 hv = w[n].qh[mm];
          const uint4 xl = x.q[4 * i + mm], xh = x.q[4 * i + 2 + mm];
          auto lo = [&](uint32_t q, uint32_t h) { return (q & 0x0f0f0f0fu) | (((h >> (2 * i)) & 0x01010101u) << 4); };
          auto hi = [&](uint32_t q, uint32_t h) {
            return ((q >> 4) & 0x0f0f0f0fu) | (((h >> (2 * i + 1)) & 0x01010101u) << 4);
          };
          slo = dot4(lo(qv.x, hv.x), xl.x, slo);
          slo = dot4(lo(qv.y, hv.y), xl.y, slo);
          slo = dot4(lo(qv.z, hv.z), xl.z, slo);
          slo = dot4(lo(qv.w, hv.w), xl.w, slo);
          shi = dot4(hi(qv.x, hv.x), xh.x, shi);
          shi = dot4(hi(qv.y, hv.y), xh.y, shi);
          shi = dot4(hi(qv.z, hv.z), xh.z, shi);
          shi = dot4(hi(qv.w, hv.w), xh.w, shi);
        }
        isum = mad24((int)((scv >> (16 * g)) & 0xffu), slo, isum);
        isum = mad24((int)((scv >> (16 * g + 8)) & 0xffu), shi, isum);
      }
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c000c00u), b.x, imin);
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c010c01u), b.y, imin);
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c020c02u), b.z, imin);
      imin = sdot2(__builtin_amdgcn_perm(0u, mv, 0x0c030c03u), b.w, imin);
      ri[n] = isum;
      rm[n] = imin;
    }
  } else if constexpr (T == T_IQ3_XXS) {
    // part p: sub-blocks 4p + i; group l of 8 weights takes grid entries from
    // index bytes 2l, 2l + 1 of the sub-block and its 7-bit sign pattern
    const uint32_t *g3 = reinterpret_cast<const uint32_t *>(lds_grid);
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      int isum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ib = 4 * part + i;
        const uint32_t aux = u4c(w[n].sas, i);
        const uint4 xa = x.q[2 * ib], xb = x.q[2 * ib + 1];
        const uint32_t xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        int s = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
          const uint32_t iw = w[n].gi[2 * i + (l >> 1)];
          const uint32_t g1 = g3[(iw >> (16 * (l & 1))) & 0xffu], g2 = g3[(iw >> (16 * (l & 1) + 8)) & 0xffu];
          const uint64_t m = lds_signs[(aux >> (7 * l)) & 127u];
          const uint32_t mlo = (uint32_t)m, mhi = (uint32_t)(m >> 32);
          s = dot4(sign_bytes(g1, mlo), xs[2 * l], s);
          s = dot4(sign_bytes(g2, mhi), xs[2 * l + 1], s);
        }
        isum = mad24(2 * (int)(aux >> 28) + 1, s, isum);
      }
      ri[n] = isum;
      rm[n] = 0;
    }
  } else if constexpr (T == T_IQ4_XS) {
    // part p: sub-blocks 4p..4p+3, sub-block ib's 16 qs bytes in q[ib - 4p]: low
    // nibbles pair with activation chunk 2ib, high nibbles with 2ib + 1; the
    // 16-byte value table is in lds_grid
    const uint32_t t0 = (uint32_t)lds_grid[0], t1 = (uint32_t)(lds_grid[0] >> 32);
    const uint32_t t2 = (uint32_t)lds_grid[1], t3 = (uint32_t)(lds_grid[1] >> 32);
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      int isum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ib = 4 * part + i;
        const uint4 qv = w[n].q[i];
        const uint4 xl = x.q[2 * ib], xh = x.q[2 * ib + 1];
        int s = 0;
        s = dot4(lut16(qv.x & 0x0f0f0f0fu, t0, t1, t2, t3), xl.x, s);
        s = dot4(lut16(qv.y & 0x0f0f0f0fu, t0, t1, t2, t3), xl.y, s);
        s = dot4(lut16(qv.z & 0x0f0f0f0fu, t0, t1, t2, t3), xl.z, s);
        s = dot4(lut16(qv.w & 0x0f0f0f0fu, t0, t1, t2, t3), xl.w, s);
        s = dot4(lut16((qv.x >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3), xh.x, s);
        s = dot4(lut16((qv.y >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3), xh.y, s);
        s = dot4(lut16((qv.z >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3), xh.z, s);
        s = dot4(lut16((qv.w >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3), xh.w, s);
        isum = mad24(iq4_scale(w[n].hdr.x, w[n].hdr.y, ib), s, isum);
      }
      ri[n] = isum;
      rm[n] = 0;
    }
  } else if constexpr (T == T_Q6_K) {
    // half h = part: weight 128h + 32g + l sits in activation chunk 8h + 2g + (l >> 4),
    // which is also its 16-weight sub-block; value (nibble | 2 bits << 4) - 32,
    // the -32 folded in as -32 * sum sc * bsum
    const uint4 b0 = x.bs[0], b1 = x.bs[1];
    const uint32_t bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      int isum = 0, soff = 0;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int c = 8 * part + 2 * g + kk;  // chunk = sub-block
          const uint4 xv = x.q[c];
          const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
          int s = 0;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t q = w[n].ql[8 * (g & 1) + 4 * kk + d];
            const uint32_t lo = g < 2 ? (q & 0x0f0f0f0fu) : ((q >> 4) & 0x0f0f0f0fu);
            const uint32_t hb = ((w[n].qh[4 * kk + d] >> (2 * g)) & 0x03030303u) << 4;
            s = dot4(lo | hb, xs[d], s);
          }
          const int sl = 2 * g + kk;  // scale byte within the half
          const int sc = (int)(int8_t)(w[n].sc[sl >> 2] >> (8 * (sl & 3)));
          isum = mad24(sc, s, isum);
          soff = mad24(sc, (int)(int16_t)(bs[c >> 1] >> (16 * (c & 1))), soff);
        }
      ri[n] = isum - 32 * soff;
      rm[n] = 0;
    }
  } else {  // IQ2_XXS: sub-block ib uses qs dwords 2ib (4 grid indices), 2ib+1 (4 x 7-bit signs, 4-bit scale)
    int isum[NW];
#pragma unroll
    for (int n = 0; n < NW; ++n) isum[n] = 0;
    // all table reads of a batch of sub-blocks (two for a single weight row)
    // are issued before the first dot that uses them
    constexpr int IBB = NW == 1 ? 2 : 1;
    constexpr int NSB = HALF ? 4 : 8;      // sub-blocks in the unit
    const int xb = HALF ? 4 * part : 0;    // first sub-block of the unit in the block
#pragma unroll
    for (int ib0 = 0; ib0 < NSB; ib0 += IBB) {
      uint64_t g[IBB][NW][4], m[IBB][NW][4];
#pragma unroll
      for (int bb = 0; bb < IBB; ++bb)
#pragma unroll
        for (int n = 0; n < NW; ++n) {
          const int ib = ib0 + bb;
          const uint32_t aux0 = u4c(w[n].q[ib >> 1], 2 * (ib & 1)), aux1 = u4c(w[n].q[ib >> 1], 2 * (ib & 1) + 1);
#pragma unroll
          for (int l = 0; l < 4; ++l) {
            g[bb][n][l] = lds_grid[(aux0 >> (8 * l)) & 0xffu];
            m[bb][n][l] = lds_signs[(aux1 >> (7 * l)) & 127u];
          }
        }
#pragma unroll
      for (int bb = 0; bb < IBB; ++bb) {
        const int ib = ib0 + bb;
        const uint4 x0 = x.q[2 * (xb + ib)], x1 = x.q[2 * (xb + ib) + 1];
        const uint32_t xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int n = 0; n < NW; ++n) {
          const uint32_t aux1 = u4c(w[n].q[ib >> 1], 2 * (ib & 1) + 1);
          int sacc = 0;
#pragma unroll
          for (int l = 0; l < 4; ++l) {
            // conditional byte negate: (g ^ m) + (m & 1) per byte (no carries: 8 <= g <= 255)
            const uint64_t gv = g[bb][n][l], mv = m[bb][n][l];
            sacc = dot4(sign_bytes((uint32_t)gv, (uint32_t)mv), xs[2 * l], sacc);
            sacc = dot4(sign_bytes((uint32_t)(gv >> 32), (uint32_t)(mv >> 32)), xs[2 * l + 1], sacc);
          }
          isum[n] = mad24(2 * (int)(aux1 >> 28) + 1, sacc, isum[n]);
        }
      }
    }
#pragma unroll
    for (int n = 0; n < NW; ++n) {
      ri[n] = isum[n];
      rm[n] = 0;
    }
  }
}

// float contribution of a unit from its integer parts (ggml's vec_dot combine)
template <int T>
__device__ __forceinline__ float unit_float(const Unit<T> &w, float xd, int isum, int imin) {
  if constexpr (T == T_Q2_K) {
    const float d = h2f((uint16_t)(w.dd & 0xffffu)), dmin = h2f((uint16_t)(w.dd >> 16));
    return (xd * d) * (float)isum - (xd * dmin) * (float)imin;
  } else if constexpr (T == T_Q3_K) {
    return (xd * h2f((uint16_t)(w.d & 0xffffu))) * (float)isum;
  } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
    const float d = h2f((uint16_t)(w.hdr.x & 0xffffu)), dmin = h2f((uint16_t)(w.hdr.x >> 16));
    return (xd * d) * (float)isum - (xd * dmin) * (float)imin;
  } else if constexpr (T == T_Q6_K) {
    return (xd * h2f((uint16_t)(w.d & 0xffffu))) * (float)isum;
  } else if constexpr (T == T_IQ4_XS) {
    return (xd * h2f((uint16_t)(w.hdr.x & 0xffffu))) * (float)isum;
  } else if constexpr (T == T_IQ3_XXS) {
    return 0.25f * ((xd * h2f((uint16_t)(w.d & 0xffffu))) * (float)isum);
  } else {
    return 0.125f * ((xd * h2f((uint16_t)(w.d & 0xffffu))) * (float)isum);
  }
}

// A Q3_K half-block unit expanded before its activation is known (the decode
// kernel's first down step, while the workgroup waits for the act rows): the
// 32 plane words of unit_ints' Q3_K branch (plane j's two value bits in
// place, its high bit moved next to them), the half's 6-bit scales as bytes
// and d.  exp_dot then needs only the v_dot4s and the scale multiply-adds,
// with the same integer sums, so its result is the unit_dots result bit for bit.
struct Q3Exp {
  uint32_t v[32];  // [plane j][sub-block kk][word]
  uint32_t sh4[2];
  uint32_t d;
};
__device__ __forceinline__ void q3_expand(const Unit<T_Q3_K> &w, int part, Q3Exp &e) {
  const uint32_t a0 = w.sc[0], a1 = w.sc[1], a2 = w.sc[2];
  const int h = part;
  e.sh4[0] = h ? ((((a0 >> 4) & 0x0f0f0f0fu) | (((a2 >> 4) & 0x03030303u) << 4)) ^ 0x20202020u)
               : (((a0 & 0x0f0f0f0fu) | ((a2 & 0x03030303u) << 4)) ^ 0x20202020u);
  e.sh4[1] = h ? ((((a1 >> 4) & 0x0f0f0f0fu) | (((a2 >> 6) & 0x03030303u) << 4)) ^ 0x20202020u)
               : (((a1 & 0x0f0f0f0fu) | (((a2 >> 2) & 0x03030303u) << 4)) ^ 0x20202020u);
  e.d = w.d;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const uint4 m = w.hm[kk];
    const uint32_t c = 4u * (uint32_t)h;
    const uint32_t hm[4] = {m.x >> c, m.y >> c, m.z >> c, m.w >> c};
    const uint32_t q[4] = {w.q[kk].x, w.q[kk].y, w.q[kk].z, w.q[kk].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = j < 3 ? 2 * j + 2 : 6, sft = t - j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t pl = j < 3 ? (q[i] & (0x03030303u << (2 * j))) : ((q[i] >> 2) & 0x30303030u);
        const uint32_t hs = sft >= 0 ? (hm[i] << sft) : (hm[i] >> -sft);
        e.v[8 * j + 4 * kk + i] = pl | (hs & (0x01010101u << t));
      }
    }
  }
}
// The same for an IQ2_XXS half-block unit (sub-blocks 4 part .. 4 part + 3):
// the signed grid bytes of its 128 weights (table reads and sign application
// done), the four 4-bit scales as bytes and d.
struct IQ2Exp {
  uint32_t v[32];  // [sub-block][word]
  uint32_t ls;     // byte ib: 2 ls + 1 of sub-block ib
  uint32_t d;
};
__device__ __forceinline__ void iq2_expand(const Unit<T_IQ2_XXS> &w, const uint64_t *lds_grid,
                                           const uint64_t *lds_signs, IQ2Exp &e) {
  e.d = w.d;
  uint32_t ls = 0;
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
    const uint32_t aux0 = u4c(w.q[ib >> 1], 2 * (ib & 1)), aux1 = u4c(w.q[ib >> 1], 2 * (ib & 1) + 1);
    uint64_t g[4], m[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      g[l] = lds_grid[(aux0 >> (8 * l)) & 0xffu];
      m[l] = lds_signs[(aux1 >> (7 * l)) & 127u];
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      e.v[8 * ib + 2 * l] = sign_bytes((uint32_t)g[l], (uint32_t)m[l]);
      e.v[8 * ib + 2 * l + 1] = sign_bytes((uint32_t)(g[l] >> 32), (uint32_t)(m[l] >> 32));
    }
    ls |= (2u * (aux1 >> 28) + 1u) << (8 * ib);
  }
  e.ls = ls;
}
__device__ __forceinline__ float iq2_exp_dot(const IQ2Exp &e, int part, const XBlk &x) {
  int isum = 0;
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
    const uint4 x0 = x.q[2 * (4 * part + ib)], x1 = x.q[2 * (4 * part + ib) + 1];
    const uint32_t xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    int sacc = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) sacc = dot4(e.v[8 * ib + q], xs[q], sacc);
    isum = mad24((int)((e.ls >> (8 * ib)) & 0xffu), sacc, isum);
  }
  return 0.125f * ((x.d * h2f((uint16_t)(e.d & 0xffffu))) * (float)isum);
}
// The same for a Q4_K half-block unit (sub-blocks 4 part .. 4 part + 3): its
// nibbles as bytes, the half's scale and min bytes and (d, dmin).
struct Q4Exp {
  uint32_t v[32];  // [qs group g][16-byte chunk mm][low nibbles 0..3, high nibbles 4..7]
  uint32_t scv, mv, dd;
};
__device__ __forceinline__ void q4_expand(const Unit<T_Q4_K> &w, int part, Q4Exp &e) {
  const uint32_t u0 = w.hdr.y, u1 = w.hdr.z, u2 = w.hdr.w;
  e.scv = part == 0 ? (u0 & 0x3f3f3f3fu) : ((u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4));
  e.mv = part == 0 ? (u1 & 0x3f3f3f3fu) : (((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4));
  e.dd = w.hdr.x;
#pragma unroll
  for (int c = 0; c < 4; ++c) {  // c = 2 g + mm
    const uint4 qv = w.q[c];
    const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e.v[8 * c + i] = q[i] & 0x0f0f0f0fu;
      e.v[8 * c + 4 + i] = (q[i] >> 4) & 0x0f0f0f0fu;
    }
  }
}
__device__ __forceinline__ float q4_exp_dot(const Q4Exp &e, int part, const XBlk &x) {
  const uint4 b = x.bs[part];
  int isum = 0, imin = 0;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int i = 2 * part + g;
    int slo = 0, shi = 0;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const uint32_t *v = e.v + 8 * (2 * g + mm);
      const uint4 xl = x.q[4 * i + mm], xh = x.q[4 * i + 2 + mm];
      slo = dot4(v[0], xl.x, slo);
      slo = dot4(v[1], xl.y, slo);
      slo = dot4(v[2], xl.z, slo);
      slo = dot4(v[3], xl.w, slo);
      shi = dot4(v[4], xh.x, shi);
      shi = dot4(v[5], xh.y, shi);
      shi = dot4(v[6], xh.z, shi);
      shi = dot4(v[7], xh.w, shi);
    }
    isum = mad24((int)((e.scv >> (16 * g)) & 0xffu), slo, isum);
    isum = mad24((int)((e.scv >> (16 * g + 8)) & 0xffu), shi, isum);
  }
  imin = sdot2(__builtin_amdgcn_perm(0u, e.mv, 0x0c000c00u), b.x, imin);
  imin = sdot2(__builtin_amdgcn_perm(0u, e.mv, 0x0c010c01u), b.y, imin);
  imin = sdot2(__builtin_amdgcn_perm(0u, e.mv, 0x0c020c02u), b.z, imin);
  imin = sdot2(__builtin_amdgcn_perm(0u, e.mv, 0x0c030c03u), b.w, imin);
  const float d = h2f((uint16_t)(e.dd & 0xffffu)), dmin = h2f((uint16_t)(e.dd >> 16));
  return (x.d * d) * (float)isum - (x.d * dmin) * (float)imin;
}
// The same for a Q6_K half-block unit: its 6-bit values (without the -32) as
// bytes, the half's 8 signed scale bytes and d.
struct Q6Exp {
  uint32_t v[32];  // [sub-block 2 g + kk][word d]
  uint32_t sc[2];
  uint32_t d;
};
__device__ __forceinline__ void q6_expand(const Unit<T_Q6_K> &w, Q6Exp &e) {
  e.sc[0] = w.sc[0];
  e.sc[1] = w.sc[1];
  e.d = w.d;
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint32_t q = w.ql[8 * (g & 1) + 4 * kk + d];
        const uint32_t lo = g < 2 ? (q & 0x0f0f0f0fu) : ((q >> 4) & 0x0f0f0f0fu);
        const uint32_t hb = ((w.qh[4 * kk + d] >> (2 * g)) & 0x03030303u) << 4;
        e.v[4 * (2 * g + kk) + d] = lo | hb;
      }
}
__device__ __forceinline__ float q6_exp_dot(const Q6Exp &e, int part, const XBlk &x) {
  const uint4 b0 = x.bs[0], b1 = x.bs[1];
  const uint32_t bs[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
  int isum = 0, soff = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int c = 8 * part + 2 * g + kk;
      const uint4 xv = x.q[c];
      const uint32_t *v = e.v + 4 * (2 * g + kk);
      int sq = dot4(v[0], xv.x, 0);
      sq = dot4(v[1], xv.y, sq);
      sq = dot4(v[2], xv.z, sq);
      sq = dot4(v[3], xv.w, sq);
      const int sl = 2 * g + kk;
      const int sc = (int)(int8_t)(e.sc[sl >> 2] >> (8 * (sl & 3)));
      isum = mad24(sc, sq, isum);
      soff = mad24(sc, (int)(int16_t)(bs[c >> 1] >> (16 * (c & 1))), soff);
    }
  return (x.d * h2f((uint16_t)(e.d & 0xffffu))) * (float)(isum - 32 * soff);
}
// The same for an IQ3_XXS half-block unit: signed grid bytes of its 128
// weights, the four scales (2 ls + 1) as bytes and d.
struct IQ3Exp {
  uint32_t v[32];  // [sub-block i][word]
  uint32_t ls;
  uint32_t d;
};
__device__ __forceinline__ void iq3_expand(const Unit<T_IQ3_XXS> &w, const uint64_t *lds_grid,
                                           const uint64_t *lds_signs, IQ3Exp &e) {
  const uint32_t *g3 = reinterpret_cast<const uint32_t *>(lds_grid);
  e.d = w.d;
  uint32_t ls = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t aux = u4c(w.sas, i);
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t iw = w.gi[2 * i + (l >> 1)];
      const uint32_t g1 = g3[(iw >> (16 * (l & 1))) & 0xffu], g2 = g3[(iw >> (16 * (l & 1) + 8)) & 0xffu];
      const uint64_t m = lds_signs[(aux >> (7 * l)) & 127u];
      e.v[8 * i + 2 * l] = sign_bytes(g1, (uint32_t)m);
      e.v[8 * i + 2 * l + 1] = sign_bytes(g2, (uint32_t)(m >> 32));
    }
    ls |= (2u * (aux >> 28) + 1u) << (8 * i);
  }
  e.ls = ls;
}
__device__ __forceinline__ float iq3_exp_dot(const IQ3Exp &e, int part, const XBlk &x) {
  int isum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ib = 4 * part + i;
    const uint4 xa = x.q[2 * ib], xb = x.q[2 * ib + 1];
    const uint32_t xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    int sacc = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) sacc = dot4(e.v[8 * i + q], xs[q], sacc);
    isum = mad24((int)((e.ls >> (8 * i)) & 0xffu), sacc, isum);
  }
  return 0.25f * ((x.d * h2f((uint16_t)(e.d & 0xffffu))) * (float)isum);
}
// The same for an IQ4_XS half-block unit: its table values as bytes, the four
// sub-block scales (signed) as bytes and d.
struct IQ4Exp {
  uint32_t v[32];  // [sub-block i][low nibbles 0..3, high nibbles 4..7]
  uint32_t sc;
  uint32_t d;
};
__device__ __forceinline__ void iq4_expand(const Unit<T_IQ4_XS> &w, int part, const uint64_t *lds_grid, IQ4Exp &e) {
  const uint32_t t0 = (uint32_t)lds_grid[0], t1 = (uint32_t)(lds_grid[0] >> 32);
  const uint32_t t2 = (uint32_t)lds_grid[1], t3 = (uint32_t)(lds_grid[1] >> 32);
  e.d = w.hdr.x;
  uint32_t sc = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 qv = w.q[i];
    const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      e.v[8 * i + k] = lut16(q[k] & 0x0f0f0f0fu, t0, t1, t2, t3);
      e.v[8 * i + 4 + k] = lut16((q[k] >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3);
    }
    sc |= ((uint32_t)iq4_scale(w.hdr.x, w.hdr.y, 4 * part + i) & 0xffu) << (8 * i);
  }
  e.sc = sc;
}
__device__ __forceinline__ float iq4_exp_dot(const IQ4Exp &e, int part, const XBlk &x) {
  int isum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ib = 4 * part + i;
    const uint4 xl = x.q[2 * ib], xh = x.q[2 * ib + 1];
    const uint32_t xs[8] = {xl.x, xl.y, xl.z, xl.w, xh.x, xh.y, xh.z, xh.w};
    int sacc = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) sacc = dot4(e.v[8 * i + q], xs[q], sacc);
    isum = mad24(__builtin_amdgcn_sbfe((int)e.sc, 8 * i, 8), sacc, isum);
  }
  return (x.d * h2f((uint16_t)(e.d & 0xffffu))) * (float)isum;
}
struct NoExp {};  // the expansion slot of other down types (never dotted)
__device__ __forceinline__ float exp_dot(const NoExp &, int, const XBlk &) { return 0.0f; }
__device__ __forceinline__ float exp_dot(const IQ2Exp &e, int part, const XBlk &x) { return iq2_exp_dot(e, part, x); }
__device__ __forceinline__ float exp_dot(const Q4Exp &e, int part, const XBlk &x) { return q4_exp_dot(e, part, x); }
__device__ __forceinline__ float exp_dot(const Q6Exp &e, int part, const XBlk &x) { return q6_exp_dot(e, part, x); }
__device__ __forceinline__ float exp_dot(const IQ3Exp &e, int part, const XBlk &x) { return iq3_exp_dot(e, part, x); }
__device__ __forceinline__ float exp_dot(const IQ4Exp &e, int part, const XBlk &x) { return iq4_exp_dot(e, part, x); }
__device__ __forceinline__ float exp_dot(const Q3Exp &e, int part, const XBlk &x) {
  const int h = part;
  const uint4 bh = x.bs[h];
  const uint32_t bsw[4] = {bh.x, bh.y, bh.z, bh.w};
  int accq[4] = {0, 0, 0, 0}, soff = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint4 xv = x.q[8 * h + 2 * j + kk];
      const int sb = 2 * j + kk;
      const int bs = (int)(int16_t)(bsw[sb >> 1] >> (16 * (sb & 1)));
      const uint32_t *v = e.v + 8 * j + 4 * kk;
      int sq = dot4(v[0], xv.x, 0);
      sq = dot4(v[1], xv.y, sq);
      sq = dot4(v[2], xv.z, sq);
      sq = dot4(v[3], xv.w, sq);
      const int sc = __builtin_amdgcn_sbfe((int)e.sh4[sb >> 2], 8 * (sb & 3), 6);
      accq[j] = mad24(sc, sq, accq[j]);
      soff = mad24(sc, bs, soff);
    }
  }
  const int isum = accq[0] + (accq[1] >> 2) + ((accq[2] + accq[3]) >> 4) - 4 * soff;
  return (x.d * h2f((uint16_t)(e.d & 0xffffu))) * (float)isum;
}

// out[n] = float contribution of weight unit w[n] against activation block x
template <int T, int NW, bool HALF = false>
__device__ __forceinline__ void unit_dots(const Unit<T> (&w)[NW], int part, const XBlk &x, const uint64_t *lds_grid,
                                          const uint64_t *lds_signs, float (&out)[NW]) {
  static_assert(!HALF || T == T_IQ2_XXS, "half units: IQ2_XXS only");
  int ri[NW], rm[NW];
  unit_ints<T, NW, HALF>(w, part, x, lds_grid, lds_signs, ri, rm);
#pragma unroll
  for (int n = 0; n < NW; ++n) out[n] = unit_float<T>(w[n], x.d, ri[n], rm[n]);
}

}  // namespace zm
