// zm_device.hpp -- gfx950 device helpers shared by every zeromoe_amd kernel:
// GGUF super-block layouts, the per-lane "64-weight slice" integer dots
// against Q8_K activations, wave64 reductions and the bit-reproducible
// float helpers (exp, round-half-even) the router and quantizer use.
//
// Work unit: a 256-weight super-block is split into 4 quarters of 64
// weights; one lane owns one quarter.  A quarter is what one lane can dot
// with a handful of 16-byte loads:
//   Q2_K / Q3_K quarter q = (h, qq): qs bytes [32h+16qq, +16) hold weights
//       128h + 32j + 16qq + i (j = 0..3 bit-plane, i < 16), i.e. four
//       16-weight sub-blocks 8h + 2j + qq.
//   Q4_K quarter q: qs bytes [32q, +32) hold weights 64q + i (low nibble)
//       and 64q + 32 + i (high nibble): sub-blocks 2q and 2q+1.
//   Q5_K quarter q: as Q4_K, plus qh bytes [0, 32) whose bits 2q / 2q+1 are
//       bit 4 of the low / high nibble values.
//   Q6_K quarter q = (h, qq): weights 128h + 32g + 16qq + i (g = 0..3, i < 16):
//       low nibbles in ql bytes [64h+16qq, +16) (g = 0, 2: low / high nibble)
//       and [64h+32+16qq, +16) (g = 1, 3), top two bits at bit 2g of qh bytes
//       [32h+16qq, +16); 16-weight sub-blocks 8h + 2g + qq.
//   IQ2_XXS quarter q: 32-weight sub-blocks 2q and 2q+1 (16 bytes of qs).
//   IQ3_XXS quarter q: 32-weight sub-blocks 2q and 2q+1: grid indices at
//       bytes [2 + 16q, +16), scale+sign words at [66 + 8q, +8).
//   IQ4_XS quarter q: 32-weight sub-blocks 2q and 2q+1 = qs bytes [32q, +32)
//       (byte j of a sub-block: low nibble weight j, high nibble weight 16 + j).
// Block layouts: /root/reference/kernels/quant/kquant_matmul.cu:35-39,
// kernels/quant/iq2_matmul.cu:27.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

namespace zm {

constexpr int QK = 256;

enum : int {
  T_F32 = 0,
  T_F16 = 1,
  T_Q2_K = 10,
  T_Q3_K = 11,
  T_Q4_K = 12,
  T_Q5_K = 13,
  T_Q6_K = 14,
  T_Q8_K = 15,
  T_IQ2_XXS = 16,
  T_IQ3_XXS = 18,
  T_IQ4_XS = 23,
  T_I32 = 26,
};

__host__ __device__ constexpr int block_bytes(int t) {
  return t == T_Q2_K ? 84 : t == T_Q3_K ? 110 : t == T_Q4_K ? 144 : t == T_Q5_K ? 176 : t == T_Q6_K ? 210
       : t == T_IQ2_XXS ? 66 : t == T_IQ3_XXS ? 98 : t == T_IQ4_XS ? 136 : t == T_Q8_K ? 292 : 0;
}

// ---------------------------------------------------------------- loads

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
  uint4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
  uint2 v;
  __builtin_memcpy(&v, p, 8);
  return v;
}
__device__ __forceinline__ uint32_t ld4(const uint8_t *p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}
__device__ __forceinline__ uint16_t ld2(const uint8_t *p) {
  uint16_t v;
  __builtin_memcpy(&v, p, 2);
  return v;
}
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// bytes of g negated where the byte of the sign mask m is 0xff: (g ^ m) +
// (m & 1) per byte, carry-free for bytes 1..255, as one v_xad_u32 (the
// compiler emits xor + add) after the and
__device__ __forceinline__ uint32_t sign_bytes(uint32_t g, uint32_t m) {
  uint32_t r;
  asm("v_xad_u32 %0, %1, %2, %3" : "=v"(r) : "v"(g), "v"(m), "v"(m & 0x01010101u));
  return r;
}

// byte k (0..11) of three little-endian dwords
__device__ __forceinline__ uint32_t byte_of3(uint32_t s0, uint32_t s1, uint32_t s2, int k) {
  const uint32_t w = k < 4 ? s0 : (k < 8 ? s1 : s2);
  return (w >> (8 * (k & 3))) & 0xffu;
}

// ---------------------------------------------------------------- bit-reproducible float helpers

// ggml-quants.c nearest_int (round half to even via the 1.5*2^23 add).
__device__ __forceinline__ int nearest_int(float f) {
  const float v = f + 12582912.f;
  return (__float_as_int(v) & 0x007fffff) - 0x00400000;
}

// exp(x): Cody-Waite reduction by ln2 and a degree-7 Taylor polynomial; the
// same IEEE operation sequence as the host checker, so results are bitwise
// equal on CPU and GPU.  (Compiled with -ffp-contract=off.)
__device__ __forceinline__ float exp_f32(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __int_as_float(0x7f800000);
  if (x < -103.972084045410156f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412701138295233249664306640625e-4f;
  p = __builtin_fmaf(p, r, 1.388888922519981861114501953125e-3f);
  p = __builtin_fmaf(p, r, 8.33333376795053482055664062500e-3f);
  p = __builtin_fmaf(p, r, 4.16666679084300994873046875000e-2f);
  p = __builtin_fmaf(p, r, 1.66666671633720397949218750000e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + exp_f32(-g)); }

// ---------------------------------------------------------------- wave64 reductions
//
// Cross-lane steps use DPP (a VALU operand modifier, no LDS round trip):
// quad_perm(1,0,3,2) = xor 1, quad_perm(2,3,0,1) = xor 2, row_half_mirror and
// row_mirror combine 4- and 8-lane halves once every lane of the half holds the
// same partial; the four 16-lane rows are then combined with the row-swap
// permutes (lane_xor16 / lane_xor32).
// Every lane ends with the same result, in a fixed order (deterministic).
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
// max / min of v and v of the DPP partner lane in one VALU instruction (the
// DPP modifier on the max itself).  For canonical v (the output of an earlier
// max or min) this is fmaxf / fminf of the two; the compiler would put a
// canonicalizing max between a DPP move and fmaxf.  s_nop 1: the two wait
// states a DPP read needs after a VALU write of its source.
#define ZM_DPP_MINMAX(NAME, OP)                                                                          \
  template <int CTRL>                                                                                   \
  __device__ __forceinline__ float NAME(float v) {                                                      \
    float r;                                                                                            \
    if constexpr (CTRL == DPP_XOR1)                                                                     \
      asm("s_nop 1\n\t" OP " %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v)); \
    else if constexpr (CTRL == DPP_XOR2)                                                                \
      asm("s_nop 1\n\t" OP " %0, %1, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v)); \
    else if constexpr (CTRL == DPP_HALF_MIRROR)                                                         \
      asm("s_nop 1\n\t" OP " %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));     \
    else                                                                                                \
      asm("s_nop 1\n\t" OP " %0, %1, %1 row_mirror row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));          \
    return r;                                                                                           \
  }
ZM_DPP_MINMAX(dpp_max_f, "v_max_f32_dpp")
ZM_DPP_MINMAX(dpp_min_f, "v_min_f32_dpp")
#undef ZM_DPP_MINMAX
__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// the value of lane ^ 16 / lane ^ 32, through the gfx950 row-swap permutes
// (no trip through scalar registers); every lane of the wave must be active
__device__ __forceinline__ int lane_xor16(int v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (threadIdx.x & 16) ? (int)r[0] : (int)r[1];
}
__device__ __forceinline__ int lane_xor32(int v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? (int)r[0] : (int)r[1];
}
// sum over aligned groups of W lanes (W = 4, 8, 16, 32, 64); all lanes of a group get it
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
  v += dpp_f<DPP_XOR1>(v);
  v += dpp_f<DPP_XOR2>(v);
  if constexpr (W >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
  if constexpr (W >= 16) v += dpp_f<DPP_MIRROR>(v);
  // rows (0 + 1) + (2 + 3) in every lane (addition commutes)
  if constexpr (W >= 32) v += __int_as_float(lane_xor16(__float_as_int(v)));
  if constexpr (W == 64) v += __int_as_float(lane_xor32(__float_as_int(v)));
  return v;
}
template <int W>
__device__ __forceinline__ int group_sum_i(int v) {
  static_assert(W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
  v += dpp_i<DPP_XOR1>(v);
  v += dpp_i<DPP_XOR2>(v);
  if constexpr (W >= 8) v += dpp_i<DPP_HALF_MIRROR>(v);
  if constexpr (W >= 16) v += dpp_i<DPP_MIRROR>(v);
  if constexpr (W >= 32) v += lane_xor16(v);
  if constexpr (W == 64) v += lane_xor32(v);
  return v;
}
// LDS writes of this wave visible to its other lanes
__device__ __forceinline__ void stage_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
  v = fmaxf(v, __int_as_float(lane_xor16(__float_as_int(v))));
  return fmaxf(v, __int_as_float(lane_xor32(__float_as_int(v))));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  auto step = [](double x, auto ctrl_tag) -> double {
    constexpr int C = decltype(ctrl_tag)::value;
    const long long b = __double_as_longlong(x);
    const int lo = dpp_i<C>((int)(b & 0xffffffffll)), hi = dpp_i<C>((int)(b >> 32));
    return x + __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
  };
  v = step(v, std::integral_constant<int, DPP_XOR1>{});
  v = step(v, std::integral_constant<int, DPP_XOR2>{});
  v = step(v, std::integral_constant<int, DPP_HALF_MIRROR>{});
  v = step(v, std::integral_constant<int, DPP_MIRROR>{});
  // rows (0 + 1) + (2 + 3), the same sums in every lane (addition commutes)
  auto x16 = [](double x) {
    const long long b = __double_as_longlong(x);
    const int lo = lane_xor16((int)(b & 0xffffffffll)), hi = lane_xor16((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
  };
  auto x32 = [](double x) {
    const long long b = __double_as_longlong(x);
    const int lo = lane_xor32((int)(b & 0xffffffffll)), hi = lane_xor32((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
  };
  v = v + x16(v);
  return v + x32(v);
}

// Strict order "higher score, then lower index" as one 64-bit key: the
// order-preserving bits of the score above the complemented index.  Keys of
// distinct experts never tie; 0 is below every key.
__device__ __forceinline__ unsigned long long rank_key(float v, int e) {
  const uint32_t u = __float_as_uint(v + 0.0f);  // -0 -> +0: equal scores tie on the index
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)o << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}

// order-preserving 32-bit image of a score (the upper half of rank_key)
__device__ __forceinline__ uint32_t score_key(float v) {
  const uint32_t u = __float_as_uint(v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
  auto step = [&](auto tag) {
    constexpr int C = decltype(tag)::value;
    const uint32_t o = (uint32_t)dpp_i<C>((int)k);
    k = o > k ? o : k;
  };
  step(std::integral_constant<int, DPP_XOR1>{});
  step(std::integral_constant<int, DPP_XOR2>{});
  step(std::integral_constant<int, DPP_HALF_MIRROR>{});
  step(std::integral_constant<int, DPP_MIRROR>{});
  k = max(k, (uint32_t)lane_xor16((int)k));
  return max(k, (uint32_t)lane_xor32((int)k));
}
// inverse of score_key (-0 comes back as +0)
__device__ __forceinline__ float score_from_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// maximum over aligned groups of W lanes (W = 16, 32, 64); all lanes of a group get it
__device__ __forceinline__ uint32_t group_max_u32(uint32_t k, int W) {
  auto step = [&](auto tag) {
    constexpr int C = decltype(tag)::value;
    const uint32_t o = (uint32_t)dpp_i<C>((int)k);
    k = o > k ? o : k;
  };
  step(std::integral_constant<int, DPP_XOR1>{});
  step(std::integral_constant<int, DPP_XOR2>{});
  step(std::integral_constant<int, DPP_HALF_MIRROR>{});
  step(std::integral_constant<int, DPP_MIRROR>{});
  if (W >= 32) k = max(k, (uint32_t)lane_xor16((int)k));
  if (W >= 64) k = max(k, (uint32_t)lane_xor32((int)k));
  return k;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
  auto step = [&](auto tag) {
    constexpr int C = decltype(tag)::value;
    const uint32_t lo = (uint32_t)dpp_i<C>((int)(uint32_t)k), hi = (uint32_t)dpp_i<C>((int)(uint32_t)(k >> 32));
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    k = o > k ? o : k;
  };
  step(std::integral_constant<int, DPP_XOR1>{});
  step(std::integral_constant<int, DPP_XOR2>{});
  step(std::integral_constant<int, DPP_HALF_MIRROR>{});
  step(std::integral_constant<int, DPP_MIRROR>{});
  unsigned long long best = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 16 * r);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 16 * r);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    best = o > best ? o : best;
  }
  return best;
}

// ---------------------------------------------------------------- Q8_K activations (planar)
//
// Internal activation rows use a planar layout with the content of ggml's
// block_q8_K (292 B per 256): qs[nb*256] | bsums[nb*16] (i16) | d[nb] (f32),
// the row padded to 16 bytes, so every 16-byte read of qs or bsums is aligned.
__host__ __device__ constexpr size_t q8_row_bytes(int nb) { return ((size_t)nb * 292 + 15) & ~(size_t)15; }
__host__ __device__ constexpr size_t q8_bs_off(int nb) { return (size_t)nb * 256; }
__host__ __device__ constexpr size_t q8_d_off(int nb) { return (size_t)nb * 288; }

struct Q8Slice {
  uint4 q[4];    // 64 int8, in the order the weight quarter needs them
  int bs[4];     // sums of 16-weight groups used by the quarter (type dependent)
  float d;
};

// positions of the 64 activations matching weight quarter q of block b
template <int T>
__device__ __forceinline__ void load_q8_slice(const uint8_t *row, int nb, int b, int q, Q8Slice &s) {
  const uint8_t *qs = row + (size_t)b * 256;
  const int16_t *bs = reinterpret_cast<const int16_t *>(row + q8_bs_off(nb)) + b * 16;
  s.d = reinterpret_cast<const float *>(row + q8_d_off(nb))[b];
  if constexpr (T == T_Q2_K || T == T_Q3_K || T == T_Q6_K) {
    const int h = q >> 1, qq = q & 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s.q[j] = *reinterpret_cast<const uint4 *>(qs + 128 * h + 32 * j + 16 * qq);
      s.bs[j] = bs[8 * h + 2 * j + qq];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) s.q[j] = *reinterpret_cast<const uint4 *>(qs + 64 * q + 16 * j);
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
#pragma unroll
      for (int j = 0; j < 4; ++j) s.bs[j] = bs[4 * q + j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) s.bs[j] = 0;
    }
  }
}

// ---------------------------------------------------------------- weight quarters

struct WSlice {
  uint4 a;     // Q2/Q3: qs16 ; Q4/Q5: qs[0..16) ; Q6: ql[64h+16qq, +16) ; IQ2: qs 16 B
  uint4 b;     // Q3: hmask16 ; Q4/Q5: qs[16..32) ; Q6: ql[64h+32+16qq, +16)
  uint4 c;     // Q4/Q5: header (d, dmin, scales) ; Q3: scales(12) + d in .w low half
  uint4 g;     // Q5: qh[0..16) ; Q6: qh[32h+16qq, +16)
  uint4 hh;    // Q5: qh[16..32)
  uint2 e;     // Q2: scales[8h .. 8h+8) ; Q6: scales[8h .. 8h+8)
  uint32_t f;  // Q2: d|dmin ; Q6, IQ2: d
};

template <int T>
__device__ __forceinline__ void load_w_slice(const uint8_t *blk, int q, WSlice &w) {
  if constexpr (T == T_Q2_K) {
    w.e = ld8(blk + 8 * (q >> 1));
    w.a = ld16(blk + 16 + 16 * q);
    w.f = ld4(blk + 80);
  } else if constexpr (T == T_Q3_K) {
    w.b = ld16(blk + 16 * (q & 1));
    w.a = ld16(blk + 32 + 16 * q);
    w.c.x = ld4(blk + 96);
    w.c.y = ld4(blk + 100);
    w.c.z = ld4(blk + 104);
    w.c.w = ld2(blk + 108);
  } else if constexpr (T == T_Q4_K) {
    w.c = ld16(blk);
    w.a = ld16(blk + 16 + 32 * q);
    w.b = ld16(blk + 32 + 32 * q);
  } else if constexpr (T == T_Q5_K) {
    w.c = ld16(blk);
    w.g = ld16(blk + 16);
    w.hh = ld16(blk + 32);
    w.a = ld16(blk + 48 + 32 * q);
    w.b = ld16(blk + 64 + 32 * q);
  } else if constexpr (T == T_IQ3_XXS) {
    w.f = ld2(blk);
    w.a = ld16(blk + 2 + 16 * q);
    w.e = ld8(blk + 66 + 8 * q);
  } else if constexpr (T == T_IQ4_XS) {
    w.e = ld8(blk);  // d | scales_h, scales_l
    w.a = ld16(blk + 8 + 32 * q);
    w.b = ld16(blk + 24 + 32 * q);
  } else if constexpr (T == T_Q6_K) {
    const int h = q >> 1, qq = q & 1;
    w.a = ld16(blk + 64 * h + 16 * qq);
    w.b = ld16(blk + 64 * h + 32 + 16 * qq);
    w.g = ld16(blk + 128 + 32 * h + 16 * qq);
    w.e = ld8(blk + 192 + 8 * h);
    w.f = ld2(blk + 208);
  } else {  // IQ2_XXS
    w.f = ld2(blk);
    w.a = ld16(blk + 2 + 16 * q);
  }
}

// ---- the same slices through buffer loads: `vo` is the lane's byte offset of
// the block start inside the resource (VGPR), `so` a wave-uniform byte offset
// (SGPR, e.g. expert * expert_bytes + row * row_bytes).  Out-of-range reads
// return zero instead of faulting.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// lane offset past every buffer extent (all < 2^31): a load through it returns
// zeros, a store through it is dropped
constexpr int OOR = (int)0x80000000u;
__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bld16(rsrc_t r, int vo, int so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 bld8(rsrc_t r, int vo, int so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t bld4(rsrc_t r, int vo, int so) { return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0); }
__device__ __forceinline__ uint32_t bld2(rsrc_t r, int vo, int so) { return __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0); }

template <int T>
__device__ __forceinline__ void load_w_slice_b(rsrc_t r, int vo, int so, int q, WSlice &w) {
  if constexpr (T == T_Q2_K) {
    w.e = bld8(r, vo + 8 * (q >> 1), so);
    w.a = bld16(r, vo + 16 + 16 * q, so);
    w.f = bld4(r, vo + 80, so);
  } else if constexpr (T == T_Q3_K) {
    w.b = bld16(r, vo + 16 * (q & 1), so);
    w.a = bld16(r, vo + 32 + 16 * q, so);
    w.c.x = bld4(r, vo + 96, so);
    w.c.y = bld4(r, vo + 100, so);
    w.c.z = bld4(r, vo + 104, so);
    w.c.w = bld2(r, vo + 108, so);
  } else if constexpr (T == T_Q4_K) {
    w.c = bld16(r, vo, so);
    w.a = bld16(r, vo + 16 + 32 * q, so);
    w.b = bld16(r, vo + 32 + 32 * q, so);
  } else if constexpr (T == T_Q5_K) {
    w.c = bld16(r, vo, so);
    w.g = bld16(r, vo + 16, so);
    w.hh = bld16(r, vo + 32, so);
    w.a = bld16(r, vo + 48 + 32 * q, so);
    w.b = bld16(r, vo + 64 + 32 * q, so);
  } else if constexpr (T == T_IQ3_XXS) {
    w.f = bld2(r, vo, so);
    w.a = bld16(r, vo + 2 + 16 * q, so);
    w.e = bld8(r, vo + 66 + 8 * q, so);
  } else if constexpr (T == T_IQ4_XS) {
    w.e = bld8(r, vo, so);
    w.a = bld16(r, vo + 8 + 32 * q, so);
    w.b = bld16(r, vo + 24 + 32 * q, so);
  } else if constexpr (T == T_Q6_K) {
    const int h = q >> 1, qq = q & 1;
    w.a = bld16(r, vo + 64 * h + 16 * qq, so);
    w.b = bld16(r, vo + 64 * h + 32 + 16 * qq, so);
    w.g = bld16(r, vo + 128 + 32 * h + 16 * qq, so);
    w.e = bld8(r, vo + 192 + 8 * h, so);
    w.f = bld2(r, vo + 208, so);
  } else {  // IQ2_XXS
    w.f = bld2(r, vo, so);
    w.a = bld16(r, vo + 2 + 16 * q, so);
  }
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ uint32_t u4_get(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// four 4-bit indices (one per byte) -> the four signed table bytes of a
// 16-entry table held as four dwords (two byte permutes and a select on bit 3)
__device__ __forceinline__ uint32_t lut16(uint32_t idx, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  const uint32_t sel = idx & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel), hi = __builtin_amdgcn_perm(t3, t2, sel);
  const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xffu;
  return (hi & m) | (lo & ~m);
}

// 6-bit IQ4_XS scale of sub-block ib (value ls - 32) from the header dwords
// x = d | scales_h << 16, y = scales_l
__device__ __forceinline__ int iq4_scale(uint32_t x, uint32_t y, int ib) {
  return (int)(((y >> (4 * ib)) & 15u) | (((x >> (16 + 2 * ib)) & 3u) << 4)) - 32;
}

// Integer parts of one quarter: isum = sum_sub sc*dot (Q3_K: includes the
// -4*bsum term of missing high bits), imin = sum_sub m*bsum (Q2_K/Q4_K).
struct QInt {
  int isum, imin;
};

template <int T>
__device__ __forceinline__ QInt quarter_int(const WSlice &w, int q, const Q8Slice &a, const uint64_t *lds_grid,
                                            const uint64_t *lds_signs) {
  QInt r{0, 0};
  if constexpr (T == T_Q2_K) {
    // Bit-plane j is masked in place (no shift for j < 3): the dot then carries
    // a factor 4^j that is folded into the scale, so 16*isum is accumulated
    // exactly and shifted back at the end.
    const int qq = q & 1;
    const uint32_t lo = w.e.x >> (8 * qq), hi = w.e.y >> (8 * qq);
    int s16 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t scb = ((j < 2 ? lo : hi) >> (16 * (j & 1))) & 0xffu;
      int dj = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t x = u4_get(w.a, i);
        const uint32_t m = j < 3 ? (x & (0x03030303u << (2 * j))) : ((x >> 2) & 0x30303030u);
        dj = dot4(m, u4_get(a.q[j], i), dj);
      }
      s16 += (int)((scb & 15u) << (j == 0 ? 4 : (j == 1 ? 2 : 0))) * dj;
      r.imin += (int)(scb >> 4) * a.bs[j];
    }
    r.isum = s16 >> 4;
  } else if constexpr (T == T_Q3_K) {
    // value c + 4*hbit (0..7) is assembled in place at bit 2j (j < 3) or 4 (j = 3),
    // the 4^j factor folded into the scale as for Q2_K; the -4 offset is -4*bsum.
    const int h = q >> 1, qq = q & 1;
    int s16 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = 2 * j + qq;  // scales byte index of the low nibble
      const uint32_t lo4 = (byte_of3(w.c.x, w.c.y, w.c.z, k) >> (4 * h)) & 15u;
      const uint32_t hi2 = (byte_of3(w.c.x, w.c.y, w.c.z, 8 + 2 * (j & 1) + qq) >> (2 * (2 * h + (j >> 1)))) & 3u;
      const int sc = (int)(lo4 | (hi2 << 4)) - 32;
      int dj = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t x = u4_get(w.a, i);
        const uint32_t hb = (u4_get(w.b, i) >> (4 * h + j)) & 0x01010101u;
        const uint32_t v = j < 3 ? ((x & (0x03030303u << (2 * j))) | (hb << (2 * j + 2)))
                                 : (((x >> 2) & 0x30303030u) | (hb << 6));
        dj = dot4(v, u4_get(a.q[j], i), dj);
      }
      s16 += sc * ((dj << (j == 0 ? 4 : (j == 1 ? 2 : 0))) - 64 * a.bs[j]);
    }
    r.isum = s16 >> 4;
  } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
    // 6-bit (scale, min) of sub-blocks 2q and 2q+1 without a branch: scales bytes
    // 0..11 are header dwords y (A), z (B), w (C); sub-block j < 4 keeps them in
    // A[j] / B[j], j >= 4 splits them over C[j-4] (low bits) and the top bits of
    // A[j-4] / B[j-4] (get_scale_min_k4).
    const uint32_t sh = 16u * (uint32_t)(q & 1);
    const uint32_t hA = w.c.y >> sh, hB = w.c.z >> sh, hC = w.c.w >> sh;
    const bool lo_half = q < 2;
    uint32_t sc0, m0, sc1, m1;
    {
      const uint32_t a0 = hA & 0xffu, b0 = hB & 0xffu, c0 = hC & 0xffu;
      const uint32_t a1 = (hA >> 8) & 0xffu, b1 = (hB >> 8) & 0xffu, c1 = (hC >> 8) & 0xffu;
      sc0 = lo_half ? (a0 & 63u) : ((c0 & 15u) | ((a0 >> 6) << 4));
      m0 = lo_half ? (b0 & 63u) : ((c0 >> 4) | ((b0 >> 6) << 4));
      sc1 = lo_half ? (a1 & 63u) : ((c1 & 15u) | ((a1 >> 6) << 4));
      m1 = lo_half ? (b1 & 63u) : ((c1 >> 4) | ((b1 >> 6) << 4));
    }
    // qs bytes [0,16) low nibbles pair with activations [0,16), bytes [16,32) with
    // [16,32); the high nibbles with [32,48) and [48,64).  Q5_K: bit 2q (low
    // nibbles) / 2q+1 (high) of qh byte l is bit 4 of the value of weight l.
    auto h5 = [&](const uint4 &hv, int i, int bit) -> uint32_t {
      if constexpr (T == T_Q5_K) return ((u4_get(hv, i) >> bit) & 0x01010101u) << 4;
      else return 0u;
    };
    const int bl = 2 * q, bh = 2 * q + 1;
    int dl = 0, dh = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) dl = dot4((u4_get(w.a, i) & 0x0f0f0f0fu) | h5(w.g, i, bl), u4_get(a.q[0], i), dl);
#pragma unroll
    for (int i = 0; i < 4; ++i) dl = dot4((u4_get(w.b, i) & 0x0f0f0f0fu) | h5(w.hh, i, bl), u4_get(a.q[1], i), dl);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dh = dot4(((u4_get(w.a, i) >> 4) & 0x0f0f0f0fu) | h5(w.g, i, bh), u4_get(a.q[2], i), dh);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dh = dot4(((u4_get(w.b, i) >> 4) & 0x0f0f0f0fu) | h5(w.hh, i, bh), u4_get(a.q[3], i), dh);
    r.isum = (int)sc0 * dl + (int)sc1 * dh;
    r.imin = (int)m0 * (a.bs[0] + a.bs[1]) + (int)m1 * (a.bs[2] + a.bs[3]);
  } else if constexpr (T == T_IQ3_XXS) {
    // lds_grid holds the 256 x u32 grid; sub-block 2q + sb: grid-index dwords
    // 2sb, 2sb + 1 of a (two entries = 8 weights per group l), word e.x / e.y
    const uint32_t *g3 = reinterpret_cast<const uint32_t *>(lds_grid);
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const uint32_t aux = sb == 0 ? w.e.x : w.e.y;
      const uint32_t i0 = u4_get(w.a, 2 * sb), i1 = u4_get(w.a, 2 * sb + 1);
      int dsum = 0;
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const uint32_t iw = l < 2 ? i0 : i1;
        const uint32_t g1 = g3[(iw >> (16 * (l & 1))) & 0xffu], g2 = g3[(iw >> (16 * (l & 1) + 8)) & 0xffu];
        const uint64_t m = lds_signs[(aux >> (7 * l)) & 127u];
        const uint32_t mlo = (uint32_t)m, mhi = (uint32_t)(m >> 32);
        const int qi = 2 * (4 * sb + l);  // dword index inside the 64 activations
        dsum = dot4(sign_bytes(g1, mlo), u4_get(a.q[qi >> 2], qi & 3), dsum);
        dsum = dot4(sign_bytes(g2, mhi), u4_get(a.q[(qi + 1) >> 2], (qi + 1) & 3), dsum);
      }
      r.isum += (2 * (int)(aux >> 28) + 1) * dsum;
    }
  } else if constexpr (T == T_IQ4_XS) {
    // lds_grid holds the 16-byte value table; sub-block 2q: bytes of a (low
    // nibbles -> activations [0,16), high -> [16,32)), 2q + 1: bytes of b
    const uint32_t t0 = (uint32_t)lds_grid[0], t1 = (uint32_t)(lds_grid[0] >> 32);
    const uint32_t t2 = (uint32_t)lds_grid[1], t3 = (uint32_t)(lds_grid[1] >> 32);
    int d0 = 0, d1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d0 = dot4(lut16(u4_get(w.a, i) & 0x0f0f0f0fu, t0, t1, t2, t3), u4_get(a.q[0], i), d0);
      d0 = dot4(lut16((u4_get(w.a, i) >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3), u4_get(a.q[1], i), d0);
      d1 = dot4(lut16(u4_get(w.b, i) & 0x0f0f0f0fu, t0, t1, t2, t3), u4_get(a.q[2], i), d1);
      d1 = dot4(lut16((u4_get(w.b, i) >> 4) & 0x0f0f0f0fu, t0, t1, t2, t3), u4_get(a.q[3], i), d1);
    }
    r.isum = iq4_scale(w.e.x, w.e.y, 2 * q) * d0 + iq4_scale(w.e.x, w.e.y, 2 * q + 1) * d1;
  } else if constexpr (T == T_Q6_K) {
    // group g: low nibbles of a (g = 0) / b (g = 1), high nibbles for g = 2, 3;
    // top bits at bit 2g of the qh bytes; value q - 32 folded in as -32 * bsum;
    // signed 8-bit scale of sub-block 8h + 2g + qq = byte qq + 2g of e
    const int qq = q & 1;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 &src = (g & 1) ? w.b : w.a;
      int dg = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = g < 2 ? (u4_get(src, i) & 0x0f0f0f0fu) : ((u4_get(src, i) >> 4) & 0x0f0f0f0fu);
        const uint32_t hi = ((u4_get(w.g, i) >> (2 * g)) & 0x03030303u) << 4;
        dg = dot4(lo | hi, u4_get(a.q[g], i), dg);
      }
      const int sc = (int)(int8_t)((g < 2 ? w.e.x : w.e.y) >> (8 * (qq + 2 * (g & 1))));
      r.isum += sc * (dg - 32 * a.bs[g]);
    }
  } else {  // IQ2_XXS: sub-blocks 2q, 2q+1; words (aux0, aux1) each
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const uint32_t aux0 = sb == 0 ? w.a.x : w.a.z;
      const uint32_t aux1 = sb == 0 ? w.a.y : w.a.w;
      int dsum = 0;
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const uint64_t g = lds_grid[(aux0 >> (8 * l)) & 0xffu];
        const uint64_t m = lds_signs[(aux1 >> (7 * l)) & 127u];
        const uint32_t glo = (uint32_t)g, ghi = (uint32_t)(g >> 32);
        const uint32_t mlo = (uint32_t)m, mhi = (uint32_t)(m >> 32);
        // conditional byte negate: (g ^ m) + (m & 1) per byte (no carries: 8 <= g <= 255)
        const uint32_t vlo = sign_bytes(glo, mlo);
        const uint32_t vhi = sign_bytes(ghi, mhi);
        const int qi = 2 * (4 * sb + l);  // dword index inside the 64 activations
        dsum = dot4(vlo, u4_get(a.q[qi >> 2], qi & 3), dsum);
        dsum = dot4(vhi, u4_get(a.q[(qi + 1) >> 2], (qi + 1) & 3), dsum);
      }
      r.isum += (2 * (int)(aux1 >> 28) + 1) * dsum;
    }
  }
  return r;
}

// Float value of one quarter's contribution to the dot.
template <int T>
__device__ __forceinline__ float quarter_dot(const WSlice &w, int q, const Q8Slice &a, const uint64_t *g,
                                             const uint64_t *sg) {
  const QInt r = quarter_int<T>(w, q, a, g, sg);
  if constexpr (T == T_Q2_K) {
    const float d = h2f((uint16_t)(w.f & 0xffffu)), dmin = h2f((uint16_t)(w.f >> 16));
    return (a.d * d) * (float)r.isum - (a.d * dmin) * (float)r.imin;
  } else if constexpr (T == T_Q3_K) {
    const float d = h2f((uint16_t)(w.c.w & 0xffffu));
    return (a.d * d) * (float)r.isum;
  } else if constexpr (T == T_Q4_K || T == T_Q5_K) {
    const float d = h2f((uint16_t)(w.c.x & 0xffffu)), dmin = h2f((uint16_t)(w.c.x >> 16));
    return (a.d * d) * (float)r.isum - (a.d * dmin) * (float)r.imin;
  } else if constexpr (T == T_Q6_K) {
    return (a.d * h2f((uint16_t)(w.f & 0xffffu))) * (float)r.isum;
  } else if constexpr (T == T_IQ4_XS) {
    return (a.d * h2f((uint16_t)(w.e.x & 0xffffu))) * (float)r.isum;
  } else if constexpr (T == T_IQ3_XXS) {
    return 0.25f * ((a.d * h2f((uint16_t)(w.f & 0xffffu))) * (float)r.isum);
  } else {
    const float d = h2f((uint16_t)(w.f & 0xffffu));
    return 0.125f * ((a.d * d) * (float)r.isum);
  }
}

}  // namespace zm
