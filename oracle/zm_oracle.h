/*
 * zm_oracle.h -- CPU restatement of ggml's routed-expert MUL_MAT_ID path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code: it is the checker that tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg compare the HIP path against.
 *
 * The arithmetic follows ggml (llama.cpp ggml/, pinned by the reference at
 * commit 8baabd53b77d1c48c6ef8d3b620436292f3f6231, "ggml 0.27.0", see
 * /root/reference/patches/README.md:6).  ggml itself is not vendored in the
 * reference, so each function below cites the in-tree file the restatement
 * follows.  Pinning status per function is recorded in zm_oracle.c.
 */
#ifndef ZM_ORACLE_H
#define ZM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZMO_QK_K 256

/* GGUF / ggml type ids (ggml.h enum ggml_type). */
enum {
  ZMO_TYPE_F32 = 0,
  ZMO_TYPE_Q2_K = 10,
  ZMO_TYPE_Q3_K = 11,
  ZMO_TYPE_Q4_K = 12,
  ZMO_TYPE_Q5_K = 13,
  ZMO_TYPE_Q6_K = 14,
  ZMO_TYPE_Q8_K = 15,
  ZMO_TYPE_IQ2_XXS = 16,
  ZMO_TYPE_IQ3_XXS = 18,
  ZMO_TYPE_IQ4_XS = 23,
  ZMO_TYPE_I32 = 26,
};

/* Block layouts: /root/reference/kernels/quant/kquant_matmul.cu:35-39 (Q5_K
 * and Q6_K at :37-38, sizes at backends/cpu/kquant_dequant.hpp:491-492),
 * kernels/quant/iq2_matmul.cu:27, backends/cpu/kernels_cpu.cpp:22-32. */
typedef struct { uint8_t scales[16]; uint8_t qs[64]; uint16_t d, dmin; } zmo_block_q2_K;      /* 84 B  */
typedef struct { uint8_t hmask[32]; uint8_t qs[64]; uint8_t scales[12]; uint16_t d; } zmo_block_q3_K; /* 110 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } zmo_block_q4_K;     /* 144 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } zmo_block_q5_K; /* 176 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } zmo_block_q6_K;   /* 210 B */
typedef struct { uint16_t d; uint16_t qs[32]; } zmo_block_iq2_xxs;
typedef struct { uint16_t d; uint16_t scales_h; uint8_t scales_l[4]; uint8_t qs[128]; } zmo_block_iq4_xs; /* 136 B */
typedef struct { uint16_t d; uint8_t qs[96]; } zmo_block_iq3_xxs; /* 98 B: grid indices[64] | scales+signs u32[8] */                            /* 66 B  */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } zmo_block_q8_K;                /* 292 B */

/* ---- helpers ---- */
float zmo_fp16_to_fp32(uint16_t h);
uint16_t zmo_fp32_to_fp16(float f);
size_t zmo_row_size(int type, int64_t n); /* bytes of one row of n weights */
int zmo_nearest_int(float f);
float zmo_expf(float x);                  /* shared exp used by both router implementations */
void zmo_fill_normal(uint64_t seed, float mean, float sd, float *out, int64_t n);

/* IQ2_XXS lookup tables.  The sign table is closed form; the grid is a runtime
 * table (ggml's values are not in the reference tree).  zmo_iq2xxs_grid()
 * returns the table in use; zmo_set_iq2xxs_grid() replaces it. */
const uint64_t *zmo_iq2xxs_grid(void);
void zmo_set_iq2xxs_grid(const uint64_t grid[256]);
void zmo_iq2xxs_standin_grid(uint64_t grid[256]);
uint8_t zmo_ksigns_iq2xs(int i);

/* IQ4_XS 16-entry non-linear value table (ggml's kvalues_iq4nl).  Its values
 * are not in the reference tree; the default is ggml's published table and
 * zmo_set_iq4nl_table() replaces it. */
const int8_t *zmo_iq4nl_table(void);

/* IQ3_XXS grid (256 x u32, four byte values each; ggml's iq3xxs_grid, not in
 * the reference tree): a stand-in by default, replaced by zmo_set_iq3xxs_grid. */
const uint32_t *zmo_iq3xxs_grid(void);
void zmo_set_iq3xxs_grid(const uint32_t grid[256]);
void zmo_iq3xxs_standin_grid(uint32_t grid[256]);
void zmo_set_iq4nl_table(const int8_t table[16]);

/* ---- quantizers (valid blocks; bit identity with ggml's quantizer bytes is unpinned) ---- */
void zmo_quantize_row_q8_K(const float *x, zmo_block_q8_K *y, int64_t k);
void zmo_quantize_row_q2_K(const float *x, zmo_block_q2_K *y, int64_t k);
void zmo_quantize_row_q3_K(const float *x, zmo_block_q3_K *y, int64_t k);
void zmo_quantize_row_q4_K(const float *x, zmo_block_q4_K *y, int64_t k);
void zmo_quantize_row_q5_K(const float *x, zmo_block_q5_K *y, int64_t k);
void zmo_quantize_row_q6_K(const float *x, zmo_block_q6_K *y, int64_t k);
void zmo_quantize_row_iq2_xxs(const float *x, zmo_block_iq2_xxs *y, int64_t k);
void zmo_quantize_row_iq4_xs(const float *x, zmo_block_iq4_xs *y, int64_t k);
void zmo_quantize_row_iq3_xxs(const float *x, zmo_block_iq3_xxs *y, int64_t k);
/* quantize `rows` rows of n floats of `type` into dst (rows * row_size bytes) */
void zmo_quantize_rows(int type, const float *x, void *dst, int64_t rows, int64_t n);

/* ---- dequant ---- */
void zmo_dequantize_row(int type, const void *src, float *y, int64_t n);

/* ---- dots (ggml x86 float order where pinned) ---- */
float zmo_vec_dot_q8_K(int type, int n, const void *x, const zmo_block_q8_K *y);
/* Per-super-block integer parts: for K-quants isum = sum_j sc_j * dot_j and
 * imin = sum_j m_j * bsum_j (Q2_K/Q4_K/Q5_K; 0 for Q3_K and Q6_K, whose
 * values are signed: q - 4 for a clear Q3_K high bit, q6 - 32); IQ2_XXS isum = sum_sub
 * (2ls+1) * dot.  Written into isum[nb], imin[nb]. */
void zmo_block_dots(int type, int n, const void *x, const zmo_block_q8_K *y, int32_t *isum, int32_t *imin);

/* ---- the op ---- */
typedef struct {
  int type;
  int64_t ne[4];
  size_t nb[4];
  void *data;
} zmo_tensor;

/* ggml_compute_forward_mul_mat_id semantics (patches/ggml/0002...:46-58):
 * dst[:, id, t] = W[ids[id,t]] . src1[:, id % ne11, t]; negative id -> zeros.
 * nthreads > 1 parallelises over output rows (results identical). */
int zmo_mul_mat_id(const zmo_tensor *src0, const zmo_tensor *src1, const zmo_tensor *ids, zmo_tensor *dst,
                   int nthreads);

/* ---- router / bucketing / combine ---- */
enum { ZMO_GATING_SOFTMAX = 0, ZMO_GATING_SIGMOID = 1, ZMO_GATING_SQRT_SOFTPLUS = 2 };
typedef struct {
  int gating;
  int n_experts;
  int topk;
  int n_groups;
  int n_groups_used;
  int weights_norm;
  float weights_scale;
} zmo_router_spec;

/* logits [S, E] (ggml [E, S]); logit_bias [E] added to logits before gating
 * (may be NULL); sel_bias [E] added to probs for selection only (may be NULL);
 * route_map [E] int32 slot table (may be NULL, -1 = not resident) with
 * route_mask [E] (may be NULL -> 1 where route_map >= 0).
 * Outputs ids [S, K] and weights [S, K]. */
void zmo_router(const zmo_router_spec *spec, const float *logits, const float *logit_bias, const float *sel_bias,
                int S, int32_t *ids, float *weights);
void zmo_apply_slot_table(const int32_t *route_map, const float *route_mask, int S, int K, int32_t *ids,
                          float *weights);

/* counts[E], offs[E+1], pairs[S*K] (flat s*K+k, sorted by expert, token-major
 * stable). Negative ids are not bucketed. Returns number of bucketed pairs. */
int zmo_bucket(const int32_t *ids, int S, int K, int E, int32_t *counts, int32_t *offs, int32_t *pairs);

void zmo_swiglu(const float *g, const float *u, float *out, int64_t n);

/* Full routed layer (moe_routed::expert_ffn + ggml_mul + sum_topk):
 * x [S, H] f32, ids/weights [S, K] from zmo_router, weights ggml-layout
 * gate/up [H, F, E], down [F, H, E].  Optional shared expert (all tokens,
 * weight 1) added after the top-k sum.  out [S, H]. */
typedef struct {
  int H, F, E, K, S;
  int type_gate, type_up, type_down;
  const void *w_gate, *w_up, *w_down;
  /* shared expert (may be NULL) */
  int F_shared;
  int type_shared;
  const void *ws_gate, *ws_up, *ws_down;
} zmo_moe_desc;
void zmo_moe_forward(const zmo_moe_desc *d, const float *x, const int32_t *ids, const float *weights, float *out,
                     int nthreads);
/* CPU baseline: the same layer with AVX-512 VNNI dots where the host has
 * them (Q2_K, Q3_K), ggml's two-region thread structure; bit-identical to
 * zmo_moe_forward (no shared expert). */
int zmo_cpu_has_avx512(void);
float zmo_vec_dot_q8_K_fast(int type, int n, const void *x, const zmo_block_q8_K *y);
void zmo_moe_forward_fast(const zmo_moe_desc *d, const float *x, const int32_t *ids, const float *weights,
                          float *out, int nthreads);

/* Router GEMV: logits[s][e] = sum_i W[e][i] x[s][i], W [E][H] f32 (ggml [H, E]). */
void zmo_router_gemv(const float *W, const float *x, int H, int E, int S, float *logits);

#ifdef __cplusplus
}
#endif
#endif
