/*
 * zeromoe.h -- C ABI of libzeromoe_hip.so, the MI355X (gfx950) routed-expert
 * MUL_MAT_ID path.
 *
 * Every entry point takes plain pointers and sizes.  Device pointers are HIP
 * device memory; `stream` is a hipStream_t (NULL = the legacy default
 * stream).  Work is stream-ordered; nothing synchronises unless stated.
 * Return convention: int entry points return 0 on success and a negative
 * code on a rejected call (zm_last_error() says why); zm_mul_mat_id follows
 * the ggml hook convention instead (1 = handled / supported, 0 = declined).
 *
 * Each declaration cites the reference interface it replaces
 * (/root/reference/<file>:<line>).
 */
#ifndef ZEROMOE_H
#define ZEROMOE_H

#include <stddef.h>
#include <stdint.h>
#ifndef __cplusplus
#include <stdbool.h>
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ggml tensor descriptor: type (ggml_type id), ne[] (elements, fastest
 * first), nb[] (byte strides), data (device pointer).  The subset of
 * struct ggml_tensor that ggml_cuda_mul_mat_id hands to its quant hook
 * (patches/ggml/0010-...:9-27). */
typedef struct zm_tensor {
  int32_t type;
  int64_t ne[4];
  size_t nb[4];
  void *data;
} zm_tensor;

/* ggml_type ids used on this path */
enum {
  ZM_TYPE_F32 = 0,
  ZM_TYPE_Q2_K = 10,
  ZM_TYPE_Q3_K = 11,
  ZM_TYPE_Q4_K = 12,
  ZM_TYPE_Q5_K = 13,
  ZM_TYPE_Q6_K = 14,
  ZM_TYPE_Q8_K = 15,
  ZM_TYPE_IQ2_XXS = 16,
  ZM_TYPE_IQ3_XXS = 18,
  ZM_TYPE_IQ4_XS = 23,
  ZM_TYPE_I32 = 26,
};

/* ---------------------------------------------------------------- library */

/* Per-device set-up of the current device (IQ2 tables).  Idempotent.
 * Replaces init_iq2_grids (kernels/quant/iq2_matmul.cu:55-70). */
int zm_init(void);
const char *zm_last_error(void);
const char *zm_version(void);

/* Load the IQ2_XXS grid (256 x u64, ggml's iq2xxs_grid) for the current
 * device.  Without a call the built-in stand-in grid is used.
 * Replaces the grid copy of init_iq2_grids (iq2_matmul.cu:60). */
int zm_set_iq2xxs_grid(const uint64_t grid[256]);
void zm_iq2xxs_builtin_grid(uint64_t grid[256]);
/* Load the IQ4_XS value table (16 x i8, ggml's kvalues_iq4nl) for the current
 * device.  The built-in default is ggml's published table; its values are
 * not in the reference tree.  Replaces init_iq4xs_table
 * (kernels/quant/iq4xs_matmul.cu:41-49). */
int zm_set_iq4nl_table(const int8_t table[16]);
void zm_iq4nl_builtin_table(int8_t table[16]);
/* Load the IQ3_XXS grid (256 x u32, ggml's iq3xxs_grid) for the current
 * device.  Without a call a stand-in grid is used.  Replaces the grid copy
 * of init_iq3_grids (kernels/quant/iq3_matmul.cu:66-78). */
int zm_set_iq3xxs_grid(const uint32_t grid[256]);
void zm_iq3xxs_builtin_grid(uint32_t grid[256]);

/* Capability flags the graph builders probe before emitting negative
 * (inactive) expert ids: both are 1, the HIP path skips id < 0 in decode and
 * in batched prefill.  Replace ggml_cpu_mul_mat_id_negative_skip and
 * ggml_cuda_mul_mat_id_negative_skip_batched
 * (backends/ggml/mmid_route_skip.hpp:22,41). */
int zm_mul_mat_id_negative_skip(void);
int zm_mul_mat_id_negative_skip_batched(void);

/* ---------------------------------------------------------------- the op */

/* GGML_OP_MUL_MAT_ID hook: dst[:, id, t] = W[ids[id, t]] . src1[:, id % ne11, t]
 * with src1 quantized to Q8_K (ggml CPU semantics), id < 0 -> zero row,
 * id >= n_experts -> NaN row.
 *   src0: Q2_K / Q3_K / Q4_K / Q5_K / Q6_K / IQ2_XXS / IQ3_XXS / IQ4_XS [I, O, E] (row-contiguous)
 *   src1: F32 [I, ne11, S], ne11 == 1 or n_ids;  ids: I32 [n_ids, S]
 *   dst : F32 [O, n_ids, S]
 * execute = 0 is a pure capability query; execute = 1 launches on `stream`.
 * Returns 1 when handled/supported, 0 when declined.
 * Like the reference hook it allocates nothing and borrows every tensor
 * (kquant_matmul.cu:644-646): its scratch (Q8_K rows of src1, the bucket
 * arrays) lives in a caller-owned workspace bound to the stream with
 * zm_mul_mat_id_set_workspace.  The query (any stream, ggml passes NULL)
 * accepts a shape only if the smallest workspace bound on the current device
 * holds it; an execute call uses the workspace bound to its stream and
 * declines when there is none or it is too small.  Calls on one stream are
 * stream-ordered; streams with workspaces of their own never share scratch.
 * Launches only (kernels and one device-to-device copy of ids): safe under
 * HIP-graph capture once the workspace is bound.
 * Replaces native_f32_quant_hook / zeromoe_install_f32_quant_graph_hook
 * (kernels/quant/kquant_matmul.cu:702-761, patches/ggml/0010-...:9-27). */
int zm_mul_mat_id(const zm_tensor *src0, const zm_tensor *src1, const zm_tensor *ids, zm_tensor *dst, void *stream,
                  int execute);
/* Workspace bytes zm_mul_mat_id needs for this shape (0: shape declined).
 * The reference hook needs none (its FP32 kernels read src1 directly); this
 * path stages Q8_K activations and expert buckets.  Sizing call for the
 * workspace of zm_mul_mat_id_set_workspace. */
size_t zm_mul_mat_id_workspace_size(const zm_tensor *src0, const zm_tensor *src1, const zm_tensor *ids,
                                    const zm_tensor *dst);
/* Bind a caller-owned device buffer (256-byte aligned, `bytes` long) as
 * zm_mul_mat_id's workspace for (current device, stream); NULL unbinds.  At
 * most 64 bindings.  The caller keeps the buffer alive and unmodified while
 * work that uses it is queued.  The counterpart of the scratch a ggml backend
 * context owns per stream (the reference hook's caller,
 * patches/ggml/0010-...:57-61, passes ctx.stream()). */
int zm_mul_mat_id_set_workspace(void *stream, void *workspace, size_t bytes);
/* zm_mul_mat_id with no workspace at all, for callers that cannot allocate
 * or bind memory (code under HIP-graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Its scratch is a
 * 16 MiB device array compiled into the library (one per GPU, held until the
 * process ends); shapes that need more (zm_mul_mat_id_workspace_size) are
 * declined with an error.  zm_init must have run on the device (it looks up
 * the array's address); the call itself only launches.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race and must be serialised by the caller.  Same arguments,
 * semantics and return convention as zm_mul_mat_id. */
int zm_mul_mat_id_static(const zm_tensor *src0, const zm_tensor *src1, const zm_tensor *ids, zm_tensor *dst,
                         void *stream, int execute);
/* Count of executed zm_mul_mat_id launches (kquant_matmul.cu:762-764). */
uint64_t zm_mul_mat_id_launches(void);

/* ---------------------------------------------------------------- pieces */

/* f32 rows -> ggml block_q8_K rows (292 B per 256), bit-exact to ggml's
 * quantize_row_q8_K.  Replaces the from_float step of
 * ggml_compute_forward_mul_mat_id (patches/ggml/0002-...:18-45). */
int zm_quantize_q8_K(const float *x, int64_t rows, int64_t n, void *y, void *stream);

/* Router: gating (0 softmax, 1 sigmoid, 2 sqrt-softplus), optional grouped
 * selection, top-k (descending, lowest index on ties), weight norm/scale,
 * optional slot table.  logits [S][E]; ids/weights [S][K].
 * Replaces moe_routed::gate_probs/select_ids/route_weights
 * (models/graph/moe_routed_ggml.hpp:52-141) and make_branch_inputs
 * (backends/ggml/moe_partial_route_ggml.hpp:21-35). */
typedef struct zm_router_spec {
  int32_t gating;
  int32_t n_experts;
  int32_t topk;
  int32_t n_groups;
  int32_t n_groups_used;
  int32_t weights_norm;
  float weights_scale;
} zm_router_spec;
int zm_router(const zm_router_spec *spec, const float *logits, const float *logit_bias, const float *sel_bias,
              const int32_t *route_map, const float *route_mask, int S, int32_t *ids, float *weights, void *stream);

/* Stable bucketing of the S*K (token, slot) pairs by expert: counts[E],
 * offs[E+1] (exclusive scan), pairs[S*K] (flat s*K+k, token-major within an
 * expert), active[E] (experts with count > 0, ascending), n_active[1].
 * Negative ids are not bucketed.  E <= 512.
 * Replaces the CSR build of core/batched_dispatch_pipeline.cpp:1181-1202. */
int zm_bucket(const int32_t *ids, int S, int K, int E, int32_t *counts, int32_t *offs, int32_t *pairs,
              int32_t *active, int32_t *n_active, void *stream);

/* Debug/verification: per-super-block integer parts of one weight row
 * against f32 activations quantized to Q8_K: isum[b], imin[b] as defined in
 * oracle/zm_oracle.h (zmo_block_dots).  Both device dot paths (the bucketed
 * GEMV's and the fused decode kernel's) compute every block; where they
 * disagree isum[b] is INT32_MIN.  Not on the hot path. */
int zm_block_dots(int type, const void *w_row, const float *x, int n, int32_t *isum, int32_t *imin, void *stream);

/* ---------------------------------------------------------------- routed layer */

/* One routed MoE FFN layer (moe_routed::expert_ffn + ggml_mul + sum_topk,
 * models/graph/moe_routed_ggml.hpp:166-214, models/graph/moe_block.hpp:86-105,
 * plus the shared-expert add of moe_block.hpp:201-202).
 * Weights in ggml layout, contiguous: gate/up [H, F, n_slots], down
 * [F, H, n_slots].  route_map (optional) maps the router's n_experts ids to
 * weight slots (-1 = not resident: route skipped, weight masked). */
typedef struct zm_moe_layer {
  int32_t H, F;
  int32_t n_slots;          /* experts held by the weight tensors */
  zm_router_spec router;    /* router.n_experts = E of the router, router.topk = K */
  int32_t type_gate, type_up, type_down;
  const void *w_gate, *w_up, *w_down;
  const float *router_w;    /* optional fp32 router [E][H] (ggml [H, E]); NULL: logits are an input */
  const float *logit_bias;  /* optional [E] */
  const float *sel_bias;    /* optional [E] */
  const int32_t *route_map; /* optional [E] */
  const float *route_mask;  /* optional [E] */
  int32_t F_shared, type_shared; /* shared expert (F_shared = 0: none) */
  const void *ws_gate, *ws_up, *ws_down;
} zm_moe_layer;

/* Workspace bytes for S tokens.  The workspace must be zero-filled once
 * before its first use (it holds the decode kernel's sync words, which every
 * call leaves at zero); calls sharing one workspace must not overlap. */
size_t zm_moe_workspace_size(const zm_moe_layer *layer, int S);
/* Synchronises `stream` and returns (then clears) the decode kernel's error
 * word for this workspace: 0 = ok, 1 = a bounded wait expired. */
int zm_moe_status(const zm_moe_layer *layer, int S, void *workspace, void *stream);
/* x [S][H] f32; logits [S][E] (ignored when router_w is set); out [S][H];
 * ids_out / weights_out [S][K] (optional): the routes after the slot table.
 * workspace: device memory of zm_moe_workspace_size() bytes. */
int zm_moe_forward(const zm_moe_layer *layer, const float *x, const float *logits, int S, float *out,
                   int32_t *ids_out, float *weights_out, void *workspace, size_t workspace_size, void *stream);

/* ---------------------------------------------------------------- FP32-activation path
 *
 * Quantized weights times f32 activations, no Q8_K step: the reference's CUDA
 * executor semantics, not ggml's CPU ones.  Weight rows are I/256 super-blocks
 * (Q2_K / Q3_K / Q4_K / Q5_K / Q6_K / IQ2_XXS / IQ3_XXS / IQ4_XS); x must be 16-byte aligned.  Accumulation is
 * fp32 in a fixed order (deterministic; not the reference's order).  The void
 * launchers keep the reference's signatures; a rejected call launches nothing
 * and leaves the reason in zm_last_error(). */

/* y[S][O] = x[S][I] . dequant(W[O][I])^T on the legacy default stream / on
 * `stream`.  Replace launch_q2_K_matmul ... launch_iq2_xxs_matmul
 * (backends/cuda/cuda_kernel_dispatcher.cpp:17-28; kernels/quant/kquant_matmul.cu:575-599,
 * kernels/quant/iq2_matmul.cu:180-183) and the _stream variants. */
void launch_q2_K_matmul(float *y, const float *x, const void *w, int S, int I, int O);
void launch_q2_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
void launch_q3_K_matmul(float *y, const float *x, const void *w, int S, int I, int O);
void launch_q3_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
void launch_q4_K_matmul(float *y, const float *x, const void *w, int S, int I, int O);
void launch_q4_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
void launch_iq2_xxs_matmul(float *y, const float *x, const void *w, int S, int I, int O);
/* Q5_K / Q6_K: replace launch_q5_K_matmul / launch_q6_K_matmul
 * (kernels/quant/kquant_matmul.cu:615-629, declared at
 * backends/cuda/cuda_kernel_dispatcher.cpp:23-26); the _stream variants have
 * no reference counterpart and exist for symmetry with the other types. */
void launch_q5_K_matmul(float *y, const float *x, const void *w, int S, int I, int O);
void launch_q5_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
void launch_q6_K_matmul(float *y, const float *x, const void *w, int S, int I, int O);
void launch_q6_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
/* IQ4_XS: replaces launch_iq4_xs_matmul (kernels/quant/iq4xs_matmul.cu:137-140,
 * declared at backends/cuda/cuda_kernel_dispatcher.cpp:37). */
void launch_iq4_xs_matmul(float *y, const float *x, const void *w, int S, int I, int O);
/* IQ3_XXS: replaces launch_iq3_xxs_matmul (kernels/quant/iq3_matmul.cu:159-162). */
void launch_iq3_xxs_matmul(float *y, const float *x, const void *w, int S, int I, int O);
void launch_iq3_xxs_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
void launch_iq4_xs_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
/* y[g][O] = x[g][I] . dequant(W_g)^T for g < groups, W_g at byte
 * g * group_stride_bytes (a multiple of 176), legacy default stream; returns
 * false (launching nothing) on a rejected shape.  Replaces
 * launch_q5_K_matmul_grouped (kernels/quant/kquant_matmul.cu:607-614). */
bool launch_q5_K_matmul_grouped(float *y, const float *x, const void *w, int groups, size_t group_stride_bytes,
                                 int I, int O);
void launch_iq2_xxs_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream);
/* The same by type id, returning 0 / -1.  Replaces CudaKernelDispatcher::matmul
 * (backends/cuda/cuda_kernel_dispatcher.cpp:109-189) for these eight types. */
int zm_f32_matmul(int type, float *y, const float *x, const void *w, int S, int I, int O, void *stream);

/* FP32 quant-matmul hook with the acceptance rules of native_f32_quant_hook
 * (kernels/quant/kquant_matmul.cu:702-756), widened from Q2_K/Q3_K to the four
 * types: MUL_MAT_ID (ids set; id < 0 -> 0 row, id >= ne2 -> NaN row), plain
 * MUL_MAT (ids NULL, 2-D) and the grouped form (ids NULL, ne2 > 1: matrix g
 * times x[:, :, g]).  Same conventions as zm_mul_mat_id (1 handled, 0
 * declined; execute = 0 is a pure query); also counted by
 * zm_mul_mat_id_launches. */
int zm_mul_mat_id_f32(const zm_tensor *src0, const zm_tensor *src1, const zm_tensor *ids, zm_tensor *dst,
                      void *stream, int execute);

/* prod[i] = clamp(silu(gate) * up) (fused = 0) or silu(min(gate, c)) *
 * clamp(up) (fused = 1), clamps applied when clamp > 0; d_bad (device, 2 x
 * int, optional) += NaN count, Inf count of (gate, up).
 * Replaces launch_expert_swiglu (kernels/math/expert_activation.cu:61-70). */
void launch_expert_swiglu(float *prod, const float *gate, const float *up, int n, float clamp, int fused, int *d_bad,
                          void *stream);
/* dst[tok[i]][:] += w[i] * src[i][:] for i < n (w NULL: += src), rows with
 * tok outside [0, S) skipped; the tok of one call must be distinct.
 * Replace launch_expert_scatter_accum / launch_expert_scatter_add
 * (kernels/math/expert_accum.cu:39-60). */
void launch_expert_scatter_accum(const float *src, const int *tok, const float *w, float *dst, int n, int D, int S,
                                 void *stream);
void launch_expert_scatter_add(const float *src, const int *tok, float *dst, int n, int D, int S, void *stream);
/* Router post-processing for S tokens: logits [S][E] overwritten with the
 * gated probabilities (softmax 0 / sigmoid 1 / sqrt-softplus 2), the chosen
 * ones then set to -FLT_MAX; ids/weights [S][K]: top-K of prob + bias (bias
 * optional), ties to the lower index, weight = unbiased prob, optional
 * normalisation 1/max(sum, 2^-14) and scale (when != 0).  E <= 4096, K <= 64.
 * Replaces launch_glm5next_router_topk (kernels/models/glm5next_router.cu:95-105). */
void launch_glm5next_router_topk(float *logits, const float *bias, int32_t *ids, float *weights, int S, int n_experts,
                                 int topk, int gating_func, int normalize, float weight_scale, void *stream);

/* Per-expert executor over one device slab laid out [gate | up | down]
 * (up / down at byte offsets from the gate), f32 activations.
 * Replaces GpuExpertScratch (memory/scratch_buffers.hpp:14-34) and
 * expert_ffn_gpu_issue / _finish_stage1 / _finish_stage2
 * (core/gpu_expert_executor.hpp:42-58, core/gpu_expert_executor.cpp:213-533).
 * The caller owns the struct (zero-initialised before first use); ensure()
 * grows its buffers monotonically; release() frees them. */
typedef struct zm_expert_scratch {
  int32_t *d_bad;   /* 2 counters: NaN, Inf seen by the SwiGLU */
  float *d_x, *d_gate, *d_up, *d_prod, *d_down;
  size_t cap_sd, cap_si; /* capacity in floats: S*D and S*F */
  int32_t device_id;
} zm_expert_scratch;
int zm_expert_scratch_ensure(zm_expert_scratch *s, int S, int D, int F, int device);
void zm_expert_scratch_release(zm_expert_scratch *s);
/* x (host [S][D], uploaded on `stream`) or device_x (device [S][D]) ->
 * d_gate, d_up [S][F] on the current device. */
int zm_expert_ffn_issue(zm_expert_scratch *s, const void *slab, size_t up_offset, int gate_type, int up_type,
                        const float *host_x, int S, int D, int F, const float *device_x, void *stream);
/* d_prod = SwiGLU(d_gate, d_up) (counting non-finite inputs), d_down = d_prod . W_down^T. */
int zm_expert_ffn_finish_stage1(zm_expert_scratch *s, const void *slab, size_t down_offset, int down_type, int S,
                                int D, int F, float swiglu_clamp, int fused_clamp, void *stream);
/* d_down -> host_out [S][D]; synchronises `stream`. */
int zm_expert_ffn_finish_stage2(zm_expert_scratch *s, float *host_out, int S, int D, void *stream);
/* Read (and optionally reset) the NaN / Inf counters. */
int zm_expert_bad_counts(zm_expert_scratch *s, int32_t counts[2], int reset);

/* ---------------------------------------------------------------- expert records
 *
 * Device-local unpack of expert-major transfer records [gate | up | down]
 * (record i at src + i*src_stride; gate_bytes, up_bytes, down_bytes each)
 * into the three planar per-expert tensors: record i's gate bytes go to
 * gate + e*gate_stride, and likewise for up and down, where e = i
 * (launch_ggml_moe_unpack) or e = dst_slots[i] (_scatter; a negative slot
 * skips the record).  Bytes outside each part are not written; two records
 * with the same slot race.  Stream-ordered; returns a hipError_t value: 0 on
 * success, hipErrorInvalidValue (1) for a NULL pointer or count <= 0.
 * Replace launch_ggml_moe_unpack / launch_ggml_moe_unpack_scatter
 * (kernels/math/ggml_moe_pack.cu:127-179; called from
 * backends/ggml/ggml_moe_transfer_manager.cpp:395,598,725,859). */
int launch_ggml_moe_unpack(const void *src, void *gate, void *up, void *down, int count, size_t src_stride,
                           size_t gate_bytes, size_t up_bytes, size_t down_bytes, size_t gate_stride,
                           size_t up_stride, size_t down_stride, void *stream);
int launch_ggml_moe_unpack_scatter(const void *src, void *gate, void *up, void *down, const int32_t *dst_slots,
                                   int count, size_t src_stride, size_t gate_bytes, size_t up_bytes,
                                   size_t down_bytes, size_t gate_stride, size_t up_stride, size_t down_stride,
                                   void *stream);

/* Debug: copy the last decode launch's phase timestamps (8 per workgroup,
 * wall_clock64 ticks; recorded only when ZEROMOE_TRACE=1) into host[n].
 * Synchronises the device.  Returns the count copied. */
int zm_debug_trace(uint64_t *host, int n);

/* ---------------------------------------------------------------- CPU lane (hot/cold split) */

/* The cold branch of a layer whose experts are split between VRAM (hot) and
 * host memory (cold): the cold experts run on the host cores while the GPU
 * computes the hot ones.  Replaces EarlyReadyLane
 * (models/graph/early_ready_lane.hpp:75-211) with the branch semantics of
 * backends/ggml/moe_partial_route_ggml.hpp:21-60: a route (token s, slot k) of
 * expert e is cold when route_map[e] >= 0 (its host slot); its weight is
 * w * route_mask[e] (1 when route_mask is NULL).  The caller runs the hot
 * branch itself (zm_moe_forward with the hot slot table) and the lane adds
 * sum over cold routes (k ascending) of w' * expert(x) to its output.
 * Weights are ggml expert tensors in host memory: gate/up [n_slots][F][row(H)],
 * down [n_slots][H][row(F)], Q2_K, Q3_K or Q4_K. */
typedef struct zm_cold_lane zm_cold_lane;
typedef struct zm_cold_lane_desc {
  int32_t H, F, n_experts, topk;
  int32_t type_gate, type_up, type_down;
  const void *w_gate, *w_up, *w_down; /* host memory, borrowed */
  int32_t n_slots;                     /* host expert slots */
  const int32_t *route_map;            /* [n_experts] expert -> host slot or -1 (copied) */
  const float *route_mask;             /* [n_experts] or NULL (copied) */
  int32_t max_tokens;                  /* tokens per call */
  int32_t n_threads;                   /* host threads of the lane */
  int32_t scalar;                      /* 1: scalar dots even on AVX-512 hosts (same bits) */
} zm_cold_lane_desc;
typedef struct zm_cold_lane_stats {
  int64_t fork_ns, compute_begin_ns, compute_end_ns, merge_ns; /* steady-clock times of the last call */
  int32_t vectorized;                                          /* AVX-512 VNNI dots in use */
} zm_cold_lane_stats;
/* Create (NULL on a bad descriptor or unsupported types, zm_last_error says
 * why).  Host memory only; device buffers and the lane thread are set up on
 * the first fork.  Replaces EarlyReadyLane::prepare (early_ready_lane.hpp:196). */
zm_cold_lane *zm_cold_lane_create(const zm_cold_lane_desc *desc);
void zm_cold_lane_destroy(zm_cold_lane *lane);
/* Fork: stream-ordered copies of x [S][H], ids [S][topk] (router expert ids)
 * and weights [S][topk] (device pointers) into the lane's pinned buffers; the
 * lane thread starts as soon as they land, while the caller queues the hot
 * GPU work.  The fork of early_ready_lane.hpp:3-10. */
int zm_cold_lane_fork(zm_cold_lane *lane, const float *x, const int32_t *ids, const float *weights, int S,
                      void *stream);
/* Merge: waits (host) for the lane's result, uploads it on the lane's own
 * stream and makes `stream` add it to out [S][H] (device).  The merge of
 * early_ready_lane.hpp:7-9 / moe_block.hpp:182-184. */
int zm_cold_lane_merge(zm_cold_lane *lane, float *out, int S, void *stream);
/* The lane's computation on host buffers, synchronously (no device): out [S][H]
 * = the cold branch.  For callers without a GPU stream and for tests. */
int zm_cold_lane_compute_host(zm_cold_lane *lane, const float *x, const int32_t *ids, const float *weights, int S,
                              float *out);
int zm_cold_lane_get_stats(const zm_cold_lane *lane, zm_cold_lane_stats *stats);

#ifdef __cplusplus
}
#endif
#endif
