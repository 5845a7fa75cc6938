// zm_exec.hip -- C ABI of the FP32-activation expert path: the per-type
// launchers (launch_<type>_matmul[_stream]), the FP32 MUL_MAT_ID hook, the
// SwiGLU / scatter-accumulate / GLM5Next router helpers under the reference's
// own symbol names, and the per-expert executor stages over a caller-owned
// scratch.  Declared in include/zeromoe.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>

#include "../../include/zeromoe.h"
#include "zm_f32.hpp"
#include "zm_host.hpp"

using namespace zm;

namespace {

bool f32_type(int t) {
  return t == T_Q2_K || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_IQ2_XXS || t == T_IQ3_XXS ||
         t == T_IQ4_XS;
}

template <int T>
void launch_mm_t(const F32MMArgs &a, int n_route, hipStream_t st) {
  const unsigned gx = (unsigned)((a.O + 4 * F32_RPW - 1) / (4 * F32_RPW));
  if (a.ids || a.n_tok == 1) {
    hipLaunchKernelGGL((k_f32_mm<T, 1>), dim3(gx, (unsigned)a.n_tok, (unsigned)n_route), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL((k_f32_mm<T, 4>), dim3(gx, (unsigned)((a.n_tok + 3) / 4), (unsigned)n_route), dim3(256), 0,
                       st, a);
  }
}

// a validated F32MMArgs; n_route <= 65535, n_tok <= 65535 (* 4 without ids)
int launch_mm(int type, F32MMArgs a, int n_route, hipStream_t st) {
  if ((type == T_IQ2_XXS || type == T_IQ3_XXS || type == T_IQ4_XS) && device_table(type, &a.grid)) return -1;
  switch (type) {
  case T_Q2_K: launch_mm_t<T_Q2_K>(a, n_route, st); break;
  case T_Q3_K: launch_mm_t<T_Q3_K>(a, n_route, st); break;
  case T_Q4_K: launch_mm_t<T_Q4_K>(a, n_route, st); break;
  case T_Q5_K: launch_mm_t<T_Q5_K>(a, n_route, st); break;
  case T_Q6_K: launch_mm_t<T_Q6_K>(a, n_route, st); break;
  case T_IQ4_XS: launch_mm_t<T_IQ4_XS>(a, n_route, st); break;
  case T_IQ3_XXS: launch_mm_t<T_IQ3_XXS>(a, n_route, st); break;
  case T_IQ2_XXS: launch_mm_t<T_IQ2_XXS>(a, n_route, st); break;
  default: return fail("unsupported weight type %d", type);
  }
  HIP_OK(hipGetLastError());
  return 0;
}

// y[S,O] = x[S,I] . dequant(W[O,I])^T
int plain_matmul(int type, float *y, const float *x, const void *w, int S, int I, int O, hipStream_t st) {
  if (!y || !x || !w) return fail("launch_matmul: null pointer");
  if (S <= 0 || O <= 0) return 0;
  if (I <= 0 || I % QK) return fail("launch_matmul: I=%d is not a positive multiple of 256", I);
  if ((uintptr_t)x & 15) return fail("launch_matmul: x must be 16-byte aligned");
  if ((S + 3) / 4 > 65535 && S > 1) return fail("launch_matmul: S=%d too large", S);
  F32MMArgs a{};
  a.w = (const uint8_t *)w;
  a.w_row = (size_t)(I / QK) * block_bytes(type);
  a.x = x;
  a.x_tok = (size_t)I;
  a.x_routes = 1;
  a.y = y;
  a.y_tok = (size_t)O;
  a.I = I;
  a.O = O;
  a.n_tok = S;
  return launch_mm(type, a, 1, st);
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- per-type launchers

void launch_q2_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_Q2_K, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_q2_K_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_Q2_K, y, x, w, S, I, O, nullptr);
}
void launch_q3_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_Q3_K, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_q3_K_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_Q3_K, y, x, w, S, I, O, nullptr);
}
void launch_q4_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_Q4_K, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_q4_K_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_Q4_K, y, x, w, S, I, O, nullptr);
}
void launch_q5_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_Q5_K, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_q5_K_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_Q5_K, y, x, w, S, I, O, nullptr);
}
void launch_q6_K_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_Q6_K, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_q6_K_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_Q6_K, y, x, w, S, I, O, nullptr);
}
// y[g][O] = x[g][I] . dequant(W_g)^T, W_g at g * group_stride_bytes; false when
// the shape is rejected (the caller then loops over the groups itself)
bool launch_q5_K_matmul_grouped(float *y, const float *x, const void *w, int groups, size_t group_stride_bytes, int I,
                                int O) {
  if (!y || !x || !w || groups <= 0 || groups > 65535 || O <= 0 || I <= 0 || I % QK || ((uintptr_t)x & 15) ||
      group_stride_bytes % block_bytes(T_Q5_K) || group_stride_bytes < (size_t)O * (I / QK) * block_bytes(T_Q5_K)) {
    fail("launch_q5_K_matmul_grouped: rejected shape (groups %d, I %d, O %d, stride %zu)", groups, I, O,
         group_stride_bytes);
    return false;
  }
  F32MMArgs a{};
  a.w = (const uint8_t *)w;
  a.w_row = (size_t)(I / QK) * block_bytes(T_Q5_K);
  a.w_mat = group_stride_bytes;
  a.x = x;
  a.x_tok = (size_t)groups * I;
  a.x_route = (size_t)I;
  a.x_routes = groups;
  a.y = y;
  a.y_tok = (size_t)groups * O;
  a.y_route = (size_t)O;
  a.I = I;
  a.O = O;
  a.n_tok = 1;
  a.mat_by_route = 1;
  return launch_mm(T_Q5_K, a, groups, nullptr) == 0;
}
void launch_iq3_xxs_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_IQ3_XXS, y, x, w, S, I, O, nullptr);
}
void launch_iq3_xxs_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_IQ3_XXS, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_iq4_xs_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_IQ4_XS, y, x, w, S, I, O, nullptr);
}
void launch_iq4_xs_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_IQ4_XS, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_iq2_xxs_matmul_stream(float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  plain_matmul(T_IQ2_XXS, y, x, w, S, I, O, (hipStream_t)stream);
}
void launch_iq2_xxs_matmul(float *y, const float *x, const void *w, int S, int I, int O) {
  plain_matmul(T_IQ2_XXS, y, x, w, S, I, O, nullptr);
}

int zm_f32_matmul(int type, float *y, const float *x, const void *w, int S, int I, int O, void *stream) {
  if (!f32_type(type)) return fail("zm_f32_matmul: unsupported weight type %d", type);
  return plain_matmul(type, y, x, w, S, I, O, (hipStream_t)stream);
}

// ---------------------------------------------------------------- FP32 MUL_MAT_ID hook

int zm_mul_mat_id_f32(const zm_tensor *w, const zm_tensor *x, const zm_tensor *ids, zm_tensor *y, void *stream,
                      int execute) {
  if (!w || !x || !y || !f32_type(w->type) || x->type != T_F32 || y->type != T_F32) return 0;
  if (w->ne[0] <= 0 || w->ne[0] > INT_MAX || w->ne[1] <= 0 || w->ne[1] > INT_MAX || w->ne[0] % QK) return 0;
  if (x->nb[0] != 4 || y->nb[0] != 4) return 0;
  const int I = (int)w->ne[0], O = (int)w->ne[1];
  const size_t row = (size_t)(I / QK) * block_bytes(w->type);
  if (w->nb[1] != row || x->ne[0] != I || y->ne[0] != O) return 0;
  // float4 activation loads
  if (((uintptr_t)x->data & 15) || x->nb[1] % 16 || x->nb[2] % 16) return 0;
  if (y->nb[1] % 4 || y->nb[2] % 4) return 0;
  F32MMArgs a{};
  a.w = (const uint8_t *)w->data;
  a.w_row = w->nb[1];
  a.x = (const float *)x->data;
  a.y = (float *)y->data;
  a.I = I;
  a.O = O;
  int n_route = 1;
  if (ids) {
    if (ids->type != T_I32 || ids->nb[0] != 4 || ids->ne[0] <= 0 || ids->ne[0] > 65535 || ids->ne[1] <= 0 ||
        ids->ne[1] > 65535 || w->ne[2] > INT_MAX || w->ne[3] != 1 || (x->ne[1] != 1 && x->ne[1] != ids->ne[0]) ||
        x->ne[2] != ids->ne[1] || x->ne[3] != 1 || y->ne[1] != ids->ne[0] || y->ne[2] != ids->ne[1] || y->ne[3] != 1)
      return 0;
    if (!execute) return 1;
    a.w_mat = w->nb[2];
    a.x_tok = x->nb[2] / 4;
    a.x_route = x->nb[1] / 4;
    a.x_routes = (int)x->ne[1];
    a.y_tok = y->nb[2] / 4;
    a.y_route = y->nb[1] / 4;
    a.ids = (const uint8_t *)ids->data;
    a.id_tok = ids->nb[1];
    a.id_route = ids->nb[0];
    a.E = (int)w->ne[2];
    a.n_tok = (int)ids->ne[1];
    n_route = (int)ids->ne[0];
  } else if (w->ne[2] == 1 && w->ne[3] == 1 && x->ne[2] == 1 && x->ne[3] == 1 && x->ne[1] > 0 && x->ne[1] <= 65535 &&
             y->ne[1] == x->ne[1] && x->nb[1] == (size_t)I * 4 && y->nb[1] == (size_t)O * 4) {
    if (!execute) return 1;
    a.x_tok = (size_t)I;
    a.x_routes = 1;
    a.y_tok = (size_t)O;
    a.n_tok = (int)x->ne[1];
  } else if (w->ne[3] == 1 && w->ne[2] > 1 && w->ne[2] <= 65535 && x->ne[2] == w->ne[2] && x->ne[3] == 1 &&
             x->ne[1] > 0 && x->ne[1] <= 65535 && y->ne[1] == x->ne[1] && y->ne[2] == w->ne[2] && y->ne[3] == 1) {
    if (!execute) return 1;
    a.w_mat = w->nb[2];
    a.x_tok = x->nb[1] / 4;
    a.x_route = x->nb[2] / 4;
    a.x_routes = (int)w->ne[2];
    a.y_tok = y->nb[1] / 4;
    a.y_route = y->nb[2] / 4;
    a.n_tok = (int)x->ne[1];
    a.mat_by_route = 1;
    n_route = (int)w->ne[2];
  } else {
    return 0;
  }
  if (launch_mm(w->type, a, n_route, (hipStream_t)stream)) return 0;
  count_mmid_launch();
  return 1;
}

// ---------------------------------------------------------------- helpers

void launch_expert_swiglu(float *prod, const float *gate, const float *up, int n, float clamp, int fused, int *d_bad,
                          void *stream) {
  if (n <= 0) return;
  hipLaunchKernelGGL(k_swiglu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, prod, gate, up,
                     n, clamp, fused, d_bad);
}

void launch_expert_scatter_accum(const float *src, const int *tok, const float *w, float *dst, int n, int D, int S,
                                 void *stream) {
  if (n <= 0 || D <= 0) return;
  hipLaunchKernelGGL(k_scatter_accum, dim3((unsigned)n), dim3(256), 0, (hipStream_t)stream, src, tok, w, dst, D, S);
}

void launch_expert_scatter_add(const float *src, const int *tok, float *dst, int n, int D, int S, void *stream) {
  launch_expert_scatter_accum(src, tok, nullptr, dst, n, D, S, stream);
}

void launch_glm5next_router_topk(float *logits, const float *bias, int32_t *ids, float *weights, int S, int n_experts,
                                 int topk, int gating_func, int normalize, float weight_scale, void *stream) {
  if (S <= 0 || n_experts <= 0 || topk <= 0 || topk > n_experts) return;
  if (n_experts > GLM_MAX_E || topk > 64) {
    fail("launch_glm5next_router_topk: n_experts <= %d and topk <= 64 required", GLM_MAX_E);
    return;
  }
  hipLaunchKernelGGL(k_glm_router_topk, dim3((unsigned)S), dim3(64), 0, (hipStream_t)stream, logits, bias, ids,
                     weights, n_experts, topk, gating_func, normalize, weight_scale);
}

// ---------------------------------------------------------------- executor stages

int zm_expert_scratch_ensure(zm_expert_scratch *s, int S, int D, int F, int device) {
  if (!s || S <= 0 || D <= 0 || F <= 0) return fail("zm_expert_scratch_ensure: bad arguments");
  HIP_OK(hipSetDevice(device));
  if (s->device_id >= 0 && s->device_id != device) zm_expert_scratch_release(s);
  s->device_id = device;
  if (!s->d_bad) {
    HIP_OK(hipMalloc((void **)&s->d_bad, 2 * sizeof(int32_t)));
    HIP_OK(hipMemset(s->d_bad, 0, 2 * sizeof(int32_t)));
  }
  const size_t sd = (size_t)S * D, si = (size_t)S * F;
  if (sd > s->cap_sd) {
    HIP_OK(hipDeviceSynchronize());
    (void)hipFree(s->d_x);
    (void)hipFree(s->d_down);
    s->d_x = s->d_down = nullptr;
    s->cap_sd = 0;
    HIP_OK(hipMalloc((void **)&s->d_x, sd * 4));
    HIP_OK(hipMalloc((void **)&s->d_down, sd * 4));
    s->cap_sd = sd;
  }
  if (si > s->cap_si) {
    HIP_OK(hipDeviceSynchronize());
    (void)hipFree(s->d_gate);
    (void)hipFree(s->d_up);
    (void)hipFree(s->d_prod);
    s->d_gate = s->d_up = s->d_prod = nullptr;
    s->cap_si = 0;
    HIP_OK(hipMalloc((void **)&s->d_gate, si * 4));
    HIP_OK(hipMalloc((void **)&s->d_up, si * 4));
    HIP_OK(hipMalloc((void **)&s->d_prod, si * 4));
    s->cap_si = si;
  }
  return 0;
}

void zm_expert_scratch_release(zm_expert_scratch *s) {
  if (!s) return;
  if (s->device_id >= 0) (void)hipSetDevice(s->device_id);
  (void)hipDeviceSynchronize();
  for (void *p : {(void *)s->d_bad, (void *)s->d_x, (void *)s->d_gate, (void *)s->d_up, (void *)s->d_prod,
                  (void *)s->d_down})
    if (p) (void)hipFree(p);
  *s = zm_expert_scratch{};
  s->device_id = -1;
}

int zm_expert_ffn_issue(zm_expert_scratch *s, const void *slab, size_t up_offset, int gate_type, int up_type,
                        const float *host_x, int S, int D, int F, const float *device_x, void *stream) {
  if (!s || !slab || (!host_x && !device_x)) return fail("zm_expert_ffn_issue: null argument");
  if (!f32_type(gate_type) || !f32_type(up_type)) return fail("zm_expert_ffn_issue: unsupported type");
  int dev = 0;
  HIP_OK(hipGetDevice(&dev));
  if (zm_expert_scratch_ensure(s, S, D, F, dev)) return -1;
  hipStream_t st = (hipStream_t)stream;
  const float *xin = device_x;
  if (!xin) {
    HIP_OK(hipMemcpyAsync(s->d_x, host_x, (size_t)S * D * 4, hipMemcpyHostToDevice, st));
    xin = s->d_x;
  }
  const uint8_t *g = (const uint8_t *)slab;
  if (plain_matmul(gate_type, s->d_gate, xin, g, S, D, F, st)) return -1;
  if (plain_matmul(up_type, s->d_up, xin, g + up_offset, S, D, F, st)) return -1;
  return 0;
}

int zm_expert_ffn_finish_stage1(zm_expert_scratch *s, const void *slab, size_t down_offset, int down_type, int S,
                                int D, int F, float swiglu_clamp, int fused_clamp, void *stream) {
  if (!s || !slab || !s->d_gate || (size_t)S * F > s->cap_si || (size_t)S * D > s->cap_sd)
    return fail("zm_expert_ffn_finish_stage1: scratch not issued for this shape");
  if (!f32_type(down_type)) return fail("zm_expert_ffn_finish_stage1: unsupported type");
  HIP_OK(hipSetDevice(s->device_id));
  hipStream_t st = (hipStream_t)stream;
  launch_expert_swiglu(s->d_prod, s->d_gate, s->d_up, S * F, swiglu_clamp, fused_clamp, s->d_bad, st);
  HIP_OK(hipGetLastError());
  return plain_matmul(down_type, s->d_down, s->d_prod, (const uint8_t *)slab + down_offset, S, F, D, st);
}

int zm_expert_ffn_finish_stage2(zm_expert_scratch *s, float *host_out, int S, int D, void *stream) {
  if (!s || !host_out || !s->d_down || (size_t)S * D > s->cap_sd)
    return fail("zm_expert_ffn_finish_stage2: scratch not issued for this shape");
  HIP_OK(hipSetDevice(s->device_id));
  HIP_OK(hipMemcpyAsync(host_out, s->d_down, (size_t)S * D * 4, hipMemcpyDeviceToHost, (hipStream_t)stream));
  HIP_OK(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

int zm_expert_bad_counts(zm_expert_scratch *s, int32_t counts[2], int reset) {
  if (!s || !s->d_bad || !counts) return fail("zm_expert_bad_counts: no counter");
  HIP_OK(hipSetDevice(s->device_id));
  HIP_OK(hipMemcpy(counts, s->d_bad, 2 * sizeof(int32_t), hipMemcpyDeviceToHost));
  if (reset) HIP_OK(hipMemset(s->d_bad, 0, 2 * sizeof(int32_t)));
  return 0;
}

}  // extern "C"
