// ggml_hip_hook.cpp -- the adapter a ggml-HIP build links into the model binary
// to route GGML_OP_MUL_MAT_ID through libzeromoe_hip.so.
//
// It replaces the reference's native_f32_quant_hook registration
// (kernels/quant/kquant_matmul.cu:757-761) for ggml's HIP backend patched as in
// patches/ggml/0010-native-f32-quant-graph-hook.patch:9-27, and the weak
// capability probes of backends/ggml/mmid_route_skip.hpp:22,41.
//
// Build: g++ -std=c++17 -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include -I<ggml>/include -I<repo>/include
//            -c ggml_hip_hook.cpp
//        link with -L<repo>/zeromoe_amd/lib -lzeromoe_hip -L/opt/rocm/lib -lamdhip64
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>

#include "ggml.h"
#include "zeromoe.h"

extern "C" void ggml_cuda_set_f32_quant_matmul_hook(
    bool (*)(const ggml_tensor *, const ggml_tensor *, const ggml_tensor *, ggml_tensor *, void *, bool))
    __attribute__((weak));

namespace {

zm_tensor as_zm(const ggml_tensor *t) {
  zm_tensor z{};
  z.type = (int32_t)t->type;
  for (int i = 0; i < 4; ++i) {
    z.ne[i] = t->ne[i];
    z.nb[i] = t->nb[i];
  }
  z.data = t->data;
  return z;
}

bool zeromoe_hip_hook(const ggml_tensor *w, const ggml_tensor *x, const ggml_tensor *ids, ggml_tensor *y,
                      void *stream, bool execute) {
  if (!w || !x || !y) return false;
  const zm_tensor zw = as_zm(w), zx = as_zm(x);
  zm_tensor zy = as_zm(y);
  if (!ids) {
    // plain MUL_MAT (dense and shared FFNs): the reference hook's ids == NULL
    // branches, FP32 activations (kquant_matmul.cu:740-755); no workspace
    return zm_mul_mat_id_f32(&zw, &zx, nullptr, &zy, stream, execute ? 1 : 0) == 1;
  }
  const zm_tensor zi = as_zm(ids);
  return zm_mul_mat_id(&zw, &zx, &zi, &zy, stream, execute ? 1 : 0) == 1;
}

// workspaces bound by zeromoe_bind_hook_workspace, one per stream
std::mutex g_ws_mu;
std::map<void *, void *> g_ws;

}  // namespace

// Set-up, once per stream ggml executes on (the backend context's stream),
// before the first graph compute: one device buffer of `bytes` bound as the
// hook's workspace.  The hook itself never allocates.  Binding a stream again
// (a larger graph) replaces its buffer; the old one is freed once the stream
// has drained.  Until some workspace is bound on the device, the hook's
// capability query declines every MUL_MAT_ID shape (it answers for the
// smallest bound workspace), so bind before ggml's supports_op pass.
extern "C" bool zeromoe_bind_hook_workspace(void *stream, size_t bytes) {
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) return false;
  if (zm_mul_mat_id_set_workspace(stream, p, bytes) != 0) {
    (void)hipFree(p);
    return false;
  }
  std::lock_guard<std::mutex> lk(g_ws_mu);
  void *&slot = g_ws[stream];
  if (slot) {
    (void)hipStreamSynchronize((hipStream_t)stream);
    (void)hipFree(slot);
  }
  slot = p;
  return true;
}

// Workspace bytes one MUL_MAT_ID node needs (the largest over a graph's nodes
// sizes the buffer).
extern "C" size_t zeromoe_hook_workspace_bytes(const ggml_tensor *w, const ggml_tensor *x, const ggml_tensor *ids,
                                               const ggml_tensor *y) {
  const zm_tensor zw = as_zm(w), zx = as_zm(x), zi = as_zm(ids), zy = as_zm(y);
  return zm_mul_mat_id_workspace_size(&zw, &zx, &zi, &zy);
}

extern "C" bool zeromoe_install_f32_quant_graph_hook() {
  if (!ggml_cuda_set_f32_quant_matmul_hook || zm_init() != 0) return false;
  ggml_cuda_set_f32_quant_matmul_hook(zeromoe_hip_hook);
  return true;
}

extern "C" uint64_t zeromoe_f32_quant_graph_launches() { return zm_mul_mat_id_launches(); }

// mmid_route_skip.hpp:22,41 probe these weak symbols before emitting id = -1
extern "C" int ggml_cpu_mul_mat_id_negative_skip(void) { return zm_mul_mat_id_negative_skip(); }
extern "C" int ggml_cuda_mul_mat_id_negative_skip_batched(void) { return zm_mul_mat_id_negative_skip_batched(); }

// For tests of this adapter: the hook as registered (MUL_MAT_ID, and plain
// MUL_MAT with ids == NULL).
extern "C" bool zeromoe_hook_for_test(const ggml_tensor *w, const ggml_tensor *x, const ggml_tensor *ids,
                                      ggml_tensor *y, void *stream, bool execute) {
  return zeromoe_hip_hook(w, x, ids, y, stream, execute);
}
