"""The ggml-HIP adapter (zeromoe_amd/integration/ggml_hip_hook.cpp) compiles
against include/zeromoe.h, links against libzeromoe_hip.so and behaves as the
reference hook's caller expects on the host-only paths (no GPU needed):
declines null calls and MUL_MAT_ID calls without a bound workspace, accepts a
plain 2-D MUL_MAT (ids == NULL, the reference hook's dense branch), sizes a
workspace, and forwards the capability probes.  On the GPU the dense branch,
called through the adapter's registered hook, matches the oracle's FP32 matmul
(kquant_matmul.cu:740-746)."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

MAIN = r"""
#include <cstdio>
#include "ggml.h"
extern "C" bool zeromoe_hook_for_test(const ggml_tensor *, const ggml_tensor *, const ggml_tensor *, ggml_tensor *,
                                      void *, bool);
extern "C" size_t zeromoe_hook_workspace_bytes(const ggml_tensor *, const ggml_tensor *, const ggml_tensor *,
                                               const ggml_tensor *);
extern "C" bool zeromoe_install_f32_quant_graph_hook();
extern "C" int ggml_cpu_mul_mat_id_negative_skip(void);
extern "C" int ggml_cuda_mul_mat_id_negative_skip_batched(void);

static void dims(ggml_tensor &t, ggml_type ty, long n0, long n1, long n2, size_t e0) {
  t = ggml_tensor{};
  t.type = ty;
  t.ne[0] = n0; t.ne[1] = n1; t.ne[2] = n2; t.ne[3] = 1;
  t.nb[0] = e0;
  t.nb[1] = (ty == GGML_TYPE_Q4_K ? (n0 / 256) * 144 : n0 * e0);
  t.nb[2] = t.nb[1] * n1; t.nb[3] = t.nb[2] * n2;
  t.data = (void *)0x10000;  // never dereferenced on these paths
}

int main() {
  ggml_tensor w, x, ids, y;
  dims(w, GGML_TYPE_Q4_K, 2048, 768, 128, 144);   // [H, F, E] Q4_K
  dims(x, GGML_TYPE_F32, 2048, 1, 4, 4);          // [H, 1, S]
  dims(ids, GGML_TYPE_I32, 8, 4, 1, 4);           // [K, S]
  dims(y, GGML_TYPE_F32, 768, 8, 4, 4);           // [F, K, S]
  const size_t need = zeromoe_hook_workspace_bytes(&w, &x, &ids, &y);
  const bool q_null = zeromoe_hook_for_test(&w, &x, nullptr, &y, nullptr, false);
  ggml_tensor w2, x2, y2;                          // dense MUL_MAT: W [I, O] Q2_K, x [I, S], y [O, S]
  dims(w2, GGML_TYPE_Q2_K, 2048, 768, 1, 84);
  w2.nb[1] = (2048 / 256) * 84; w2.nb[2] = w2.nb[1] * 768; w2.nb[3] = w2.nb[2];
  dims(x2, GGML_TYPE_F32, 2048, 4, 1, 4);
  dims(y2, GGML_TYPE_F32, 768, 4, 1, 4);
  const bool q_dense = zeromoe_hook_for_test(&w2, &x2, nullptr, &y2, nullptr, false);
  const bool q_nothing = zeromoe_hook_for_test(nullptr, &x2, nullptr, &y2, nullptr, false);
  const bool q_unbound = zeromoe_hook_for_test(&w, &x, &ids, &y, nullptr, false);
  ggml_tensor bad = w; bad.ne[0] = 2000;           // not a multiple of 256
  const size_t need_bad = zeromoe_hook_workspace_bytes(&bad, &x, &ids, &y);
  std::printf("%zu %d %d %d %d %zu %d %d %d\n", need, (int)q_null, (int)q_dense, (int)q_nothing, (int)q_unbound, need_bad,
              (int)zeromoe_install_f32_quant_graph_hook(), ggml_cpu_mul_mat_id_negative_skip(),
              ggml_cuda_mul_mat_id_negative_skip_batched());
  return 0;
}
"""


def test_adapter_compiles_links_and_answers(tmp_path):
    lib_dir = os.path.join(ROOT, "zeromoe_amd", "lib")
    if not os.path.exists(os.path.join(lib_dir, "libzeromoe_hip.so")):
        pytest.fail("libzeromoe_hip.so is not built")
    main = tmp_path / "main.cpp"
    main.write_text(MAIN)
    exe = tmp_path / "adapter_test"
    cmd = ["g++", "-std=c++17", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include",
           "-I", os.path.join(ROOT, "tests", "ggml_subset"),
           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "zeromoe_amd", "integration", "ggml_hip_hook.cpp"),
           str(main), "-L", lib_dir, "-lzeromoe_hip", f"-Wl,-rpath,{lib_dir}", "-L", "/opt/rocm/lib", "-lamdhip64",
           "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    need, q_null, q_dense, q_nothing, q_unbound, need_bad, installed, skip_cpu, skip_gpu = out.stdout.split()
    assert int(need) > 4 * 2048 * 1.14  # Q8_K rows of the 4 tokens at least
    assert q_null == "0"                 # 3-D weights without ids: neither dense nor grouped form
    assert q_dense == "1"                # plain 2-D MUL_MAT: the dense branch takes it
    assert q_nothing == "0"              # null weights
    assert q_unbound == "0"              # no workspace bound: declined, nothing allocated
    assert need_bad == "0"               # shape declined
    assert installed == "0"              # no ggml hook setter linked in
    assert skip_cpu == "1" and skip_gpu == "1"


def _adapter_so(tmp_path):
    """The adapter as a shared library (g++ on the host, linked against the
    built libzeromoe_hip.so), for calling its registered hook from a test."""
    lib_dir = os.path.join(ROOT, "zeromoe_amd", "lib")
    so = tmp_path / "libzeromoe_ggml_hook.so"
    cmd = ["g++", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I", "/opt/rocm/include", "-I", os.path.join(ROOT, "tests", "ggml_subset"), "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "zeromoe_amd", "integration", "ggml_hip_hook.cpp"), "-L", lib_dir, "-lzeromoe_hip",
           f"-Wl,-rpath,{lib_dir}", "-L", "/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", str(so)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return str(so)


class GgmlTensor(C.Structure):
    _fields_ = [("type", C.c_int), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", C.c_void_p)]


def _gt(ty, ne, nb, ptr):
    t = GgmlTensor()
    t.type = ty
    for i in range(4):
        t.ne[i] = ne[i]
        t.nb[i] = nb[i]
    t.data = ptr
    return t


@pytest.mark.gpu
@pytest.mark.parametrize("t,S,I,Orows", [(10, 1, 4096, 96), (11, 5, 2048, 77), (12, 3, 1536, 64)])
def test_adapter_dense_branch_vs_oracle(tmp_path, t, S, I, Orows):
    """ids == NULL through the adapter's hook: y[S, O] = x[S, I] . dequant(W)^T
    on the GPU against the oracle's FP32 matmul (the reference hook runs
    launch_q2_K/q3_K_matmul_stream there, kquant_matmul.cu:740-746)."""
    import torch

    import zeromoe_amd as Z
    import zm_oracle as O

    Z.init()
    print(f"adapter dense t={t} S={S} I={I} O={Orows}", flush=True)
    hook = C.CDLL(_adapter_so(tmp_path)).zeromoe_hook_for_test
    hook.restype = C.c_bool
    hook.argtypes = [C.c_void_p] * 5 + [C.c_bool]
    W = O.random_blocks(t, Orows, I, seed=t + S)
    x = np.random.default_rng(I + S).standard_normal((S, I)).astype(np.float32)
    Wd, xd = torch.from_numpy(W).cuda(), torch.from_numpy(x).cuda()
    yd = torch.full((S, Orows), float("nan"), device="cuda")
    rb = W.shape[1]
    tw = _gt(t, (I, Orows, 1, 1), (rb // (I // 256), rb, rb * Orows, rb * Orows), Wd.data_ptr())
    tx = _gt(0, (I, S, 1, 1), (4, 4 * I, 4 * I * S, 4 * I * S), xd.data_ptr())
    ty = _gt(0, (Orows, S, 1, 1), (4, 4 * Orows, 4 * Orows * S, 4 * Orows * S), yd.data_ptr())
    stream = torch.cuda.current_stream().cuda_stream
    assert hook(C.byref(tw), C.byref(tx), None, C.byref(ty), stream, False)  # capability query
    assert hook(C.byref(tw), C.byref(tx), None, C.byref(ty), stream, True)
    torch.cuda.synchronize()
    got = yd.cpu().numpy().astype(np.float64)
    ref = O.f32_matmul(t, W, x)
    bound = O.f32_matmul_absbound(t, W, x)
    assert np.all(np.abs(got - ref) <= 2e-5 * bound + 1e-30)
