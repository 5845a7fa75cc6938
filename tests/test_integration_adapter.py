"""The ggml-HIP adapter (zeromoe_amd/integration/ggml_hip_hook.cpp) compiles
against include/zeromoe.h, links against libzeromoe_hip.so and behaves as the
reference hook's caller expects on the host-only paths (no GPU needed):
declines null / non-MUL_MAT_ID calls and every call without a bound
workspace, sizes a workspace, and forwards the capability probes."""
import os
import subprocess

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
  const bool q_unbound = zeromoe_hook_for_test(&w, &x, &ids, &y, nullptr, false);
  ggml_tensor bad = w; bad.ne[0] = 2000;           // not a multiple of 256
  const size_t need_bad = zeromoe_hook_workspace_bytes(&bad, &x, &ids, &y);
  std::printf("%zu %d %d %zu %d %d %d\n", need, (int)q_null, (int)q_unbound, need_bad,
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
    need, q_null, q_unbound, need_bad, installed, skip_cpu, skip_gpu = out.stdout.split()
    assert int(need) > 4 * 2048 * 1.14  # Q8_K rows of the 4 tokens at least
    assert q_null == "0"                 # MUL_MAT (no ids) stays with ggml
    assert q_unbound == "0"              # no workspace bound: declined, nothing allocated
    assert need_bad == "0"               # shape declined
    assert installed == "0"              # no ggml hook setter linked in
    assert skip_cpu == "1" and skip_gpu == "1"
