"""In-tree build of libzeromoe_hip.so for gfx950 (hipcc, no JIT cache).

    python -m zeromoe_amd.build
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
SRC = os.path.join(PKG_DIR, "csrc")
OUT = os.path.join(PKG_DIR, "lib", "libzeromoe_hip.so")
SOURCES = ("zm_api.hip", "zm_dec_a.hip", "zm_dec_b.hip", "zm_exec.hip", "zm_pack.hip", "zm_lane.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: the quantizer, router and SwiGLU are bit-reproducible
# IQ2/K-quant arithmetic only if no multiply-add is fused behind our back.
# -packed-fp32-ops off: packed fp32 VALU forms are avoided on this target.
# -amdgpu-mfma-vgpr-form: MFMA results land in ordinary VGPRs, so the float
# epilogue of the prefill tiles reads them without v_accvgpr_read copies.
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-Wall", "-Wno-unused-function"]


def build(verbose: bool = False) -> str:
    """Compile each translation unit in parallel (hipcc -c), then link."""
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    obj_dir = os.path.join(PKG_DIR, "lib", "obj")
    os.makedirs(obj_dir, exist_ok=True)
    cflags = [f for f in FLAGS if f != "-shared"]
    jobs = []
    for f in SOURCES:
        obj = os.path.join(obj_dir, f.replace(".hip", ".o"))
        cmd = [HIPCC, *cflags, "-c", "-o", obj, os.path.join(SRC, f)]
        jobs.append((cmd, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    msgs, failed = [], None
    for cmd, _, p in jobs:
        out = p.communicate()[0]
        msgs += [l for l in out.splitlines() if "packed-fp32-ops" not in l]
        if p.returncode != 0 and failed is None:
            failed = cmd
    if failed is not None:
        raise RuntimeError(f"hipcc failed:\n{' '.join(failed)}\n" + "\n".join(msgs))
    link = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", OUT, *[o for _, o, _ in jobs]]
    r = subprocess.run(link, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(link)}\n{r.stdout}{r.stderr}")
    if verbose and any(m.strip() for m in msgs):
        print("\n".join(msgs))
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
    sys.exit(0)
