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
SOURCES = ("zm_api.hip", "zm_exec.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: the quantizer, router and SwiGLU are bit-reproducible
# IQ2/K-quant arithmetic only if no multiply-add is fused behind our back.
# -packed-fp32-ops off: packed fp32 VALU forms are avoided on this target.
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-shared", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    cmd = [HIPCC, *FLAGS, "-o", OUT, *[os.path.join(SRC, f) for f in SOURCES]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{' '.join(cmd)}\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
    sys.exit(0)
