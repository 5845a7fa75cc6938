"""Writes tests/golden/ref_dots.npz: Q2_K x Q8_K and Q4_K x Q8_K dot products
computed by the reference's own kernels (bench/q2k_dot_bench.cpp:31-63, ggml's
stock AVX2 Q2_K dot; bench/q3k_q4k_dot_bench.cpp:73-125, the 512-bit Q4_K dot
stated bit-exact to ggml's stock), compiled from the reference tree into
oracle/_ref/libzmref.so by oracle/Makefile.  Inputs are random valid blocks
(random bytes, finite fp16 scales) and Q8_K rows of N(0, s) activations.

    make -C oracle ref && python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import zm_oracle as O  # noqa: E402


def main():
    R = O.ref_lib()
    if R is None:
        raise SystemExit("oracle/_ref/libzmref.so missing: run `make -C oracle ref`")
    rng = np.random.default_rng(20261003)
    out = {}
    for name, t, fn in (("q2_K", O.TYPE_Q2_K, R.zmref_dot_q2_K), ("q4_K", O.TYPE_Q4_K, R.zmref_dot_q4_K)):
        nbs, ws, qs, dots = [], [], [], []
        for i in range(48):
            nb = int(rng.integers(1, 9))
            n = nb * 256
            w = O.random_blocks(t, 1, n, seed=1000 + i)[0]
            x = (rng.standard_normal(n) * rng.uniform(0.01, 50)).astype(np.float32)
            if i % 7 == 0:
                x[rng.integers(0, n, n // 2)] = 0.0
            q = O.quantize_q8_K(x)
            nbs.append(nb)
            ws.append(np.pad(w, (0, 8 * O.BLOCK_BYTES[t] - w.size)))
            qs.append(np.pad(q.view(np.uint8), (0, 8 * 292 - q.nbytes)))
            dots.append(np.float32(fn(n, w.ctypes.data, q.ctypes.data)))
        out[name + "_nb"] = np.array(nbs, np.int32)
        out[name + "_w"] = np.stack(ws)
        out[name + "_q8"] = np.stack(qs)
        out[name + "_dot"] = np.array(dots, np.float32)
    np.savez_compressed(os.path.join(HERE, "ref_dots.npz"), **out)
    print("wrote", os.path.join(HERE, "ref_dots.npz"))


if __name__ == "__main__":
    main()
