"""ctypes binding of the CPU oracle (oracle/zm_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg, as the checker.  The shipped library never
imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libzmoracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libzmref.so")

QK_K = 256
TYPE_F32, TYPE_Q2_K, TYPE_Q3_K, TYPE_Q4_K, TYPE_Q8_K, TYPE_IQ2_XXS, TYPE_I32 = 0, 10, 11, 12, 15, 16, 26
TYPE_Q5_K, TYPE_Q6_K, TYPE_IQ4_XS, TYPE_IQ3_XXS = 13, 14, 23, 18
BLOCK_BYTES = {TYPE_Q2_K: 84, TYPE_Q3_K: 110, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210, TYPE_IQ4_XS: 136, TYPE_IQ3_XXS: 98, TYPE_IQ2_XXS: 66, TYPE_Q8_K: 292}
TYPE_NAMES = {TYPE_Q2_K: "q2_K", TYPE_Q3_K: "q3_K", TYPE_Q4_K: "q4_K", TYPE_Q5_K: "q5_K", TYPE_Q6_K: "q6_K", TYPE_IQ4_XS: "iq4_xs", TYPE_IQ3_XXS: "iq3_xxs", TYPE_IQ2_XXS: "iq2_xxs", TYPE_Q8_K: "q8_K"}
GATING_SOFTMAX, GATING_SIGMOID, GATING_SQRT_SOFTPLUS = 0, 1, 2

Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
assert Q8K_DTYPE.itemsize == 292


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    if os.path.isdir("/root/reference"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, I, I64, F = C.c_void_p, C.c_int, C.c_int64, C.c_float
        L.zmo_fp16_to_fp32.restype = F
        L.zmo_fp16_to_fp32.argtypes = [C.c_uint16]
        L.zmo_fp32_to_fp16.restype = C.c_uint16
        L.zmo_fp32_to_fp16.argtypes = [F]
        L.zmo_expf.restype = F
        L.zmo_expf.argtypes = [F]
        L.zmo_nearest_int.restype = I
        L.zmo_nearest_int.argtypes = [F]
        L.zmo_fill_normal.argtypes = [C.c_uint64, F, F, P, I64]
        L.zmo_iq2xxs_grid.restype = P
        L.zmo_set_iq2xxs_grid.argtypes = [P]
        L.zmo_iq2xxs_standin_grid.argtypes = [P]
        L.zmo_iq3xxs_grid.restype = P
        L.zmo_set_iq3xxs_grid.argtypes = [P]
        L.zmo_iq4nl_table.restype = P
        L.zmo_set_iq4nl_table.argtypes = [P]
        L.zmo_ksigns_iq2xs.restype = C.c_uint8
        L.zmo_ksigns_iq2xs.argtypes = [I]
        L.zmo_quantize_rows.argtypes = [I, P, P, I64, I64]
        L.zmo_quantize_row_q8_K.argtypes = [P, P, I64]
        L.zmo_dequantize_row.argtypes = [I, P, P, I64]
        L.zmo_vec_dot_q8_K.restype = F
        L.zmo_vec_dot_q8_K.argtypes = [I, I, P, P]
        L.zmo_block_dots.argtypes = [I, I, P, P, P, P]
        L.zmo_mul_mat_id.restype = I
        L.zmo_mul_mat_id.argtypes = [P, P, P, P, I]
        L.zmo_router.argtypes = [P, P, P, P, I, P, P]
        L.zmo_apply_slot_table.argtypes = [P, P, I, I, P, P]
        L.zmo_bucket.restype = I
        L.zmo_bucket.argtypes = [P, I, I, I, P, P, P]
        L.zmo_swiglu.argtypes = [P, P, P, I64]
        L.zmo_moe_forward.argtypes = [P, P, P, P, P, I]
        L.zmo_moe_forward_fast.argtypes = [P, P, P, P, P, I]
        L.zmo_vec_dot_q8_K_fast.restype = F
        L.zmo_vec_dot_q8_K_fast.argtypes = [I, I, P, P]
        L.zmo_cpu_has_avx512.restype = I
        L.zmo_router_gemv.argtypes = [P, P, I, I, I, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle needs contiguous arrays"
    return a.ctypes.data


def row_size(t: int, n: int) -> int:
    return n * 4 if t == TYPE_F32 else (n // QK_K) * BLOCK_BYTES[t]


# ---------------------------------------------------------------- numerics

def fill_normal(seed: int, n: int, mean: float = 0.0, sd: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().zmo_fill_normal(seed, mean, sd, _p(out), n)
    return out


def expf(x: float) -> float:
    return lib().zmo_expf(x)


def fp16_to_fp32(h: int) -> float:
    return lib().zmo_fp16_to_fp32(h)


def fp32_to_fp16(f: float) -> int:
    return lib().zmo_fp32_to_fp16(f)


def iq2xxs_grid() -> np.ndarray:
    ptr = lib().zmo_iq2xxs_grid()
    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint64)), (256,)).copy()


def iq3xxs_grid() -> np.ndarray:
    ptr = lib().zmo_iq3xxs_grid()
    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint32)), (256,)).copy()


def iq4nl_table() -> np.ndarray:
    ptr = lib().zmo_iq4nl_table()
    return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_int8)), (16,)).copy()


def ksigns() -> np.ndarray:
    return np.array([lib().zmo_ksigns_iq2xs(i) for i in range(128)], np.uint8)


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    """Quantize rows of x (..., n) to type t; returns uint8 (..., row_bytes)."""
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(x.shape[:-1] + (row_size(t, n),), np.uint8)
    lib().zmo_quantize_rows(t, _p(x), _p(out), rows, n)
    return out


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    n = x.shape[-1]
    out = np.empty(x.shape[:-1] + (n // QK_K,), Q8K_DTYPE)
    lib().zmo_quantize_rows(TYPE_Q8_K, _p(x), _p(out), x.size // n, n)
    return out


def dequantize(t: int, w: np.ndarray, n: int) -> np.ndarray:
    w = np.ascontiguousarray(w)
    rows = w.size * w.itemsize // row_size(t, n)
    out = np.empty((rows, n), np.float32)
    rs = row_size(t, n)
    raw = w.view(np.uint8).reshape(rows, rs)
    for r in range(rows):
        lib().zmo_dequantize_row(t, raw[r].ctypes.data, out[r].ctypes.data, n)
    return out


def vec_dot(t: int, w_row: np.ndarray, q8_row: np.ndarray) -> float:
    n = (q8_row.size * q8_row.itemsize // 292) * QK_K
    return lib().zmo_vec_dot_q8_K(t, n, _p(np.ascontiguousarray(w_row)), _p(np.ascontiguousarray(q8_row)))


def vec_dot_fast(t: int, w_row: np.ndarray, q8_row: np.ndarray) -> float:
    n = (q8_row.size * q8_row.itemsize // 292) * QK_K
    return lib().zmo_vec_dot_q8_K_fast(t, n, _p(np.ascontiguousarray(w_row)), _p(np.ascontiguousarray(q8_row)))


def block_dots(t: int, w_row: np.ndarray, q8_row: np.ndarray):
    nb = q8_row.size * q8_row.itemsize // 292
    isum = np.zeros(nb, np.int32)
    imin = np.zeros(nb, np.int32)
    lib().zmo_block_dots(t, nb * QK_K, _p(np.ascontiguousarray(w_row)), _p(np.ascontiguousarray(q8_row)), _p(isum),
                         _p(imin))
    return isum, imin


def random_blocks(t: int, n_rows: int, n: int, seed: int, scale: float = 0.02) -> np.ndarray:
    """Random but valid quantized rows (random bytes, finite fp16 scales sized
    so dequantized weights have roughly `scale` magnitude)."""
    rng = np.random.default_rng(seed)
    rs = row_size(t, n)
    raw = rng.integers(0, 256, size=(n_rows, rs), dtype=np.uint8)
    nb = n // QK_K
    blk = raw.reshape(n_rows, nb, BLOCK_BYTES[t])

    def h(v):
        return np.asarray(v, np.float16).view(np.uint16)

    def put16(off, vals):
        u = h(vals)
        blk[..., off] = (u & 0xFF).astype(np.uint8)
        blk[..., off + 1] = (u >> 8).astype(np.uint8)

    shp = (n_rows, nb)
    if t == TYPE_Q2_K:  # qs values 0..3, scale 0..15: w ~ d*sc*q -> d ~ scale/20
        put16(80, rng.uniform(0.5, 1.5, shp) * scale / 20)
        put16(82, rng.uniform(0.5, 1.5, shp) * scale / 8)
    elif t == TYPE_Q3_K:  # q in -4..3, sc in -32..31
        put16(108, rng.uniform(0.5, 1.5, shp) * scale / 40)
    elif t == TYPE_Q4_K:  # q 0..15, sc 0..63
        put16(0, rng.uniform(0.5, 1.5, shp) * scale / 200)
        put16(2, rng.uniform(0.5, 1.5, shp) * scale / 60)
    elif t == TYPE_Q5_K:  # q 0..31, sc 0..63
        put16(0, rng.uniform(0.5, 1.5, shp) * scale / 400)
        put16(2, rng.uniform(0.5, 1.5, shp) * scale / 60)
    elif t == TYPE_Q6_K:  # q-32 in -32..31, sc in -128..127
        put16(208, rng.uniform(0.5, 1.5, shp) * scale / 2000)
    elif t == TYPE_IQ3_XXS:  # grid 4..62, (0.5+ls)*0.5 up to ~8
        put16(0, rng.uniform(0.5, 1.5, shp) * scale / 150)
    elif t == TYPE_IQ4_XS:  # table up to 127, ls-32 in -32..31
        put16(0, rng.uniform(0.5, 1.5, shp) * scale / 2000)
    elif t == TYPE_IQ2_XXS:  # grid 8..43, (0.5+ls)*0.25 up to ~4
        put16(0, rng.uniform(0.5, 1.5, shp) * scale / 40)
    return raw


# ---------------------------------------------------------------- op / layer

class _Tensor(C.Structure):
    _fields_ = [("type", C.c_int), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", C.c_void_p)]


def tensor(t: int, ne, data: np.ndarray, nb=None) -> _Tensor:
    ne = list(ne) + [1] * (4 - len(ne))
    if nb is None:
        if t in (TYPE_F32, TYPE_I32):
            nb0 = 4
            nb = [4, 4 * ne[0]]
        else:
            nb0 = BLOCK_BYTES[t]
            nb = [nb0, row_size(t, ne[0])]
        nb.append(nb[1] * ne[1])
        nb.append(nb[2] * ne[2])
    T = _Tensor()
    T.type = t
    for i in range(4):
        T.ne[i] = ne[i]
        T.nb[i] = nb[i]
    T.data = data.ctypes.data
    return T


def mul_mat_id(t: int, W: np.ndarray, x: np.ndarray, ids: np.ndarray, nthreads: int = 1) -> np.ndarray:
    """ggml_mul_mat_id(W [I, O, E], x [I, ne11, S], ids [n_ids, S]) -> [S, n_ids, O].

    numpy shapes: W (E, O, row_bytes) uint8, x (S, ne11, I) f32, ids (S, n_ids) i32."""
    E, O, _ = W.shape
    S, ne11, I = x.shape
    n_ids = ids.shape[1]
    W = np.ascontiguousarray(W)
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    dst = np.zeros((S, n_ids, O), np.float32)
    t0 = tensor(t, [I, O, E], W)
    t1 = tensor(TYPE_F32, [I, ne11, S], x)
    ti = tensor(TYPE_I32, [n_ids, S], ids)
    td = tensor(TYPE_F32, [O, n_ids, S], dst)
    rc = lib().zmo_mul_mat_id(C.byref(t0), C.byref(t1), C.byref(ti), C.byref(td), nthreads)
    if rc != 0:
        raise ValueError(f"zmo_mul_mat_id rc={rc}")
    return dst


class _RouterSpec(C.Structure):
    _fields_ = [("gating", C.c_int), ("n_experts", C.c_int), ("topk", C.c_int), ("n_groups", C.c_int),
                ("n_groups_used", C.c_int), ("weights_norm", C.c_int), ("weights_scale", C.c_float)]


def router(logits: np.ndarray, topk: int, gating: int = GATING_SOFTMAX, logit_bias=None, sel_bias=None,
           n_groups: int = 0, n_groups_used: int = 0, weights_norm: bool = False, weights_scale: float = 0.0):
    logits = np.ascontiguousarray(logits, np.float32)
    S, E = logits.shape
    spec = _RouterSpec(gating, E, topk, n_groups, n_groups_used, int(weights_norm), weights_scale)
    ids = np.zeros((S, topk), np.int32)
    w = np.zeros((S, topk), np.float32)
    lb = None if logit_bias is None else np.ascontiguousarray(logit_bias, np.float32)
    sb = None if sel_bias is None else np.ascontiguousarray(sel_bias, np.float32)
    lib().zmo_router(C.byref(spec), _p(logits), None if lb is None else _p(lb), None if sb is None else _p(sb), S,
                     _p(ids), _p(w))
    return ids, w


def apply_slot_table(route_map: np.ndarray, ids: np.ndarray, w: np.ndarray, route_mask=None):
    ids = np.ascontiguousarray(ids, np.int32).copy()
    w = np.ascontiguousarray(w, np.float32).copy()
    rm = np.ascontiguousarray(route_map, np.int32)
    mk = None if route_mask is None else np.ascontiguousarray(route_mask, np.float32)
    lib().zmo_apply_slot_table(_p(rm), None if mk is None else _p(mk), ids.shape[0], ids.shape[1], _p(ids), _p(w))
    return ids, w


def bucket(ids: np.ndarray, E: int):
    ids = np.ascontiguousarray(ids, np.int32)
    S, K = ids.shape
    counts = np.zeros(E, np.int32)
    offs = np.zeros(E + 1, np.int32)
    pairs = np.zeros(max(1, S * K), np.int32)
    n = lib().zmo_bucket(_p(ids), S, K, E, _p(counts), _p(offs), _p(pairs))
    return counts, offs, pairs[:n]


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().zmo_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


class _MoeDesc(C.Structure):
    _fields_ = [("H", C.c_int), ("F", C.c_int), ("E", C.c_int), ("K", C.c_int), ("S", C.c_int),
                ("type_gate", C.c_int), ("type_up", C.c_int), ("type_down", C.c_int),
                ("w_gate", C.c_void_p), ("w_up", C.c_void_p), ("w_down", C.c_void_p),
                ("F_shared", C.c_int), ("type_shared", C.c_int),
                ("ws_gate", C.c_void_p), ("ws_up", C.c_void_p), ("ws_down", C.c_void_p)]


def moe_forward(x, ids, weights, tg, tu, td, Wg, Wu, Wd, shared=None, nthreads: int = 1,
                fast: bool = False) -> np.ndarray:
    """Routed layer: x (S,H) f32, ids/weights (S,K); Wg/Wu (E,F,rowH), Wd (E,H,rowF) uint8.
    shared = (type, F_shared, Sg, Su, Sd) or None.  fast: the AVX-512 CPU
    baseline (zmo_moe_forward_fast, bit-identical, no shared expert)."""
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    weights = np.ascontiguousarray(weights, np.float32)
    S, H = x.shape
    K = ids.shape[1]
    E, F = Wg.shape[0], Wg.shape[1]
    d = _MoeDesc(H, F, E, K, S, tg, tu, td, _p(Wg), _p(Wu), _p(Wd), 0, 0, None, None, None)
    if shared is not None:
        ts, Fs, Sg, Su, Sd = shared
        d.F_shared, d.type_shared = Fs, ts
        d.ws_gate, d.ws_up, d.ws_down = _p(Sg), _p(Su), _p(Sd)
    out = np.zeros((S, H), np.float32)
    if fast:
        assert shared is None, "the CPU baseline has no shared expert"
        lib().zmo_moe_forward_fast(C.byref(d), _p(x), _p(ids), _p(weights), _p(out), nthreads)
    else:
        lib().zmo_moe_forward(C.byref(d), _p(x), _p(ids), _p(weights), _p(out), nthreads)
    return out


def has_avx512() -> bool:
    return bool(lib().zmo_cpu_has_avx512())


def router_gemv(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    E, H = W.shape
    S = x.shape[0]
    out = np.zeros((S, E), np.float32)
    lib().zmo_router_gemv(_p(W), _p(x), H, E, S, _p(out))
    return out


# ---------------------------------------------------------------- FP32-activation path (numpy)
#
# The reference's CUDA executor computes with f32 activations and no Q8_K
# step.  These restatements define the results; the device kernels sum in a
# different order, so parity is to a float tolerance.


def f32_matmul(t: int, W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y[S, O] = x[S, I] . dequant(W[O])^T in float64
    (kernels/quant/kquant_matmul.cu:575-599 launch_<type>_matmul; dequant per
    kquant_matmul.cu:55-92,161-200, iq2_matmul.cu:73-91)."""
    x = np.asarray(x, np.float32)
    Wd = dequantize(t, np.ascontiguousarray(W, np.uint8), x.shape[-1]).astype(np.float64)
    return x.astype(np.float64) @ Wd.T


def f32_matmul_absbound(t: int, W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sum_i |w_oi x_si|: the scale of the float rounding of one output."""
    Wd = dequantize(t, np.ascontiguousarray(W, np.uint8), x.shape[-1]).astype(np.float64)
    return np.abs(np.asarray(x, np.float64)) @ np.abs(Wd).T


def expert_swiglu(g: np.ndarray, u: np.ndarray, clamp: float = 0.0, fused: bool = False):
    """launch_expert_swiglu (kernels/math/expert_activation.cu:31-59): returns
    (prod f32, [n_nan, n_inf]) where a NaN in g or u counts as NaN, else an
    Inf in either counts as Inf.  silu uses the oracle's exp (zmo_expf)."""
    g = np.asarray(g, np.float32).ravel()
    u = np.asarray(u, np.float32).ravel()
    nan = np.isnan(g) | np.isnan(u)
    inf = ~nan & (np.isinf(g) | np.isinf(u))
    out = np.empty_like(g)
    c = np.float32(clamp)
    for i in range(g.size):
        gi, ui = g[i], u[i]
        with np.errstate(all="ignore"):
            if fused:
                if c > 0:
                    gi = np.fmin(gi, c)
                    ui = np.fmax(-c, np.fmin(c, ui))
                out[i] = gi / (np.float32(1.0) + np.float32(expf(float(-gi)))) * ui
            else:
                o = gi / (np.float32(1.0) + np.float32(expf(float(-gi)))) * ui
                if c > 0:
                    o = np.fmax(-c, np.fmin(c, o))
                out[i] = o
    return out, [int(nan.sum()), int(inf.sum())]


def scatter_accum(src: np.ndarray, tok: np.ndarray, dst: np.ndarray, w=None) -> np.ndarray:
    """dst[tok[i]] += w[i] * src[i], tok outside [0, S) skipped
    (kernels/math/expert_accum.cu:22-37; w None: expert_accum.cu:54-60)."""
    dst = np.array(dst, np.float32, copy=True)
    S = dst.shape[0]
    for i, s in enumerate(np.asarray(tok)):
        if 0 <= s < S:
            wt = np.float32(1.0) if w is None else np.float32(w[i])
            dst[s] = (np.float64(wt) * src[i].astype(np.float64) + dst[s]).astype(np.float32)
    return dst


def glm5next_router_topk(logits: np.ndarray, topk: int, bias=None, gating: int = GATING_SOFTMAX,
                         normalize: bool = False, scale: float = 0.0):
    """kernels/models/glm5next_router.cu:33-93, one token at a time: returns
    (row, ids, weights) where row is what the kernel leaves in `logits` (the
    gated probabilities, chosen ones replaced by -FLT_MAX)."""
    L = np.array(logits, np.float32, copy=True)
    S, E = L.shape
    NEG = np.float32(-3.402823466e38)
    ids = np.zeros((S, topk), np.int32)
    ws = np.zeros((S, topk), np.float32)
    b = None if bias is None else np.asarray(bias, np.float32)
    for s in range(S):
        row = L[s]
        if gating == GATING_SOFTMAX:
            mx = np.float32(np.nanmax(row)) if not np.all(np.isnan(row)) else np.float32(np.nan)
            ex = np.array([expf(float(np.float32(v - mx))) for v in row], np.float32)
            total_e = np.float32(0.0)
            for v in ex:
                total_e = np.float32(total_e + v)
            row[:] = ex * (np.float32(1.0) / total_e)
        elif gating == GATING_SIGMOID:
            row[:] = [np.float32(1.0) / (np.float32(1.0) + np.float32(expf(float(-v)))) for v in row]
        elif gating == GATING_SQRT_SOFTPLUS:
            r64 = row.astype(np.float64)
            row[:] = np.sqrt(np.where(r64 > 0, r64 + np.log1p(np.exp(-r64)), np.log1p(np.exp(r64))))
        total = np.float32(0.0)
        for k in range(topk):
            best, best_score = -1, np.float32(0)
            for e in range(E):
                sc = np.float32(row[e] + (b[e] if b is not None else np.float32(0)))
                if best < 0 or sc > best_score or (sc == best_score and e < best):
                    best, best_score = e, sc
            ids[s, k] = best
            ws[s, k] = row[best]
            row[best] = NEG
            total = np.float32(total + ws[s, k])
        if normalize:
            ws[s] = ws[s] * (np.float32(1.0) / np.fmax(total, np.float32(6.103515625e-5)))
        if scale != 0.0:
            ws[s] = ws[s] * np.float32(scale)
    return L, ids, ws


# ---------------------------------------------------------------- expert records (numpy)


def moe_unpack(src: np.ndarray, gate: np.ndarray, up: np.ndarray, down: np.ndarray, count: int, src_stride: int,
               part_bytes, dst_strides=None, slots=None) -> None:
    """In place: record i of `src` (bytes [i*src_stride, +gate+up+down)) is
    split into gate/up/down at expert e*dst_stride, e = i or slots[i]
    (negative: skipped).  kernels/math/ggml_moe_pack.cu:13-60 (unpack) and
    :62-113 (scatter): a plain byte copy per part, parts consecutive in the
    record, nothing outside a part written."""
    gb, ub, db = part_bytes
    strides = dst_strides if dst_strides is not None else part_bytes
    for i in range(count):
        e = i if slots is None else int(slots[i])
        if e < 0:
            continue
        base = i * src_stride
        off = base
        for dst, nbytes, st in ((gate, gb, strides[0]), (up, ub, strides[1]), (down, db, strides[2])):
            dst[e * st:e * st + nbytes] = src[off:off + nbytes]
            off += nbytes


def moe_pack(gate: np.ndarray, up: np.ndarray, down: np.ndarray, experts, src_stride: int, part_bytes,
             dst_strides=None, fill: int = 0) -> np.ndarray:
    """The transfer records the unpack consumes, built the other way round
    (expert rows concatenated, each record padded to src_stride with `fill`)
    -- the inverse used to pin moe_unpack by round trip
    (backends/ggml/ggml_moe_transfer_manager.cpp:700-712 copies one record of
    weight_raw_expert_stride_ bytes per expert)."""
    gb, ub, db = part_bytes
    strides = dst_strides if dst_strides is not None else part_bytes
    recs = []
    for e in experts:
        r = np.concatenate([gate[e * strides[0]:e * strides[0] + gb], up[e * strides[1]:e * strides[1] + ub],
                            down[e * strides[2]:e * strides[2] + db]])
        recs.append(np.concatenate([r, np.full(src_stride - r.size, fill, np.uint8)]))
    return np.concatenate(recs) if recs else np.zeros(0, np.uint8)


# ---------------------------------------------------------------- reference build (oracle/_ref)

_ref = None


def ref_lib():
    """oracle/_ref/libzmref.so: the reference's own bench dot kernels, or None."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        L = C.CDLL(REF_PATH)
        for name in ("zmref_dot_q2_K", "zmref_dot_q4_K"):
            f = getattr(L, name)
            f.restype = C.c_float
            f.argtypes = [C.c_int, C.c_void_p, C.c_void_p]
        _ref = L
    return _ref
