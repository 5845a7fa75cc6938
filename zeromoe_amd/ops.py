"""Torch-facing wrappers over the C ABI (device tensors in, device tensors out)."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Optional

import torch

from ._lib import ZmColdLaneDesc, ZmColdLaneStats, ZmExpertScratch, ZmMoeLayer, ZmRouterSpec, ZmTensor, check, lib

GGML_TYPES = {"f32": 0, "q2_K": 10, "q3_K": 11, "q4_K": 12, "q5_K": 13, "q6_K": 14, "q8_K": 15, "iq2_xxs": 16, "iq3_xxs": 18, "iq4_xs": 23, "i32": 26}
BLOCK_BYTES = {10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 15: 292, 16: 66, 18: 98, 23: 136}
QK_K = 256
GATING = {"softmax": 0, "sigmoid": 1, "sqrt_softplus": 2}


def row_size(t: int, n: int) -> int:
    return n * 4 if t in (0, 26) else (n // QK_K) * BLOCK_BYTES[t]


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor, name: str):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")


def init() -> None:
    check(lib().zm_init(), "zm_init")


def set_iq2xxs_grid(grid) -> None:
    import numpy as np

    g = np.ascontiguousarray(grid, dtype=np.uint64)
    assert g.shape == (256,)
    check(lib().zm_set_iq2xxs_grid(g.ctypes.data), "zm_set_iq2xxs_grid")


def set_iq4nl_table(table) -> None:
    """Load the IQ4_XS value table (16 int8) for the current device."""
    import numpy as np

    t = np.ascontiguousarray(np.asarray(table, np.int8))
    if t.shape != (16,):
        raise ValueError("the IQ4_XS table has 16 entries")
    check(lib().zm_set_iq4nl_table(t.ctypes.data), "zm_set_iq4nl_table")


def set_iq3xxs_grid(grid) -> None:
    """Load the IQ3_XXS grid (256 uint32) for the current device."""
    import numpy as np

    g = np.ascontiguousarray(np.asarray(grid, np.uint32))
    if g.shape != (256,):
        raise ValueError("the IQ3_XXS grid has 256 entries")
    check(lib().zm_set_iq3xxs_grid(g.ctypes.data), "zm_set_iq3xxs_grid")


def builtin_iq3xxs_grid():
    import numpy as np

    g = np.zeros(256, np.uint32)
    lib().zm_iq3xxs_builtin_grid(g.ctypes.data)
    return g


def builtin_iq4nl_table():
    import numpy as np

    t = np.zeros(16, np.int8)
    lib().zm_iq4nl_builtin_table(t.ctypes.data)
    return t


def builtin_iq2xxs_grid():
    import numpy as np

    g = np.zeros(256, np.uint64)
    lib().zm_iq2xxs_builtin_grid(g.ctypes.data)
    return g


def _tensor(t: int, x: torch.Tensor, ne_order) -> ZmTensor:
    """ggml descriptor of a torch tensor whose dims are given slowest-first;
    ne/nb are written fastest-first.  For quantized rows the last torch dim
    is bytes and counts as `ne0` weights."""
    T = ZmTensor()
    T.type = t
    shape = list(x.shape)
    stride = list(x.stride())
    es = x.element_size()
    nd = len(shape)
    ne = [1, 1, 1, 1]
    nb = [0, 0, 0, 0]
    for i in range(nd):
        ne[i] = shape[nd - 1 - i]
        nb[i] = stride[nd - 1 - i] * es
    if t in BLOCK_BYTES:  # quantized: ne0 counts weights, nb0 = block bytes
        ne[0] = ne_order
        nb[0] = BLOCK_BYTES[t]
    for i in range(nd, 4):
        nb[i] = nb[i - 1] * ne[i - 1]
    for i in range(4):
        T.ne[i] = ne[i]
        T.nb[i] = nb[i]
    T.data = x.data_ptr()
    return T


def mul_mat_id(W: torch.Tensor, wtype: int, n_in: int, x: torch.Tensor, ids: torch.Tensor,
               out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """ggml_mul_mat_id: W (E, O, row_bytes) uint8 of type `wtype` holding rows of
    `n_in` weights; x (S, ne11, n_in) f32; ids (S, n_ids) int32 -> (S, n_ids, O)."""
    for t, n in ((W, "W"), (x, "x"), (ids, "ids")):
        _dev(t, n)
    E, O, _ = W.shape
    S, ne11, I = x.shape
    n_ids = ids.shape[1]
    if out is None:
        out = torch.empty((S, n_ids, O), dtype=torch.float32, device=x.device)
    tw = _tensor(wtype, W, n_in)
    tx = _tensor(0, x, None)
    ti = _tensor(26, ids, None)
    ty = _tensor(0, out, None)
    st = _stream(stream)
    bind_mmid_workspace(st, lib().zm_mul_mat_id_workspace_size(C.byref(tw), C.byref(tx), C.byref(ti), C.byref(ty)),
                        x.device)
    ok = lib().zm_mul_mat_id(C.byref(tw), C.byref(tx), C.byref(ti), C.byref(ty), st, 1)
    if ok != 1:
        raise RuntimeError(f"zm_mul_mat_id declined: {lib().zm_last_error().decode()}")
    return out


# stream handle -> device buffer bound as zm_mul_mat_id's workspace (the role
# of a ggml backend context's per-stream scratch)
_MMID_WS: dict = {}


def bind_mmid_workspace(stream: int, need: int, device) -> None:
    """Bind (or grow) the caller-owned workspace of `stream`.  Growing happens
    here, outside the op: a buffer freed by torch is reused only by work
    ordered after it on the same stream."""
    cur = _MMID_WS.get((device.index, stream))
    if cur is not None and cur.numel() >= need:
        return
    buf = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=device)
    check(lib().zm_mul_mat_id_set_workspace(stream, buf.data_ptr(), buf.numel()), "zm_mul_mat_id_set_workspace")
    _MMID_WS[(device.index, stream)] = buf


def mul_mat_id_supported(W, wtype, n_in, x, ids, out, stream=None) -> bool:
    """The hook's capability query (execute = 0).  The library answers it for
    the smallest workspace bound on the device, so the shape's workspace is
    bound to `stream` first (as mul_mat_id would); a shape the library
    declines has a workspace size of 0 and is answered False."""
    tw, tx, ti, ty = _tensor(wtype, W, n_in), _tensor(0, x, None), _tensor(26, ids, None), _tensor(0, out, None)
    need = lib().zm_mul_mat_id_workspace_size(C.byref(tw), C.byref(tx), C.byref(ti), C.byref(ty))
    if need == 0:
        return False
    bind_mmid_workspace(_stream(stream), need, x.device)
    return lib().zm_mul_mat_id(C.byref(tw), C.byref(tx), C.byref(ti), C.byref(ty), None, 0) == 1


def quantize_q8_K(x: torch.Tensor, stream=None) -> torch.Tensor:
    _dev(x, "x")
    x = x.contiguous()
    rows, n = x.shape
    y = torch.empty((rows, (n // QK_K) * 292), dtype=torch.uint8, device=x.device)
    check(lib().zm_quantize_q8_K(x.data_ptr(), rows, n, y.data_ptr(), _stream(stream)), "zm_quantize_q8_K")
    return y


def _spec(E, topk, gating, n_groups, n_groups_used, weights_norm, weights_scale) -> ZmRouterSpec:
    g = GATING[gating] if isinstance(gating, str) else int(gating)
    return ZmRouterSpec(g, E, topk, n_groups, n_groups_used, int(weights_norm), float(weights_scale))


def router(logits: torch.Tensor, topk: int, gating="softmax", logit_bias=None, sel_bias=None, n_groups: int = 0,
           n_groups_used: int = 0, weights_norm: bool = False, weights_scale: float = 0.0, route_map=None,
           route_mask=None, stream=None):
    _dev(logits, "logits")
    logits = logits.contiguous()
    S, E = logits.shape
    ids = torch.empty((S, topk), dtype=torch.int32, device=logits.device)
    w = torch.empty((S, topk), dtype=torch.float32, device=logits.device)
    spec = _spec(E, topk, gating, n_groups, n_groups_used, weights_norm, weights_scale)
    check(lib().zm_router(C.byref(spec), logits.data_ptr(), _p(logit_bias), _p(sel_bias), _p(route_map),
                          _p(route_mask), S, ids.data_ptr(), w.data_ptr(), _stream(stream)), "zm_router")
    return ids, w


def bucket(ids: torch.Tensor, E: int, stream=None):
    _dev(ids, "ids")
    ids = ids.contiguous()
    S, K = ids.shape
    dev = ids.device
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offs = torch.empty(E + 1, dtype=torch.int32, device=dev)
    pairs = torch.full((max(1, S * K),), -1, dtype=torch.int32, device=dev)
    active = torch.full((E,), -1, dtype=torch.int32, device=dev)
    n_active = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib().zm_bucket(ids.data_ptr(), S, K, E, counts.data_ptr(), offs.data_ptr(), pairs.data_ptr(),
                          active.data_ptr(), n_active.data_ptr(), _stream(stream)), "zm_bucket")
    return counts, offs, pairs, active, n_active


def block_dots(wtype: int, w_row: torch.Tensor, x: torch.Tensor, stream=None):
    n = x.numel()
    isum = torch.empty(n // QK_K, dtype=torch.int32, device=x.device)
    imin = torch.empty(n // QK_K, dtype=torch.int32, device=x.device)
    check(lib().zm_block_dots(wtype, w_row.data_ptr(), x.data_ptr(), n, isum.data_ptr(), imin.data_ptr(),
                              _stream(stream)), "zm_block_dots")
    return isum, imin


@dataclass
class MoELayer:
    """One routed MoE FFN layer on device.

    Weights are uint8 tensors in ggml layout: gate/up (n_slots, F, row_bytes(H)),
    down (n_slots, H, row_bytes(F)); the shared expert (optional) the same
    without the expert axis."""

    H: int
    F: int
    n_experts: int
    topk: int
    type_gate: int
    type_up: int
    type_down: int
    w_gate: torch.Tensor
    w_up: torch.Tensor
    w_down: torch.Tensor
    gating: str = "softmax"
    n_groups: int = 0
    n_groups_used: int = 0
    weights_norm: bool = False
    weights_scale: float = 0.0
    router_w: Optional[torch.Tensor] = None
    logit_bias: Optional[torch.Tensor] = None
    sel_bias: Optional[torch.Tensor] = None
    route_map: Optional[torch.Tensor] = None
    route_mask: Optional[torch.Tensor] = None
    F_shared: int = 0
    type_shared: int = 0
    ws_gate: Optional[torch.Tensor] = None
    ws_up: Optional[torch.Tensor] = None
    ws_down: Optional[torch.Tensor] = None
    _ws: dict = field(default_factory=dict, repr=False)

    def desc(self) -> ZmMoeLayer:
        cached = self._ws.get("desc")
        if cached is not None:
            return cached
        d = ZmMoeLayer()
        d.H, d.F, d.n_slots = self.H, self.F, self.w_gate.shape[0]
        d.router = _spec(self.n_experts, self.topk, self.gating, self.n_groups, self.n_groups_used,
                         self.weights_norm, self.weights_scale)
        d.type_gate, d.type_up, d.type_down = self.type_gate, self.type_up, self.type_down
        d.w_gate, d.w_up, d.w_down = _p(self.w_gate), _p(self.w_up), _p(self.w_down)
        d.router_w, d.logit_bias, d.sel_bias = _p(self.router_w), _p(self.logit_bias), _p(self.sel_bias)
        d.route_map, d.route_mask = _p(self.route_map), _p(self.route_mask)
        d.F_shared, d.type_shared = self.F_shared, self.type_shared
        d.ws_gate, d.ws_up, d.ws_down = _p(self.ws_gate), _p(self.ws_up), _p(self.ws_down)
        self._ws["desc"] = d  # tensors are fixed for the layer's lifetime
        return d

    def workspace(self, S: int, device) -> torch.Tensor:
        if S not in self._ws:
            d = self.desc()
            n = lib().zm_moe_workspace_size(C.byref(d), S)
            if n == 0:
                raise RuntimeError(f"zm_moe_workspace_size: {lib().zm_last_error().decode()}")
            self._ws[S] = torch.zeros(n, dtype=torch.uint8, device=device)  # sync words start at zero
        return self._ws[S]

    def forward(self, x: torch.Tensor, logits: Optional[torch.Tensor] = None, out=None, ids=None, weights=None,
                stream=None):
        _dev(x, "x")
        S = x.shape[0]
        dev = x.device
        if out is None:
            out = torch.empty((S, self.H), dtype=torch.float32, device=dev)
        if ids is None:
            ids = torch.empty((S, self.topk), dtype=torch.int32, device=dev)
        if weights is None:
            weights = torch.empty((S, self.topk), dtype=torch.float32, device=dev)
        ws = self.workspace(S, dev)
        d = self.desc()
        check(lib().zm_moe_forward(C.byref(d), x.data_ptr(), _p(logits), S, out.data_ptr(), ids.data_ptr(),
                                   weights.data_ptr(), ws.data_ptr(), ws.numel(), _stream(stream)), "zm_moe_forward")
        return out, ids, weights

    def status(self, S: int, stream=None) -> int:
        """0 when the last decode launches on this workspace completed normally."""
        d = self.desc()
        return lib().zm_moe_status(C.byref(d), S, self._ws[S].data_ptr(), _stream(stream))


# ---------------------------------------------------------------- FP32-activation path


def f32_matmul(W: torch.Tensor, wtype: int, n_in: int, x: torch.Tensor, out=None, stream=None) -> torch.Tensor:
    """y[S, O] = x[S, n_in] . dequant(W)^T with f32 activations (no Q8_K step);
    W (O, row_bytes) uint8 holding rows of type `wtype`."""
    _dev(W, "W")
    _dev(x, "x")
    x = x.contiguous()
    S = x.shape[0]
    O = W.shape[0]
    if out is None:
        out = torch.empty((S, O), dtype=torch.float32, device=x.device)
    check(lib().zm_f32_matmul(wtype, out.data_ptr(), x.data_ptr(), W.data_ptr(), S, n_in, O, _stream(stream)),
          "zm_f32_matmul")
    return out


def mul_mat_id_f32(W: torch.Tensor, wtype: int, n_in: int, x: torch.Tensor, ids: torch.Tensor,
                   out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """The FP32 MUL_MAT_ID hook: W (E, O, row_bytes), x (S, ne11, n_in), ids (S, n_ids) -> (S, n_ids, O)."""
    for t, n in ((W, "W"), (x, "x"), (ids, "ids")):
        _dev(t, n)
    O = W.shape[1]
    S, n_ids = ids.shape
    if out is None:
        out = torch.empty((S, n_ids, O), dtype=torch.float32, device=x.device)
    tw, tx, ti, ty = _tensor(wtype, W, n_in), _tensor(0, x, None), _tensor(26, ids, None), _tensor(0, out, None)
    if lib().zm_mul_mat_id_f32(C.byref(tw), C.byref(tx), C.byref(ti), C.byref(ty), _stream(stream), 1) != 1:
        raise RuntimeError(f"zm_mul_mat_id_f32 declined: {lib().zm_last_error().decode()}")
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor, clamp: float = 0.0, fused: bool = False, bad=None, stream=None):
    """launch_expert_swiglu; `bad` (2 x int32 device tensor) accumulates NaN / Inf counts."""
    _dev(gate, "gate")
    _dev(up, "up")
    gate, up = gate.contiguous(), up.contiguous()
    prod = torch.empty_like(gate)
    lib().launch_expert_swiglu(prod.data_ptr(), gate.data_ptr(), up.data_ptr(), gate.numel(), float(clamp),
                               int(fused), _p(bad), _stream(stream))
    return prod


def scatter_accum(src: torch.Tensor, tok: torch.Tensor, dst: torch.Tensor, w: Optional[torch.Tensor] = None,
                  stream=None) -> torch.Tensor:
    """dst[tok[i]] += w[i] * src[i] (in place; w None: unweighted add)."""
    n, D = src.shape
    S = dst.shape[0]
    if w is None:
        lib().launch_expert_scatter_add(src.data_ptr(), tok.data_ptr(), dst.data_ptr(), n, D, S, _stream(stream))
    else:
        lib().launch_expert_scatter_accum(src.data_ptr(), tok.data_ptr(), w.data_ptr(), dst.data_ptr(), n, D, S,
                                          _stream(stream))
    return dst


def glm5next_router_topk(logits: torch.Tensor, topk: int, bias=None, gating="softmax", normalize: bool = False,
                         scale: float = 0.0, stream=None):
    """launch_glm5next_router_topk; `logits` (S, E) is overwritten (probs, chosen ones -FLT_MAX)."""
    _dev(logits, "logits")
    assert logits.is_contiguous()
    S, E = logits.shape
    ids = torch.empty((S, topk), dtype=torch.int32, device=logits.device)
    w = torch.empty((S, topk), dtype=torch.float32, device=logits.device)
    g = GATING[gating] if isinstance(gating, str) else int(gating)
    lib().launch_glm5next_router_topk(logits.data_ptr(), _p(bias), ids.data_ptr(), w.data_ptr(), S, E, topk, g,
                                      int(normalize), float(scale), _stream(stream))
    return ids, w


class ExpertExecutor:
    """The per-expert issue / finish_stage1 / finish_stage2 pipeline over one
    device slab [gate | up | down] (uint8 tensor), host activations in and out."""

    def __init__(self):
        self.s = ZmExpertScratch()
        self.s.device_id = -1

    def run(self, slab: torch.Tensor, up_offset: int, down_offset: int, types, x_host, D: int, F: int,
            clamp: float = 0.0, fused: bool = False, stream=None):
        import numpy as np

        x_host = np.ascontiguousarray(x_host, dtype=np.float32)
        S = x_host.shape[0]
        st = _stream(stream)
        L = lib()
        check(L.zm_expert_ffn_issue(C.byref(self.s), slab.data_ptr(), up_offset, types[0], types[1],
                                    x_host.ctypes.data, S, D, F, None, st), "zm_expert_ffn_issue")
        check(L.zm_expert_ffn_finish_stage1(C.byref(self.s), slab.data_ptr(), down_offset, types[2], S, D, F,
                                            float(clamp), int(fused), st), "zm_expert_ffn_finish_stage1")
        out = np.empty((S, D), np.float32)
        check(L.zm_expert_ffn_finish_stage2(C.byref(self.s), out.ctypes.data, S, D, st),
              "zm_expert_ffn_finish_stage2")
        return out

    def bad_counts(self, reset: bool = False):
        import numpy as np

        c = np.zeros(2, np.int32)
        check(lib().zm_expert_bad_counts(C.byref(self.s), c.ctypes.data, int(reset)), "zm_expert_bad_counts")
        return c

    def release(self):
        lib().zm_expert_scratch_release(C.byref(self.s))


# ---------------------------------------------------------------- expert records


def moe_unpack(src: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, count: int,
               src_stride: int, part_bytes, dst_strides=None, slots: Optional[torch.Tensor] = None,
               stream=None) -> None:
    """Unpack `count` expert-major [gate | up | down] records of `src` (uint8,
    record i at byte i*src_stride) into the planar per-expert tensors `gate`,
    `up`, `down` (uint8; expert e at byte e*dst_stride).  Record i lands at
    expert i, or at slots[i] (int32 device tensor; negative = skip).
    part_bytes = (gate_bytes, up_bytes, down_bytes); dst_strides defaults to
    part_bytes.  With slots, every slot must be below the number of experts
    the destinations hold (not checked: reading slots would synchronise).  launch_ggml_moe_unpack[_scatter]
    (/root/reference/kernels/math/ggml_moe_pack.cu:127-179)."""
    for t, n in ((src, "src"), (gate, "gate"), (up, "up"), (down, "down")):
        _dev(t, n)
    gb, ub, db = (int(b) for b in part_bytes)
    gs, us, ds = (int(b) for b in (dst_strides if dst_strides is not None else part_bytes))
    if count > 0:
        if (count - 1) * src_stride + gb + ub + db > src.numel():
            raise ValueError("src holds fewer than `count` records")
        # expert slots every destination can hold; slot values are the caller's
        # contract (checking them here would synchronise the stream)
        cap = min(t.numel() // st if st else (1 << 62) for t, st, b in ((gate, gs, gb), (up, us, ub), (down, ds, db))
                  if b > 0)
        if any(b > st for b, st in ((gb, gs), (ub, us), (db, ds)) if b > 0):
            raise ValueError("a destination stride is smaller than its part")
        if slots is not None:
            _dev(slots, "slots")
            if slots.dtype != torch.int32 or slots.numel() < count:
                raise ValueError("slots must be int32 with at least `count` entries")
        elif count > cap:
            raise ValueError("destination tensors too small for `count` experts")
    if slots is None:
        rc = lib().launch_ggml_moe_unpack(src.data_ptr(), gate.data_ptr(), up.data_ptr(), down.data_ptr(), count,
                                          src_stride, gb, ub, db, gs, us, ds, _stream(stream))
    else:
        rc = lib().launch_ggml_moe_unpack_scatter(src.data_ptr(), gate.data_ptr(), up.data_ptr(), down.data_ptr(),
                                                  slots.data_ptr(), count, src_stride, gb, ub, db, gs, us, ds,
                                                  _stream(stream))
    if rc != 0:
        raise RuntimeError(f"launch_ggml_moe_unpack failed ({rc}): {lib().zm_last_error().decode()}")


# ---------------------------------------------------------------- CPU lane of a hot/cold split


class ColdLane:
    """The cold branch of a hot/cold expert split on the host cores
    (zm_cold_lane_*, the reference's EarlyReadyLane,
    models/graph/early_ready_lane.hpp:75-211).  Weights are host numpy uint8
    arrays in ggml layout: gate/up (n_slots, F, row_bytes(H)), down
    (n_slots, H, row_bytes(F)); route_map maps router experts to host slots
    (-1: not cold), route_mask optionally scales their weights."""

    def __init__(self, H, F, n_experts, topk, type_gate, type_up, type_down, w_gate, w_up, w_down, route_map,
                 route_mask=None, max_tokens=1, n_threads=8, scalar=False):
        import numpy as np

        self._keep = [np.ascontiguousarray(w_gate), np.ascontiguousarray(w_up), np.ascontiguousarray(w_down),
                      np.ascontiguousarray(route_map, np.int32)]
        if route_mask is not None:
            self._keep.append(np.ascontiguousarray(route_mask, np.float32))
        d = ZmColdLaneDesc()
        d.H, d.F, d.n_experts, d.topk = H, F, n_experts, topk
        d.type_gate, d.type_up, d.type_down = type_gate, type_up, type_down
        d.w_gate, d.w_up, d.w_down = (a.ctypes.data for a in self._keep[:3])
        d.n_slots = self._keep[0].shape[0]
        d.route_map = self._keep[3].ctypes.data
        d.route_mask = self._keep[4].ctypes.data if route_mask is not None else None
        d.max_tokens, d.n_threads, d.scalar = max_tokens, n_threads, int(scalar)
        self.H, self.topk = H, topk
        self._h = lib().zm_cold_lane_create(C.byref(d))
        if not self._h:
            raise RuntimeError(f"zm_cold_lane_create: {lib().zm_last_error().decode()}")

    def close(self):
        if getattr(self, "_h", None):
            lib().zm_cold_lane_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def compute_host(self, x, ids, weights):
        """The cold branch on host numpy arrays: x (S, H) f32, ids/weights (S, topk)."""
        import numpy as np

        x = np.ascontiguousarray(x, np.float32)
        ids = np.ascontiguousarray(ids, np.int32)
        weights = np.ascontiguousarray(weights, np.float32)
        out = np.zeros_like(x)
        check(lib().zm_cold_lane_compute_host(self._h, x.ctypes.data, ids.ctypes.data, weights.ctypes.data,
                                              x.shape[0], out.ctypes.data), "zm_cold_lane_compute_host")
        return out

    def fork(self, x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, stream=None):
        check(lib().zm_cold_lane_fork(self._h, x.data_ptr(), ids.data_ptr(), weights.data_ptr(), x.shape[0],
                                      _stream(stream)), "zm_cold_lane_fork")

    def merge(self, out: torch.Tensor, stream=None):
        check(lib().zm_cold_lane_merge(self._h, out.data_ptr(), out.shape[0], _stream(stream)), "zm_cold_lane_merge")

    def stats(self) -> dict:
        st = ZmColdLaneStats()
        check(lib().zm_cold_lane_get_stats(self._h, C.byref(st)), "zm_cold_lane_get_stats")
        return {f: getattr(st, f) for f, _ in ZmColdLaneStats._fields_}
