"""Shared builders for the GPU parity tests: the BASELINE configurations
(full size and reduced), device-resident synthetic weights, and the oracle
reference for exactly the experts a batch touches."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

import zm_oracle as O

Q2, Q3, Q4, IQ2 = O.TYPE_Q2_K, O.TYPE_Q3_K, O.TYPE_Q4_K, O.TYPE_IQ2_XXS
Q5, Q6, IQ4, IQ3 = O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_IQ4_XS, O.TYPE_IQ3_XXS


def dev_random_blocks(t: int, rows: int, n: int, seed: int, device="cuda", scale=0.02) -> torch.Tensor:
    """Random valid quantized rows generated on the device: random bytes with
    the fp16 scale fields overwritten by finite values of sensible size."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    nb = n // 256
    bb = O.BLOCK_BYTES[t]
    raw = torch.randint(0, 256, (rows, nb, bb), dtype=torch.uint8, device=device, generator=g)

    def put(off, lo, hi):
        v = (torch.rand((rows, nb), device=device, generator=g) * (hi - lo) + lo).to(torch.float16)
        raw[:, :, off:off + 2] = v.view(torch.uint8).view(rows, nb, 2)

    if t == Q2:
        put(80, 0.5 * scale / 20, 1.5 * scale / 20)
        put(82, 0.5 * scale / 8, 1.5 * scale / 8)
    elif t == Q3:
        put(108, 0.5 * scale / 40, 1.5 * scale / 40)
    elif t == Q4:
        put(0, 0.5 * scale / 200, 1.5 * scale / 200)
        put(2, 0.5 * scale / 60, 1.5 * scale / 60)
    elif t == Q5:
        put(0, 0.5 * scale / 400, 1.5 * scale / 400)
        put(2, 0.5 * scale / 60, 1.5 * scale / 60)
    elif t == Q6:
        put(208, 0.5 * scale / 2000, 1.5 * scale / 2000)
    elif t == IQ4:
        put(0, 0.5 * scale / 2000, 1.5 * scale / 2000)
    elif t == IQ3:
        put(0, 0.5 * scale / 150, 1.5 * scale / 150)
    else:
        put(0, 0.5 * scale / 40, 1.5 * scale / 40)
    return raw.view(rows, nb * bb)


@dataclass
class Cfg:
    name: str
    H: int
    F: int
    E: int            # router experts
    K: int
    S: int
    tg: int
    td: int
    gating: int = O.GATING_SOFTMAX
    n_slots: Optional[int] = None   # slot pool (config 5)
    groups: int = 0
    groups_used: int = 0
    norm: bool = False
    scale: float = 0.0
    logit_bias_sd: float = 0.0
    F_shared: int = 0
    t_shared: int = Q4
    router_gemv: bool = False
    sel_bias_sd: float = 0.0        # selection-only bias N(0, sd) (moe_routed_ggml.hpp:77-104)
    route_mask: bool = False        # non-binary per-expert mask with the slot table (moe_partial_route_ggml.hpp:21-35)


CONFIGS = {
    "c1": Cfg("c1", 2048, 768, 128, 8, 1, Q4, Q4),
    "c2": Cfg("c2", 4096, 1536, 128, 8, 1, Q2, Q3),
    "c3": Cfg("c3", 4096, 1536, 128, 8, 512, Q4, Q4, logit_bias_sd=1.5),
    "c4": Cfg("c4", 5120, 1536, 160, 8, 4, IQ2, IQ2),
    "c5": Cfg("c5", 7168, 2048, 256, 8, 1, Q2, Q2, gating=O.GATING_SIGMOID, n_slots=96, groups=8, groups_used=4,
              norm=True, scale=2.5, F_shared=2048, t_shared=Q4, router_gemv=True),
}


def reduced(c: Cfg, **kw) -> Cfg:
    d = dict(c.__dict__)
    d.update(kw)
    return Cfg(**d)


class Built:
    """Device tensors + host copies of everything the oracle needs."""

    def __init__(self, c: Cfg, seed: int = 1):
        self.c = c
        dev = "cuda"
        NS = c.n_slots or c.E
        self.NS = NS
        self.wg = dev_random_blocks(c.tg, NS * c.F, c.H, seed + 1).view(NS, c.F, -1)
        self.wu = dev_random_blocks(c.tg, NS * c.F, c.H, seed + 2).view(NS, c.F, -1)
        self.wd = dev_random_blocks(c.td, NS * c.H, c.F, seed + 3).view(NS, c.H, -1)
        rng = np.random.default_rng(seed)
        self.x = rng.standard_normal((c.S, c.H)).astype(np.float32)
        self.logits = rng.standard_normal((c.S, c.E)).astype(np.float32)
        self.logit_bias = (rng.standard_normal(c.E) * c.logit_bias_sd).astype(np.float32) if c.logit_bias_sd else None
        self.route_map = None
        if c.n_slots:
            perm = rng.permutation(c.E)
            rmap = np.full(c.E, -1, np.int32)
            rmap[perm[: c.n_slots]] = np.arange(c.n_slots, dtype=np.int32)
            self.route_map = rmap
        self.sel_bias = (rng.standard_normal(c.E) * c.sel_bias_sd).astype(np.float32) if c.sel_bias_sd else None
        self.route_mask = None
        if c.route_mask:
            # resident experts: weights in [0.25, 1.25) with every 7th one 0 (the
            # route runs, its output is weighted out); others: arbitrary values
            # that the slot table's -1 must override
            m = rng.uniform(0.25, 1.25, c.E).astype(np.float32)
            m[::7] = 0.0
            self.route_mask = m
        self.router_w = None
        if c.router_gemv:
            self.router_w = (rng.standard_normal((c.E, c.H)) * 0.02).astype(np.float32)
        self.shared = None
        if c.F_shared:
            self.sg = dev_random_blocks(c.t_shared, c.F_shared, c.H, seed + 4)
            self.su = dev_random_blocks(c.t_shared, c.F_shared, c.H, seed + 5)
            self.sd = dev_random_blocks(c.t_shared, c.H, c.F_shared, seed + 6)

    def layer(self):
        import zeromoe_amd as Z

        c = self.c
        t = lambda a, dt=None: None if a is None else torch.from_numpy(a).cuda()
        return Z.MoELayer(H=c.H, F=c.F, n_experts=c.E, topk=c.K, type_gate=c.tg, type_up=c.tg, type_down=c.td,
                          w_gate=self.wg, w_up=self.wu, w_down=self.wd,
                          gating={0: "softmax", 1: "sigmoid", 2: "sqrt_softplus"}[c.gating],
                          n_groups=c.groups, n_groups_used=c.groups_used, weights_norm=c.norm,
                          weights_scale=c.scale, router_w=t(self.router_w), logit_bias=t(self.logit_bias),
                          sel_bias=t(self.sel_bias), route_map=t(self.route_map), route_mask=t(self.route_mask),
                          F_shared=c.F_shared, type_shared=c.t_shared,
                          ws_gate=self.sg if c.F_shared else None, ws_up=self.su if c.F_shared else None,
                          ws_down=self.sd if c.F_shared else None)

    def oracle_logits(self):
        if self.router_w is not None:
            return O.router_gemv(self.router_w, self.x)
        return self.logits

    def oracle_route(self, logits=None):
        c = self.c
        lg = self.oracle_logits() if logits is None else logits
        ids, w = O.router(lg, c.K, c.gating, self.logit_bias, self.sel_bias, c.groups, c.groups_used, c.norm,
                          c.scale)
        if self.route_map is not None:
            ids, w = O.apply_slot_table(self.route_map, ids, w, self.route_mask)
        return ids, w

    def oracle_forward(self, ids, w, nthreads=8):
        """Reference layer output for given (slot) ids/weights, using host copies
        of only the touched experts."""
        c = self.c
        used = sorted(set(int(v) for v in ids.reshape(-1) if v >= 0))
        remap = {e: i for i, e in enumerate(used)}
        rid = np.array([[remap.get(int(v), -1) for v in row] for row in ids], np.int32)
        if used:
            sel = torch.tensor(used, device="cuda")
            Wg = self.wg.index_select(0, sel).cpu().numpy()
            Wu = self.wu.index_select(0, sel).cpu().numpy()
            Wd = self.wd.index_select(0, sel).cpu().numpy()
        else:
            Wg = np.zeros((1,) + tuple(self.wg.shape[1:]), np.uint8)
            Wu, Wd = Wg.copy(), np.zeros((1,) + tuple(self.wd.shape[1:]), np.uint8)
        shared = None
        if c.F_shared:
            shared = (c.t_shared, c.F_shared, self.sg.cpu().numpy(), self.su.cpu().numpy(), self.sd.cpu().numpy())
        return O.moe_forward(self.x, rid, w, c.tg, c.tg, c.td, Wg, Wu, Wd, shared=shared, nthreads=nthreads)


    def requant_slack(self, ids, w, tie: float = 2e-4) -> np.ndarray:
        """Per token: the largest output change that Q8_K rounding ties of the
        routed activation (SwiGLU output, re-quantized before the down
        projection) can cause.  An element whose scaled value x*iscale lies
        within `tie` of a half-integer rounds either way under another valid
        float summation order of the gate/up dots (ggml's own backends differ in
        that order); flipping it moves the output by d_x * |W_down column| *
        |route weight|.  The bound sums these over every tied element."""
        c = self.c
        used = sorted(set(int(v) for v in ids.reshape(-1) if v >= 0))
        slack = np.zeros(c.S, np.float64)
        if not used:
            return slack
        remap = {e: i for i, e in enumerate(used)}
        rid = np.array([[remap.get(int(v), -1) for v in row] for row in ids], np.int32)
        sel = torch.tensor(used, device="cuda")
        Wg = self.wg.index_select(0, sel).cpu().numpy()
        Wu = self.wu.index_select(0, sel).cpu().numpy()
        Wd = self.wd.index_select(0, sel).cpu().numpy()
        x = self.x[:, None, :]
        g = O.mul_mat_id(c.tg, Wg, x, rid, nthreads=8)
        u = O.mul_mat_id(c.tg, Wu, x, rid, nthreads=8)
        act = O.swiglu(g, u).reshape(c.S, c.K, c.F // O.QK_K, O.QK_K).astype(np.float64)
        # ggml quantize_row_q8_K: iscale = -127 / (value of largest magnitude)
        idx = np.abs(act).argmax(-1)
        mx = np.take_along_axis(act, idx[..., None], -1)
        iscale = np.where(mx != 0, -127.0 / np.where(mx != 0, mx, 1.0), 0.0)
        v = act * iscale
        tied = np.abs(np.abs(v - np.floor(v)) - 0.5) < tie
        dx = np.where(mx != 0, 1.0 / np.where(iscale != 0, iscale, 1.0), 0.0)  # per block d of the act row
        wdabs = {}
        for s, k in zip(*np.nonzero(tied.any(axis=(2, 3)))):
            e = rid[s, k]
            if e < 0:
                continue
            if e not in wdabs:
                wdabs[e] = np.abs(O.dequantize(c.td, Wd[e], c.F))  # (H, F)
            cols = np.nonzero(tied[s, k].reshape(-1))[0]
            dcol = np.abs(dx[s, k, cols // O.QK_K, 0])
            slack[s] += abs(float(w[s, k])) * (wdabs[e][:, cols] * dcol[None, :]).sum(1).max()
        return slack


# (label, per-token-norm max error, element-wise max relative error, elements
# counted) of every checked layer output, printed at the end of a pytest run
LAYER_ERRORS: list = []


def assert_close_layer(got: np.ndarray, ref: np.ndarray, rtol: float = 1e-3, slack=None, label: str = ""):
    """Layer-output tolerance: per token, max |got - ref| <= rtol * max |ref|
    (the 1e-3 max relative error of the north star, taken against the token's
    output scale so isolated near-zero outputs do not dominate).  `slack`
    (a callable returning a per-token bound, see Built.requant_slack) is
    consulted only for tokens over the tolerance: their excess must be
    explained by activation re-quantization ties.

    Reported beside it (not asserted): the element-wise max relative error
    |got - ref| / |ref| over the elements with |ref| >= 1e-2 * max |ref| of
    their token, the reading of "max relative error" that excludes outputs
    near zero, where a relative error is dominated by cancellation."""
    assert got.shape == ref.shape
    assert np.isfinite(got).all()
    g64, r64 = got.astype(np.float64), ref.astype(np.float64)
    scale = np.abs(r64).max(axis=-1, keepdims=True)
    big = np.abs(r64) >= 1e-2 * scale
    elem = float((np.abs(g64 - r64)[big] / np.abs(r64)[big]).max()) if big.any() else 0.0
    tok = float((np.abs(g64 - r64).max(axis=-1) / np.maximum(scale[..., 0], 1e-30)).max())
    LAYER_ERRORS.append((label, tok, elem, int(big.sum())))
    bound = None
    for s in range(ref.shape[0]):
        scale_s = float(np.abs(ref[s]).max())
        err = float(np.abs(got[s] - ref[s]).max())
        if err <= rtol * max(scale_s, 1e-30):
            continue
        assert slack is not None, (s, err, scale_s)
        if bound is None:
            bound = slack()
        assert err <= rtol * scale_s + bound[s], (s, err, scale_s, float(bound[s]))
    return tok, elem
