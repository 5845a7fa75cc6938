"""HIP path vs the CPU oracle on identical seeded inputs (MI355X).

Bars: integer/index results bit-exact (Q8_K bytes, per-block integer dots,
expert ids, bucket order); float outputs of the op and the layer within 1e-3
relative (see moe_cases.assert_close_layer for the exact norm)."""
import numpy as np
import pytest
import torch

import zm_oracle as O
from moe_cases import CONFIGS, IQ2, IQ3, IQ4, Q2, Q3, Q4, Q5, Q6, Built, assert_close_layer, dev_random_blocks, reduced

pytestmark = pytest.mark.gpu

TYPES = [Q2, Q3, Q4, Q5, Q6, IQ2, IQ3, IQ4]


@pytest.fixture(scope="module", autouse=True)
def _init():
    import zeromoe_amd as Z

    assert torch.cuda.is_available(), "GPU tests need a device"
    Z.init()
    yield


def _sync():
    torch.cuda.synchronize()


# ------------------------------------------------------------------ Q8_K activation quantization

def test_quantize_q8_K_bit_exact():
    import zeromoe_amd as Z

    rng = np.random.default_rng(0)
    rows = [rng.standard_normal(4096) * 10 ** rng.uniform(-6, 6) for _ in range(20)]
    special = np.zeros(4096)
    special[5], special[700] = -2.0, 2.0          # tie: first wins
    special[1024 + 3], special[1024 + 9] = 3.0, -3.0
    special[2048:2304] = 0.0                      # an all-zero block
    special[3072:3328] = np.linspace(-127, 127, 256)  # exact half-way roundings
    rows.append(special)
    ties = np.zeros(4096)
    ties[10] = np.inf                             # an infinite maximum: q = 0, d = -inf
    ties[256 + 3], ties[256 + 200] = -np.inf, np.inf
    ties[512 + 17], ties[512 + 40] = 5.0, -5.0    # +/- tie across lanes: the first (+5) wins
    ties[768 + 33], ties[768 + 32] = 7.0, -7.0    # +/- tie inside one lane's 16: the first (-7) wins
    ties[1024 + 255], ties[1024 + 240] = -1e-30, 1e-30
    ties[1280:1536] = rng.standard_normal(256)
    ties[1280 + 100] = -np.abs(ties[1280:1536]).max()  # negative maximum with its positive twin later
    ties[1280 + 101] = -ties[1280 + 100]
    rows.append(ties)
    x = np.stack(rows).astype(np.float32)
    got = Z.quantize_q8_K(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = O.quantize_q8_K(x).view(np.uint8).reshape(got.shape)
    np.testing.assert_array_equal(got, ref)


# ------------------------------------------------------------------ per-block integer dots

@pytest.mark.parametrize("t", TYPES)
def test_block_dots_exact(t):
    import zeromoe_amd as Z

    n = 16 * 256
    w = O.random_blocks(t, 3, n, seed=t + 100)
    rng = np.random.default_rng(t)
    for r in range(3):
        x = rng.standard_normal(n).astype(np.float32)
        gi, gm = Z.block_dots(t, torch.from_numpy(w[r]).cuda(), torch.from_numpy(x).cuda())
        ri, rm = O.block_dots(t, w[r], O.quantize_q8_K(x))
        np.testing.assert_array_equal(gi.cpu().numpy(), ri)
        if t in (Q2, Q4):
            np.testing.assert_array_equal(gm.cpu().numpy(), rm)


# ------------------------------------------------------------------ the op

def _mmid_case(t, I, O_, E, ids, ne11, seed):
    import zeromoe_amd as Z

    S, n_ids = ids.shape
    W = O.random_blocks(t, E * O_, I, seed=seed).reshape(E, O_, -1)
    x = np.random.default_rng(seed).standard_normal((S, ne11, I)).astype(np.float32)
    ref = O.mul_mat_id(t, W, x, ids, nthreads=8)
    got = Z.mul_mat_id(torch.from_numpy(W).cuda(), t, I, torch.from_numpy(x).cuda(),
                       torch.from_numpy(ids).cuda()).cpu().numpy()
    return got, ref


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("shape", [(512, 8, 3), (4096, 64, 1), (16384, 64, 1), (768, 200, 2)])
def test_mul_mat_id_vs_oracle(t, shape):
    """Reference Test 5 shapes (tests/native/tests_basic_cuda.cpp:301-322) as
    MUL_MAT_ID with 12 experts and 4 routes per token."""
    I, O_, S = shape
    E, n_ids = 12, 4
    rng = np.random.default_rng(I + O_)
    ids = np.stack([rng.permutation(E)[:n_ids] for _ in range(S)]).astype(np.int32)
    got, ref = _mmid_case(t, I, O_, E, ids, 1, seed=t * 7 + S)
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())
    # per-element relative error is the stronger statement for a single dot
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3 * np.abs(ref).max())
    assert rel.max() <= 1e-3


@pytest.mark.parametrize("t", TYPES)
def test_mul_mat_id_negative_and_broadcast(t):
    """ids {3,-1,17,-1,-1,8,-1,-1,-1,21} (bench/mmid_exact_check.cpp:41): -1 rows
    are zero; ne11 == n_ids takes one src1 row per slot."""
    ids = np.array([[3, -1, 17, -1, -1, 8, -1, -1, -1, 21]], np.int32)
    for ne11 in (1, 10):
        got, ref = _mmid_case(t, 2560 if t != IQ2 else 2560, 192, 24, ids, ne11, seed=5 + ne11)
        assert not got[0, 1].any() and not got[0, 3].any()
        np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())


def test_mul_mat_id_skewed_prefill_buckets():
    """Many tokens, skewed expert loads (bucket chunks of 4 pairs)."""
    rng = np.random.default_rng(3)
    S, n_ids, E = 96, 8, 16
    p = np.exp(rng.standard_normal(E) * 1.5)
    p /= p.sum()
    ids = np.stack([rng.choice(E, n_ids, replace=False, p=p) for _ in range(S)]).astype(np.int32)
    ids[5, 2] = -1
    got, ref = _mmid_case(Q4, 1024, 96, E, ids, 1, seed=9)
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())


@pytest.mark.parametrize("t", [Q4, Q2, Q5, Q6, IQ4, IQ2, IQ3])
@pytest.mark.parametrize("ne11", [1, 8])
def test_mul_mat_id_mfma_buckets_per_element(ne11, t):
    """Buckets of 64-80 pairs take the int8-MFMA path for Q4_K, Q2_K, Q5_K and Q6_K: every
    output element within 1e-3 relative of the oracle (the op alone, no
    re-quantization)."""
    rng = np.random.default_rng(11 + ne11)
    S, n_ids, E = 72, 8, 8
    ids = np.stack([rng.permutation(E)[:n_ids] for _ in range(S)]).astype(np.int32)
    got, ref = _mmid_case(t, 2048, 160, E, ids, ne11, seed=13 + ne11)
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-3 * np.abs(ref).max())
    assert rel.max() <= 1e-3, rel.max()


def test_iq4_xs_custom_table():
    """zm_set_iq4nl_table replaces the device table: the op then matches the
    oracle run with the same table (a permuted, rescaled one here)."""
    import zeromoe_amd as Z

    default = Z.builtin_iq4nl_table()
    np.testing.assert_array_equal(default, O.iq4nl_table())
    custom = (np.arange(16, dtype=np.int64)[::-1] * 15 - 110).astype(np.int8)
    lib_o = O.lib()
    try:
        Z.set_iq4nl_table(custom)
        lib_o.zmo_set_iq4nl_table(custom.ctypes.data)
        rng = np.random.default_rng(2)
        ids = np.stack([rng.permutation(6)[:4] for _ in range(3)]).astype(np.int32)
        got, ref = _mmid_case(IQ4, 1024, 40, 6, ids, 1, seed=4)
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    finally:
        Z.set_iq4nl_table(default)
        lib_o.zmo_set_iq4nl_table(default.ctypes.data)


def test_iq3_xxs_custom_grid():
    """zm_set_iq3xxs_grid replaces the device grid: the op then matches the
    oracle run with the same grid (the stand-in in reverse order here)."""
    import zeromoe_amd as Z

    default = Z.builtin_iq3xxs_grid()
    np.testing.assert_array_equal(default, O.iq3xxs_grid())
    custom = np.ascontiguousarray(default[::-1])
    lib_o = O.lib()
    try:
        Z.set_iq3xxs_grid(custom)
        lib_o.zmo_set_iq3xxs_grid(custom.ctypes.data)
        rng = np.random.default_rng(3)
        ids = np.stack([rng.permutation(6)[:4] for _ in range(3)]).astype(np.int32)
        got, ref = _mmid_case(IQ3, 1024, 40, 6, ids, 1, seed=5)
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    finally:
        Z.set_iq3xxs_grid(default)
        lib_o.zmo_set_iq3xxs_grid(default.ctypes.data)


def _hook_descs(W, t, I, x, ids, y):
    import ctypes as C

    from zeromoe_amd.ops import _tensor

    return [C.byref(d) for d in (_tensor(t, W, I), _tensor(0, x, None), _tensor(26, ids, None), _tensor(0, y, None))]


def test_mul_mat_id_workspace_binding_rules():
    """The hook allocates nothing: it declines (query and execute) without a
    workspace bound on the device/stream or with one too small, and runs once
    one is bound; the query uses the smallest workspace bound on the device."""
    from zeromoe_amd._lib import lib
    from zeromoe_amd.ops import _MMID_WS

    L = lib()
    for (dev, st), _ in list(_MMID_WS.items()):  # start from no bindings
        assert L.zm_mul_mat_id_set_workspace(st, None, 0) == 0
    _MMID_WS.clear()
    rng = np.random.default_rng(8)
    E, O_, I, S = 6, 64, 1024, 5
    W = torch.from_numpy(O.random_blocks(Q4, E * O_, I, seed=3).reshape(E, O_, -1)).cuda()
    x = torch.from_numpy(rng.standard_normal((S, 1, I)).astype(np.float32)).cuda()
    ids = torch.from_numpy(np.stack([rng.permutation(E)[:4] for _ in range(S)]).astype(np.int32)).cuda()
    y = torch.full((S, 4, O_), 7.0, device="cuda")
    d = _hook_descs(W, Q4, I, x, ids, y)
    need = L.zm_mul_mat_id_workspace_size(*d)
    assert need > 0
    st = torch.cuda.current_stream().cuda_stream
    assert L.zm_mul_mat_id(*d, None, 0) == 0  # nothing bound
    assert L.zm_mul_mat_id(*d, st, 1) == 0
    small = torch.empty(need - 256, dtype=torch.uint8, device="cuda")
    assert L.zm_mul_mat_id_set_workspace(st, small.data_ptr(), small.numel()) == 0
    assert L.zm_mul_mat_id(*d, None, 0) == 0 and L.zm_mul_mat_id(*d, st, 1) == 0
    _sync()
    assert (y == 7.0).all()  # a declined call launches nothing
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    assert L.zm_mul_mat_id_set_workspace(st, ws.data_ptr(), ws.numel()) == 0
    assert L.zm_mul_mat_id(*d, None, 0) == 1
    other = torch.cuda.Stream()
    assert L.zm_mul_mat_id(*d, other.cuda_stream, 1) == 0  # no workspace on that stream
    assert L.zm_mul_mat_id(*d, st, 1) == 1
    _sync()
    ref = O.mul_mat_id(Q4, W.cpu().numpy(), x.cpu().numpy(), ids.cpu().numpy(), nthreads=8)
    np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())
    # the query takes the smallest binding on the device
    assert L.zm_mul_mat_id_set_workspace(other.cuda_stream, small.data_ptr(), small.numel()) == 0
    assert L.zm_mul_mat_id(*d, None, 0) == 0
    assert L.zm_mul_mat_id_set_workspace(other.cuda_stream, None, 0) == 0
    assert L.zm_mul_mat_id_set_workspace(st, None, 0) == 0
    assert L.zm_mul_mat_id(*d, None, 0) == 0


@pytest.mark.parametrize("case", ["decode", "prefill_mfma", "strided_ids_ne11"])
def test_mul_mat_id_hook_graph_capture_replays_bit_exact(case):
    """The hook recorded into a HIP graph on a stream with a bound workspace,
    replayed several times with eager hook calls (other inputs, same
    workspace) in between: every replay gives the eager result bit for bit."""
    from zeromoe_amd._lib import lib

    L = lib()
    rng = np.random.default_rng(21)
    t, E, O_, I, S, n_ids, ne11 = {"decode": (Q2, 16, 512, 2048, 1, 8, 1),
                                   "prefill_mfma": (Q4, 8, 256, 1024, 64, 8, 1),
                                   "strided_ids_ne11": (Q3, 12, 192, 1536, 6, 4, 4)}[case]
    W = torch.from_numpy(O.random_blocks(t, E * O_, I, seed=5).reshape(E, O_, -1)).cuda()
    x = torch.from_numpy(rng.standard_normal((S, ne11, I)).astype(np.float32)).cuda()
    ids_np = np.stack([rng.permutation(E)[:n_ids] for _ in range(S)]).astype(np.int32)
    ids_np[0, 1] = -1
    if case == "strided_ids_ne11":  # ids with a row stride larger than n_ids
        big = torch.from_numpy(np.pad(ids_np, ((0, 0), (0, 3)))).cuda()
        ids = big[:, :n_ids]
    else:
        ids = torch.from_numpy(ids_np).cuda()
    y = torch.empty((S, n_ids, O_), device="cuda")
    d = _hook_descs(W, t, I, x, ids, y)
    s = torch.cuda.Stream()
    ws = torch.empty(L.zm_mul_mat_id_workspace_size(*d), dtype=torch.uint8, device="cuda")
    assert L.zm_mul_mat_id_set_workspace(s.cuda_stream, ws.data_ptr(), ws.numel()) == 0
    try:
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            assert L.zm_mul_mat_id(*d, s.cuda_stream, 1) == 1
        s.synchronize()
        eager = y.clone()
        ref = O.mul_mat_id(t, W.cpu().numpy(), x.cpu().numpy(), ids_np, nthreads=8)
        np.testing.assert_allclose(eager.cpu().numpy(), ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            assert L.zm_mul_mat_id(*d, s.cuda_stream, 1) == 1
        x2 = torch.randn_like(x)
        y2 = torch.empty_like(y)
        d2 = _hook_descs(W, t, I, x2, ids, y2)
        for rep in range(4):
            y.fill_(float(rep))
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(y.cpu().numpy(), eager.cpu().numpy())
            with torch.cuda.stream(s):  # eager use of the same workspace between replays
                assert L.zm_mul_mat_id(*d2, s.cuda_stream, 1) == 1
            s.synchronize()
    finally:
        L.zm_mul_mat_id_set_workspace(s.cuda_stream, None, 0)


def test_mul_mat_id_two_streams_concurrent():
    """Two streams with their own workspaces running the hook at the same
    time on different inputs: both results are right (no shared scratch)."""
    import zeromoe_amd as Z

    rng = np.random.default_rng(4)
    E, O_, I, S = 8, 384, 2048, 48
    W = O.random_blocks(Q4, E * O_, I, seed=9).reshape(E, O_, -1)
    Wd = torch.from_numpy(W).cuda()
    xs = [rng.standard_normal((S, 1, I)).astype(np.float32) for _ in range(2)]
    idss = [np.stack([rng.permutation(E)[:8] for _ in range(S)]).astype(np.int32) for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [None, None]
    for rep in range(3):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[i] = Z.mul_mat_id(Wd, Q4, I, torch.from_numpy(xs[i]).cuda(), torch.from_numpy(idss[i]).cuda(),
                                       stream=s)
        torch.cuda.synchronize()
        for i in range(2):
            ref = O.mul_mat_id(Q4, W, xs[i], idss[i], nthreads=8)
            np.testing.assert_allclose(outs[i].cpu().numpy(), ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())


def test_mul_mat_id_many_pairs_grid_stride():
    """More than 65535 (token, slot) pairs with negative and out-of-range ids:
    the skipped rows are strided over the launch grid (zero / NaN rows)."""
    import zeromoe_amd as Z

    rng = np.random.default_rng(6)
    E, O_, I, S, n_ids = 4, 16, 256, 9000, 8
    ids = rng.integers(-1, E, (S, n_ids)).astype(np.int32)
    ids[-1, -1] = E + 3
    W = O.random_blocks(Q4, E * O_, I, seed=2).reshape(E, O_, -1)
    x = rng.standard_normal((S, 1, I)).astype(np.float32)
    got = Z.mul_mat_id(torch.from_numpy(W).cuda(), Q4, I, torch.from_numpy(x).cuda(),
                       torch.from_numpy(ids).cuda()).cpu().numpy()
    assert np.isnan(got[-1, -1]).all()
    neg = ids < 0
    assert neg[S // 2:].any() and not got[neg].any()
    ok = (ids >= 0) & (ids < E)
    ref = O.mul_mat_id(Q4, W, x, np.where(ok, ids, -1).astype(np.int32), nthreads=8)
    np.testing.assert_allclose(got[ok], ref[ok], rtol=1e-3, atol=1e-3 * np.abs(ref).max())


def test_mul_mat_id_out_of_range_is_nan():
    ids = np.array([[2, 99]], np.int32)
    got, _ = _mmid_case(Q2, 512, 8, 4, np.array([[2, 1]], np.int32), 1, seed=1)
    import zeromoe_amd as Z

    W = O.random_blocks(Q2, 4 * 8, 512, seed=1).reshape(4, 8, -1)
    x = np.ones((1, 1, 512), np.float32)
    y = Z.mul_mat_id(torch.from_numpy(W).cuda(), Q2, 512, torch.from_numpy(x).cuda(),
                     torch.from_numpy(ids).cuda()).cpu().numpy()
    assert np.isnan(y[0, 1]).all() and np.isfinite(y[0, 0]).all()


# ------------------------------------------------------------------ router / bucketing

@pytest.mark.parametrize("name", ["c1", "c3", "c4", "c5"])
def test_router_ids_bit_exact(name):
    import zeromoe_amd as Z

    c = CONFIGS[name]
    b = Built(reduced(c, H=256, F=256, S=max(c.S, 64)), seed=11)
    lg = b.logits
    ids_r, w_r = O.router(lg, c.K, c.gating, b.logit_bias, None, c.groups, c.groups_used, c.norm, c.scale)
    t = lambda a: None if a is None else torch.from_numpy(a).cuda()
    ids, w = Z.router(t(lg), c.K, {0: "softmax", 1: "sigmoid"}[c.gating], logit_bias=t(b.logit_bias),
                      n_groups=c.groups, n_groups_used=c.groups_used, weights_norm=c.norm, weights_scale=c.scale)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_r)
    np.testing.assert_allclose(w.cpu().numpy(), w_r, rtol=1e-6, atol=0)
    if b.route_map is not None:
        ids2, w2 = Z.router(t(lg), c.K, "sigmoid", n_groups=c.groups, n_groups_used=c.groups_used,
                            weights_norm=c.norm, weights_scale=c.scale, route_map=t(b.route_map))
        i_r2, w_r2 = O.apply_slot_table(b.route_map, ids_r, w_r)
        np.testing.assert_array_equal(ids2.cpu().numpy(), i_r2)
        np.testing.assert_allclose(w2.cpu().numpy(), w_r2, rtol=1e-6, atol=0)


@pytest.mark.parametrize("gating", [0, 1])
def test_router_sel_bias_and_route_mask(gating):
    """Selection bias (added for selection only; the weights gather the
    unbiased probabilities, moe_routed_ggml.hpp:77-141) and a non-binary
    route_mask with the slot table (w' = w * mask[id], ids' = route_map[id],
    moe_partial_route_ggml.hpp:21-35): ids bit-exact, weights to 1e-6."""
    import zeromoe_amd as Z

    rng = np.random.default_rng(17 + gating)
    S, E, K = 96, 256, 8
    lg = rng.standard_normal((S, E)).astype(np.float32)
    sb = (rng.standard_normal(E) * (0.3 if gating else 0.05)).astype(np.float32)
    lb = (rng.standard_normal(E) * 0.5).astype(np.float32)
    groups = (8, 4) if gating else (0, 0)
    ids_r, w_r = O.router(lg, K, gating, lb, sb, groups[0], groups[1], True, 2.5)
    # biased selection must differ from the unbiased one somewhere, or the test pins nothing
    ids_u, _ = O.router(lg, K, gating, lb, None, groups[0], groups[1], True, 2.5)
    assert not np.array_equal(ids_u, ids_r)
    perm = rng.permutation(E)
    rmap = np.full(E, -1, np.int32)
    rmap[perm[:96]] = np.arange(96, dtype=np.int32)
    mask = rng.uniform(0.25, 1.25, E).astype(np.float32)
    mask[::7] = 0.0
    t = lambda a: torch.from_numpy(a).cuda()
    g = {0: "softmax", 1: "sigmoid"}[gating]
    ids, w = Z.router(t(lg), K, g, logit_bias=t(lb), sel_bias=t(sb), n_groups=groups[0], n_groups_used=groups[1],
                      weights_norm=True, weights_scale=2.5)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_r)
    np.testing.assert_allclose(w.cpu().numpy(), w_r, rtol=1e-6, atol=0)
    ids2, w2 = Z.router(t(lg), K, g, logit_bias=t(lb), sel_bias=t(sb), n_groups=groups[0],
                        n_groups_used=groups[1], weights_norm=True, weights_scale=2.5, route_map=t(rmap),
                        route_mask=t(mask))
    i_r2, w_r2 = O.apply_slot_table(rmap, ids_r, w_r, mask)
    np.testing.assert_array_equal(ids2.cpu().numpy(), i_r2)
    np.testing.assert_allclose(w2.cpu().numpy(), w_r2, rtol=1e-6, atol=0)
    assert (i_r2 < 0).any() and ((w_r2 == 0) & (i_r2 >= 0)).any()


def test_router_ties_lowest_index():
    import zeromoe_amd as Z

    lg = np.round(np.random.default_rng(1).standard_normal((64, 128)) * 1.5).astype(np.float32)
    ids, _ = Z.router(torch.from_numpy(lg).cuda(), 8)
    ref, _ = O.router(lg, 8)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref)


@pytest.mark.parametrize("E,K,gating,groups", [
    (32, 4, 0, (0, 0)), (64, 8, 0, (0, 0)), (128, 1, 0, (0, 0)), (128, 8, 0, (0, 0)), (128, 12, 1, (0, 0)),
    (160, 8, 0, (0, 0)), (256, 8, 1, (8, 4)), (256, 16, 0, (0, 0)), (256, 20, 0, (0, 0)), (512, 8, 1, (0, 0)),
    (1000, 6, 0, (0, 0)),
])
@pytest.mark.parametrize("ties", [False, True])
def test_router_selection_paths(E, K, gating, groups, ties):
    """Top-k selection: the candidate-ranking path (K <= 16, at most 64
    experts at or above the subset-maxima bound) and the K-round path it falls
    back to (K > 16, heavy ties, E < 64 subsets) give the oracle's ids and
    weights.  Rounded logits make exact score ties common."""
    import zeromoe_amd as Z

    rng = np.random.default_rng(E * 31 + K)
    lg = rng.standard_normal((96, E)) * 2.0
    if ties:
        lg = np.round(lg)
    lg = lg.astype(np.float32)
    ids_r, w_r = O.router(lg, K, gating, None, None, groups[0], groups[1], True, 0.0)
    ids, w = Z.router(torch.from_numpy(lg).cuda(), K, {0: "softmax", 1: "sigmoid"}[gating], n_groups=groups[0],
                      n_groups_used=groups[1], weights_norm=True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_r)
    np.testing.assert_allclose(w.cpu().numpy(), w_r, rtol=1e-6, atol=0)


@pytest.mark.parametrize("S,K,E", [(1, 8, 128), (512, 8, 128), (4, 8, 160), (64, 8, 96), (3000, 8, 256)])
def test_bucket_bit_exact(S, K, E):
    import zeromoe_amd as Z

    rng = np.random.default_rng(S + E)
    p = np.exp(rng.standard_normal(E) * 1.5)
    p /= p.sum()
    ids = np.stack([rng.choice(E, K, replace=False, p=p) for _ in range(S)]).astype(np.int32)
    ids[rng.random(ids.shape) < 0.05] = -1
    counts, offs, pairs, active, n_active = Z.bucket(torch.from_numpy(ids).cuda(), E)
    rc, ro, rp = O.bucket(ids, E)
    np.testing.assert_array_equal(counts.cpu().numpy(), rc)
    np.testing.assert_array_equal(offs.cpu().numpy(), ro)
    np.testing.assert_array_equal(pairs.cpu().numpy()[: len(rp)], rp)
    act = np.nonzero(rc)[0]
    assert int(n_active.item()) == len(act)
    np.testing.assert_array_equal(active.cpu().numpy()[: len(act)], act)


# ------------------------------------------------------------------ the routed layer

LAYER_CASES = {
    "c1_full": (CONFIGS["c1"], {}),
    "c2_full": (CONFIGS["c2"], {}),
    "c3_reduced": (CONFIGS["c3"], dict(S=64, H=1024, F=512)),
    "c4_full": (CONFIGS["c4"], {}),
    "c5_full_S1": (CONFIGS["c5"], {}),
    "c5_S64_reduced": (CONFIGS["c5"], dict(S=64, H=1024, F=512, F_shared=512)),
    "c5_S64_full": (CONFIGS["c5"], dict(S=64)),
    # prefill buckets on the MFMA path: 128 pairs per expert on average (two passes of 64)
    "c3_mmq": (CONFIGS["c3"], dict(S=256, H=1024, F=512, E=16)),
    # mixed per-layer types of real checkpoints: Q4_K gate/up with a Q6_K down
    # projection (decode and a small prefill), Q5_K gate/up with Q6_K down
    "q4k_q6k_S1": (CONFIGS["c2"], dict(tg=Q4, td=Q6)),
    "q4k_q6k_S16": (CONFIGS["c2"], dict(tg=Q4, td=Q6, S=16, H=2048, F=768)),
    "q5k_q6k_S1": (CONFIGS["c2"], dict(tg=Q5, td=Q6)),
    # both projections on the MFMA path: mixed types with one tiling (64-pair
    # runs), and with different tilings, so gate/up and down run from separate
    # work-item lists (Q2_K takes 32-pair runs)
    "q4k_q6k_mmq": (CONFIGS["c3"], dict(tg=Q4, td=Q6, S=256, H=1024, F=512, E=16)),
    "q4k_q5k_mmq": (CONFIGS["c3"], dict(tg=Q4, td=Q5, S=256, H=1024, F=512, E=16)),
    "q5k_q2k_mmq": (CONFIGS["c3"], dict(tg=Q5, td=Q2, S=256, H=1024, F=512, E=16)),
    "q2k_q6k_mmq": (CONFIGS["c3"], dict(tg=Q2, td=Q6, S=256, H=1024, F=512, E=16)),
    "iq2xxs_mmq": (CONFIGS["c3"], dict(tg=IQ2, td=IQ2, S=256, H=1024, F=512, E=16)),
    # odd K-block counts (H = 5, F = 3 super-blocks) through the two-way unrolled K loop
    "q4k_mmq_odd_nb": (CONFIGS["c3"], dict(S=256, H=1280, F=768, E=16)),
    "iq3xxs_q6k_mmq_odd_nb": (CONFIGS["c3"], dict(tg=IQ3, td=Q6, S=256, H=1280, F=768, E=16)),
    "iq3xxs_iq4xs_mmq": (CONFIGS["c3"], dict(tg=IQ3, td=IQ4, S=256, H=1024, F=512, E=16)),
    "q5k_q5k_S64": (CONFIGS["c3"], dict(tg=Q5, td=Q5, S=64, H=1024, F=512)),
    "q4k_iq4xs_S1": (CONFIGS["c2"], dict(tg=Q4, td=IQ4)),
    "iq4xs_S16": (CONFIGS["c2"], dict(tg=IQ4, td=IQ4, S=16, H=2048, F=768)),
    "iq3xxs_S1": (CONFIGS["c2"], dict(tg=IQ3, td=IQ3)),
    "iq3xxs_S16": (CONFIGS["c2"], dict(tg=IQ3, td=IQ3, S=16, H=2048, F=768)),
    "q4k_q5k_shared_q6k": (CONFIGS["c5"], dict(tg=Q4, td=Q5, t_shared=Q6, H=2048, F=512, F_shared=1024)),
    # selection-only bias and a non-binary slot-table mask (fused decode at S=1,
    # the multi-kernel path at S=64), and a selection bias on softmax gating
    "c5_selbias_mask_S1": (CONFIGS["c5"], dict(sel_bias_sd=0.3, route_mask=True)),
    "c5_selbias_mask_S64": (CONFIGS["c5"], dict(S=64, H=2048, F=1024, F_shared=1024, sel_bias_sd=0.3,
                                                route_mask=True)),
    "c2_selbias_S4": (CONFIGS["c2"], dict(S=4, sel_bias_sd=0.05)),
}


@pytest.mark.parametrize("case", list(LAYER_CASES))
def test_moe_layer_vs_oracle(case):
    c, kw = LAYER_CASES[case]
    c = reduced(c, **kw)
    b = Built(c, seed=3)
    L = b.layer()
    x = torch.from_numpy(b.x).cuda()
    lg = None if c.router_gemv else torch.from_numpy(b.logits).cuda()
    out, ids, w = L.forward(x, lg)
    _sync()
    ids_r, w_r = b.oracle_route()
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_r)
    np.testing.assert_allclose(w.cpu().numpy(), w_r, rtol=1e-5, atol=1e-7)
    ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
    ref = b.oracle_forward(ids_h, w_h)
    assert_close_layer(out.cpu().numpy(), ref, slack=lambda: b.requant_slack(ids_h, w_h), label=f"layer {case}")


def test_moe_layer_repeatable_and_stream_ordered():
    """Same inputs, two streams, many calls: identical bits (no atomics, no races)."""
    c = reduced(CONFIGS["c2"], H=2048, F=768)
    b = Built(c, seed=4)
    L = b.layer()
    x = torch.from_numpy(b.x).cuda()
    lg = torch.from_numpy(b.logits).cuda()
    first, _, _ = L.forward(x, lg)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for _ in range(5):
            o2, _, _ = L.forward(x, lg)
    s.synchronize()
    np.testing.assert_array_equal(first.cpu().numpy(), o2.cpu().numpy())


# ------------------------------------------------------------------ fused decode kernel vs multi-kernel path

FUSED_CASES = {
    "c1": (CONFIGS["c1"], {}),
    "c2": (CONFIGS["c2"], {}),
    "c2_S8": (CONFIGS["c2"], dict(S=8)),
    "c2_S3": (CONFIGS["c2"], dict(S=3)),  # x quantized by 5 workers, first groups requested before routing
    "c4": (CONFIGS["c4"], {}),
    "c5": (CONFIGS["c5"], {}),
    "c5_S2": (CONFIGS["c5"], dict(S=2)),
    "q4k_q6k": (CONFIGS["c2"], dict(tg=Q4, td=Q6)),
    "q4k_q6k_S4": (CONFIGS["c2"], dict(tg=Q4, td=Q6, S=4)),
    "q5k_q6k": (CONFIGS["c2"], dict(tg=Q5, td=Q6)),
    "iq4xs": (CONFIGS["c2"], dict(tg=IQ4, td=IQ4)),
    "iq4xs_S3": (CONFIGS["c2"], dict(tg=IQ4, td=IQ4, S=3)),
    "iq3xxs": (CONFIGS["c2"], dict(tg=IQ3, td=IQ3)),
    "iq2xxs_S2": (CONFIGS["c2"], dict(tg=IQ2, td=IQ2, S=2)),  # 16 lanes per gate/up row, half-block down units
    "c5_selbias_mask": (CONFIGS["c5"], dict(sel_bias_sd=0.3, route_mask=True)),
    "c5_S3_selbias_mask": (CONFIGS["c5"], dict(S=3, sel_bias_sd=0.3, route_mask=True)),
}


@pytest.mark.parametrize("case", list(FUSED_CASES))
def test_fused_decode_vs_multikernel_and_oracle(case, monkeypatch):
    """The single persistent decode kernel against the multi-kernel path
    (same arithmetic, different reduction order) and the oracle; 20 launches
    back to back must give identical bits (sync words reset every launch)."""
    c, kw = FUSED_CASES[case]
    c = reduced(c, **kw)
    b = Built(c, seed=21)
    L = b.layer()
    x = torch.from_numpy(b.x).cuda()
    lg = None if c.router_gemv else torch.from_numpy(b.logits).cuda()
    monkeypatch.setenv("ZEROMOE_FUSED_DECODE", "1")
    out1, ids1, w1 = L.forward(x, lg)
    first = out1.clone()
    for _ in range(20):
        out1, ids1, w1 = L.forward(x, lg)
    assert L.status(c.S) == 0
    np.testing.assert_array_equal(first.cpu().numpy(), out1.cpu().numpy())
    monkeypatch.setenv("ZEROMOE_FUSED_DECODE", "0")
    out2, ids2, w2 = L.forward(x, lg)
    _sync()
    np.testing.assert_array_equal(ids1.cpu().numpy(), ids2.cpu().numpy())
    np.testing.assert_array_equal(w1.cpu().numpy(), w2.cpu().numpy())
    assert_close_layer(out1.cpu().numpy(), out2.cpu().numpy(), rtol=1e-4)
    ref = b.oracle_forward(ids1.cpu().numpy(), w1.cpu().numpy())
    assert_close_layer(out1.cpu().numpy(), ref)


@pytest.mark.parametrize("case", ["c5_S2", "c2_S8"])
def test_fused_decode_varying_routes(case, monkeypatch):
    """Consecutive fused launches whose routing differs (with c5's slot table a
    different number of routes is resident each time, so the act rows stored
    per call change): every launch matches the oracle.  The two act buffers
    alternate between calls and each call clears the rows the other one holds,
    so no row of an earlier call can be read as stored."""
    c, kw = FUSED_CASES[case]
    c = reduced(c, **kw)
    b = Built(c, seed=23)
    L = b.layer()
    rng = np.random.default_rng(5)
    monkeypatch.setenv("ZEROMOE_FUSED_DECODE", "1")
    n_routes = set()
    for i in range(10):
        b.x = (rng.standard_normal(b.x.shape) * (0.5 + i % 3)).astype(np.float32)
        x = torch.from_numpy(b.x).cuda()
        lg_np = None if c.router_gemv else (rng.standard_normal(b.logits.shape) * (0.5 + i % 3)).astype(np.float32)
        out, ids, w = L.forward(x, None if lg_np is None else torch.from_numpy(lg_np).cuda())
        _sync()
        ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
        ids_r, _ = b.oracle_route(lg_np)
        np.testing.assert_array_equal(ids_h, ids_r)
        n_routes.add(int((ids_h >= 0).sum()))
        ref = b.oracle_forward(ids_h, w_h)
        assert_close_layer(out.cpu().numpy(), ref, slack=lambda: b.requant_slack(ids_h, w_h))
    assert L.status(c.S) == 0
    if b.route_map is not None:
        assert len(n_routes) > 1, n_routes


def test_fused_decode_expired_wait_is_loud_and_recovers(monkeypatch):
    """The fused kernel's bounded waits forced to give up from the host (a
    negative spin limit: every act-block wait expires on its first poll): the
    launch still completes and its rows are NaN, never stale; the next launch,
    which finds the error word set, writes NaN everywhere instead of trusting
    the counters; zm_moe_status reports the error and resets the sync words,
    and the launch after that matches the oracle again."""
    c = CONFIGS["c2"]
    b = Built(c, seed=61)
    L = b.layer()
    x = torch.from_numpy(b.x).cuda()
    lg = torch.from_numpy(b.logits).cuda()
    monkeypatch.setenv("ZEROMOE_FUSED_DECODE", "1")
    monkeypatch.setenv("ZEROMOE_SPIN_LIMIT", "-1")
    out1, ids, w = L.forward(x, lg)
    out1 = out1.clone()
    monkeypatch.delenv("ZEROMOE_SPIN_LIMIT")
    out2, _, _ = L.forward(x, lg)
    _sync()
    err = L.status(c.S)
    assert err != 0, "the forced give-up did not set the error word"
    assert np.isnan(out1.cpu().numpy()).all()  # every workgroup waited for act blocks
    assert np.isnan(out2.cpu().numpy()).all()  # stale counters are never trusted
    ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
    ref = b.oracle_forward(ids_h, w_h)
    assert L.status(c.S) == 0
    out3, _, _ = L.forward(x, lg)
    _sync()
    assert L.status(c.S) == 0
    assert_close_layer(out3.cpu().numpy(), ref)


@pytest.mark.parametrize("case", ["c2", "c3_small", "c5_S64_small"])
def test_hip_graph_replay_matches_eager(case):
    """The layer recorded into a HIP graph and replayed several times, with eager
    work in between, gives the eager result bit for bit on every replay.  c5 at
    S=64 runs its dense shared expert on the library's side stream (forked
    after x is quantized, joined before the combine): the fork and join are
    recorded into the graph too."""
    c = {"c2": CONFIGS["c2"], "c3_small": reduced(CONFIGS["c3"], S=32, H=1024, F=512),
         "c5_S64_small": reduced(CONFIGS["c5"], S=64, H=2048, F=1024, F_shared=1024)}[case]
    b = Built(c, seed=31)
    L = b.layer()
    x = torch.from_numpy(b.x).cuda()
    lg = None if c.router_gemv else torch.from_numpy(b.logits).cuda()
    out = torch.empty((c.S, c.H), device="cuda")
    ids = torch.empty((c.S, c.K), dtype=torch.int32, device="cuda")
    w = torch.empty((c.S, c.K), device="cuda")
    L.forward(x, lg, out=out, ids=ids, weights=w)
    _sync()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        L.forward(x, lg, out=out, ids=ids, weights=w)
    for rep in range(4):
        out.zero_()
        g.replay()
        _sync()
        np.testing.assert_array_equal(out.cpu().numpy(), eager.cpu().numpy())
        L.forward(x, lg)  # eager work between replays (own outputs)
        _sync()


PREFILL_CASES = {
    "c3_mmq": (CONFIGS["c3"], dict(S=256, H=1024, F=512, E=16)),
    "c3_skewed": (CONFIGS["c3"], dict(S=192, H=2048, F=768, E=64)),
    # Q2_K routed experts (few pairs each) + Q4_K shared expert, slot table
    "c5_S64": (CONFIGS["c5"], dict(S=64, H=2048, F=1024, F_shared=1024)),
    # mixed-type layers: Q4_K gate/up with a Q6_K down projection; all Q6_K
    "q4k_q6k_mmq": (CONFIGS["c3"], dict(td=Q6, S=256, H=1024, F=512, E=16)),
    "q6k_q6k_mmq": (CONFIGS["c3"], dict(tg=Q6, td=Q6, S=128, H=1024, F=768, E=16)),
    "q5k_q6k_mmq": (CONFIGS["c3"], dict(tg=Q5, td=Q6, S=256, H=1024, F=512, E=16)),
    "iq4xs_mmq": (CONFIGS["c3"], dict(tg=IQ4, td=IQ4, S=256, H=1024, F=512, E=16)),
    "iq2xxs_mmq": (CONFIGS["c3"], dict(tg=IQ2, td=IQ2, S=256, H=1024, F=512, E=16)),
    # odd K-block counts (H = 5, F = 3 super-blocks) through the two-way unrolled K loop
    "q4k_mmq_odd_nb": (CONFIGS["c3"], dict(S=256, H=1280, F=768, E=16)),
    "iq3xxs_q6k_mmq_odd_nb": (CONFIGS["c3"], dict(tg=IQ3, td=Q6, S=256, H=1280, F=768, E=16)),
    "iq3xxs_mmq": (CONFIGS["c3"], dict(tg=IQ3, td=IQ3, S=256, H=1024, F=512, E=16)),
}


@pytest.mark.parametrize("case", list(PREFILL_CASES))
def test_prefill_mfma_vs_gemv(case, monkeypatch):
    """The int8-MFMA bucketed GEMM (prefill) against the GEMV path on the same
    buckets (same integer sums, different float order) and the oracle."""
    c, kw = PREFILL_CASES[case]
    c = reduced(c, **kw)
    b = Built(c, seed=41)
    L = b.layer()
    x = torch.from_numpy(b.x).cuda()
    lg = None if c.router_gemv else torch.from_numpy(b.logits).cuda()
    monkeypatch.setenv("ZEROMOE_MMQ", "1")
    out1, ids1, w1 = L.forward(x, lg)
    _sync()
    monkeypatch.setenv("ZEROMOE_MMQ", "0")
    out2, ids2, w2 = L.forward(x, lg)
    _sync()
    np.testing.assert_array_equal(ids1.cpu().numpy(), ids2.cpu().numpy())
    ids_h, w_h = ids1.cpu().numpy(), w1.cpu().numpy()
    slack = lambda: b.requant_slack(ids_h, w_h)
    ref = b.oracle_forward(ids_h, w_h)
    assert_close_layer(out1.cpu().numpy(), ref, slack=slack)
    assert_close_layer(out2.cpu().numpy(), ref, slack=slack)
    # two device paths may each flip a different tied element: twice the bound.
    # With a shared expert its act re-quantization can flip as well (not in the
    # slack bound): the layer bar then applies between the paths too.
    rtol = 1e-3 if c.F_shared else 1e-4
    assert_close_layer(out1.cpu().numpy(), out2.cpu().numpy(), rtol=rtol, slack=lambda: 2 * slack())


def test_c3_full_size_vs_oracle():
    """Config c3 at its stated size: H=4096, F=1536, 128 Q4_K experts, top-8
    softmax, S=512, per-expert logit bias N(0,1.5) (0 to ~150 pairs per
    expert, the heaviest buckets cut into several MFMA work items).  Router
    ids bit-exact, weights to 1e-5, bucket arrays bit-exact, and the whole
    layer against the oracle on every token within the layer bar."""
    import zeromoe_amd as Z

    c = CONFIGS["c3"]
    b = Built(c, seed=51)
    L = b.layer()
    x = torch.from_numpy(b.x).cuda()
    out, ids, w = L.forward(x, torch.from_numpy(b.logits).cuda())
    _sync()
    ids_r, w_r = b.oracle_route()
    ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
    np.testing.assert_array_equal(ids_h, ids_r)
    np.testing.assert_allclose(w_h, w_r, rtol=1e-5, atol=1e-7)
    counts, offs, pairs, active, n_active = Z.bucket(ids, c.E)
    rc, ro, rp = O.bucket(ids_r, c.E)
    np.testing.assert_array_equal(counts.cpu().numpy(), rc)
    np.testing.assert_array_equal(offs.cpu().numpy(), ro)
    np.testing.assert_array_equal(pairs.cpu().numpy()[: len(rp)], rp)
    assert rc.max() >= 100, rc.max()  # skewed: several work items for the heaviest experts
    ref = b.oracle_forward(ids_h, w_h, nthreads=16)
    assert_close_layer(out.cpu().numpy(), ref, slack=lambda: b.requant_slack(ids_h, w_h), label="c3 full size")


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_layer_with_ggml_quantized_weights(name):
    """The configurations state weights quantized from seeded N(0, 0.02) by
    ggml's quantizers: every expert the batch routes to (and c5's shared
    expert) is filled that way here -- the oracle's restated quantizers on a
    portable splitmix64 + Box-Muller generator (seed 1000 * expert + matrix,
    the reference seeds its weights per tensor, tests/test_option_b_compact_ggml.cpp:90)
    instead of random valid blocks.  c1/c2/c4/c5 decode through the fused
    kernel, c3 (S=512) through the MFMA prefill; ids bit-exact and the layer
    against the oracle.  IQ2_XXS (c4) has no importance matrix argument in
    the restated quantizer, which is the uniform-importance case."""
    c = CONFIGS[name]
    b = Built(c, seed=71)
    ids_r, w_r = b.oracle_route()
    mats = lambda: [(b.wg, c.tg, c.F, c.H), (b.wu, c.tg, c.F, c.H), (b.wd, c.td, c.H, c.F)]
    used = sorted(set(int(v) for v in ids_r.reshape(-1) if v >= 0))
    print(f"{name}: quantizing {len(used)} experts", flush=True)
    for e in used:
        for k, (W, t, rows, n) in enumerate(mats()):
            x = O.fill_normal(1000 * e + k, rows * n, 0.0, 0.02).reshape(rows, n)
            W[e].copy_(torch.from_numpy(O.quantize(t, x)).cuda())
    if c.F_shared:
        for k, (W, rows, n) in enumerate([(b.sg, c.F_shared, c.H), (b.su, c.F_shared, c.H), (b.sd, c.H, c.F_shared)]):
            x = O.fill_normal(999_000 + k, rows * n, 0.0, 0.02).reshape(rows, n)
            W.copy_(torch.from_numpy(O.quantize(c.t_shared, x).reshape(W.shape)).cuda())
    L = b.layer()
    lg = None if c.router_gemv else torch.from_numpy(b.logits).cuda()
    out, ids, w = L.forward(torch.from_numpy(b.x).cuda(), lg)
    _sync()
    assert L.status(c.S) == 0
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_r)
    ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
    ref = b.oracle_forward(ids_h, w_h, nthreads=16)
    assert_close_layer(out.cpu().numpy(), ref, slack=lambda: b.requant_slack(ids_h, w_h),
                       label=f"{name} ggml-quantized weights")