"""FP32-activation path (per-type launchers, FP32 MUL_MAT_ID hook, SwiGLU,
scatter-accumulate, GLM5Next router top-k, per-expert executor) vs the numpy
restatements in oracle/zm_oracle.py (MI355X).

Float bars, written per test: matmul outputs within 2e-5 of sum_i |w x|
(the device sums in another order than float64), SwiGLU and scatter within
float rounding, router ids exact up to scores that tie within 2e-6."""
import ctypes as C

import numpy as np
import pytest
import torch

import zm_oracle as O
from moe_cases import IQ2, IQ3, IQ4, Q2, Q3, Q4, Q5, Q6

pytestmark = pytest.mark.gpu

TYPES = [Q2, Q3, Q4, Q5, Q6, IQ2, IQ3, IQ4]
NAMES = {Q2: "q2_K", Q3: "q3_K", Q4: "q4_K", Q5: "q5_K", Q6: "q6_K", IQ2: "iq2_xxs", IQ3: "iq3_xxs", IQ4: "iq4_xs"}
MM_TOL = 2e-5


@pytest.fixture(scope="module", autouse=True)
def _init():
    import zeromoe_amd as Z

    assert torch.cuda.is_available(), "GPU tests need a device"
    Z.init()
    yield


def _check_mm(got, W, t, x, tol=MM_TOL):
    ref = O.f32_matmul(t, W, x)
    bound = O.f32_matmul_absbound(t, W, x)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= tol * bound + 1e-30), float((err / (bound + 1e-30)).max())


# ------------------------------------------------------------------ per-type launchers

@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("S,I,Orows", [(1, 1280, 37), (3, 5120, 50), (9, 256, 17), (1, 4096, 64)])
def test_f32_matmul(t, S, I, Orows):
    import zeromoe_amd as Z

    print(f"f32_matmul t={t} S={S} I={I} O={Orows}", flush=True)
    W = O.random_blocks(t, Orows, I, seed=t * 7 + S)
    x = np.random.default_rng(S + I).standard_normal((S, I)).astype(np.float32)
    y = Z.f32_matmul(torch.from_numpy(W).cuda(), t, I, torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    _check_mm(y.cpu().numpy(), W, t, x)


@pytest.mark.parametrize("t", TYPES)
def test_reference_named_launchers(t):
    """launch_<type>_matmul (legacy default stream) and _stream (torch's stream)."""
    from zeromoe_amd._lib import lib

    S, I, Orows = 2, 768, 24
    W = O.random_blocks(t, Orows, I, seed=t)
    x = np.random.default_rng(t).standard_normal((S, I)).astype(np.float32)
    dW, dx = torch.from_numpy(W).cuda(), torch.from_numpy(x).cuda()
    y0 = torch.full((S, Orows), np.nan, device="cuda")
    y1 = torch.full((S, Orows), np.nan, device="cuda")
    torch.cuda.synchronize()
    getattr(lib(), f"launch_{NAMES[t]}_matmul")(y0.data_ptr(), dx.data_ptr(), dW.data_ptr(), S, I, Orows)
    torch.cuda.synchronize()
    getattr(lib(), f"launch_{NAMES[t]}_matmul_stream")(y1.data_ptr(), dx.data_ptr(), dW.data_ptr(), S, I, Orows,
                                                        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _check_mm(y0.cpu().numpy(), W, t, x)
    np.testing.assert_array_equal(y0.cpu().numpy(), y1.cpu().numpy())  # same kernel, same order


def test_launcher_rejects_bad_I():
    from zeromoe_amd._lib import lib

    y = torch.full((1, 4), 7.0, device="cuda")
    x = torch.zeros((1, 300), device="cuda")
    w = torch.zeros(4 * 84 * 2, dtype=torch.uint8, device="cuda")
    assert lib().zm_f32_matmul(Q2, y.data_ptr(), x.data_ptr(), w.data_ptr(), 1, 300, 4, None) != 0
    assert b"multiple of 256" in lib().zm_last_error()
    torch.cuda.synchronize()
    assert torch.all(y == 7.0)


def test_q5_K_matmul_grouped():
    """launch_q5_K_matmul_grouped: y[g] = x[g] . W_g^T with W_g at a padded
    group stride; a stride that is not a whole number of blocks is rejected."""
    from zeromoe_amd._lib import lib

    G, I, Orows = 3, 1024, 40
    row = (I // 256) * 176
    stride = Orows * row + 2 * 176
    W = O.random_blocks(Q5, G * (stride // row + 1), I, seed=9).reshape(-1)[:G * stride]
    x = np.random.default_rng(3).standard_normal((G, I)).astype(np.float32)
    y = torch.full((G, Orows), np.nan, device="cuda")
    dW, dx = torch.from_numpy(np.ascontiguousarray(W)).cuda(), torch.from_numpy(x).cuda()
    torch.cuda.synchronize()
    assert lib().launch_q5_K_matmul_grouped(y.data_ptr(), dx.data_ptr(), dW.data_ptr(), G, stride, I, Orows)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for g in range(G):
        Wg = W[g * stride:g * stride + Orows * row].reshape(Orows, row)
        _check_mm(got[g:g + 1], Wg, Q5, x[g:g + 1])
    assert not lib().launch_q5_K_matmul_grouped(y.data_ptr(), dx.data_ptr(), dW.data_ptr(), G, stride + 1, I, Orows)


# ------------------------------------------------------------------ FP32 MUL_MAT_ID hook

@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("ne11", [1, 4])
def test_mul_mat_id_f32(t, ne11):
    import zeromoe_amd as Z

    E, I, Orows, S, n_ids = 5, 512, 40, 3, 4
    W = O.random_blocks(t, E * Orows, I, seed=11 + t).reshape(E, Orows, -1)
    rng = np.random.default_rng(t + ne11)
    x = rng.standard_normal((S, ne11, I)).astype(np.float32)
    ids = np.array([[0, 4, -1, 2], [3, 3, 1, 5], [4, 0, 2, 1]], np.int32)  # -1: zero row, 5 >= E: NaN row
    y = Z.mul_mat_id_f32(torch.from_numpy(W).cuda(), t, I, torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    for s in range(S):
        for k in range(n_ids):
            e = ids[s, k]
            if e < 0:
                assert np.all(y[s, k] == 0.0)
            elif e >= E:
                assert np.all(np.isnan(y[s, k]))
            else:
                _check_mm(y[s, k][None], W[e], t, x[s, k % ne11][None])


@pytest.mark.parametrize("t", [Q2, Q4])
def test_mul_mat_id_f32_plain_and_grouped(t):
    import zeromoe_amd as Z
    from zeromoe_amd._lib import lib
    from zeromoe_amd.ops import _tensor

    I, Orows, S, G = 768, 33, 5, 3
    W = O.random_blocks(t, G * Orows, I, seed=3).reshape(G, Orows, -1)
    x = np.random.default_rng(1).standard_normal((G, S, I)).astype(np.float32)
    dW, dx = torch.from_numpy(W).cuda(), torch.from_numpy(x).cuda()
    # plain: W[0] (O, rb) times x[0] (S, I)
    y = torch.empty((S, Orows), device="cuda")
    tw, tx, ty = _tensor(t, dW[0], I), _tensor(0, dx[0], None), _tensor(0, y, None)
    assert lib().zm_mul_mat_id_f32(C.byref(tw), C.byref(tx), None, C.byref(ty), None, 0) == 1
    assert lib().zm_mul_mat_id_f32(C.byref(tw), C.byref(tx), None, C.byref(ty), None, 1) == 1
    torch.cuda.synchronize()
    _check_mm(y.cpu().numpy(), W[0], t, x[0])
    # grouped: y[g] = W[g] x[g]
    yg = torch.empty((G, S, Orows), device="cuda")
    tw, tx, ty = _tensor(t, dW, I), _tensor(0, dx, None), _tensor(0, yg, None)
    assert lib().zm_mul_mat_id_f32(C.byref(tw), C.byref(tx), None, C.byref(ty), None, 1) == 1
    torch.cuda.synchronize()
    for g in range(G):
        _check_mm(yg[g].cpu().numpy(), W[g], t, x[g])
    # declined shapes: ne0 not a multiple of 256, mismatched dst
    tw.ne[0] = 700
    assert lib().zm_mul_mat_id_f32(C.byref(tw), C.byref(tx), None, C.byref(ty), None, 0) == 0
    _ = Z


# ------------------------------------------------------------------ SwiGLU

@pytest.mark.parametrize("clamp,fused", [(0.0, False), (6.0, False), (6.0, True), (0.0, True)])
def test_expert_swiglu(clamp, fused):
    import zeromoe_amd as Z

    n = 3000
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = (rng.standard_normal(n) * 4).astype(np.float32)
    g[[7, 100]] = np.nan
    u[[8]] = np.nan
    g[[9, 2999]] = np.inf
    u[[10]] = -np.inf
    u[[100]] = np.inf  # NaN wins over Inf
    bad = torch.zeros(2, dtype=torch.int32, device="cuda")
    got = Z.swiglu(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(), clamp, fused, bad).cpu().numpy()
    got2 = Z.swiglu(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(), clamp, fused, bad).cpu().numpy()
    ref, cnt = O.expert_swiglu(g, u, clamp, fused)
    assert list(bad.cpu().numpy()) == [2 * cnt[0], 2 * cnt[1]] == [6, 6]  # counters accumulate
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    # same exp, same operation order: bit-exact
    np.testing.assert_array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    np.testing.assert_array_equal(got.view(np.uint32), got2.view(np.uint32))


# ------------------------------------------------------------------ scatter-accumulate

@pytest.mark.parametrize("weighted", [True, False])
@pytest.mark.parametrize("D", [33, 4096])
def test_scatter_accum(weighted, D):
    import zeromoe_amd as Z

    rng = np.random.default_rng(D)
    S, n = 10, 8
    src = rng.standard_normal((n, D)).astype(np.float32)
    tok = np.array([9, 0, 4, -3, 2, 10, 7, 1], np.int32)
    w = rng.random(n).astype(np.float32)
    dst = rng.standard_normal((S, D)).astype(np.float32)
    d_dst = torch.from_numpy(dst).cuda()
    Z.scatter_accum(torch.from_numpy(src).cuda(), torch.from_numpy(tok).cuda(), d_dst,
                    torch.from_numpy(w).cuda() if weighted else None)
    torch.cuda.synchronize()
    ref = O.scatter_accum(src, tok, dst, w if weighted else None)
    np.testing.assert_array_equal(d_dst.cpu().numpy(), ref)  # one fma per element: exact


# ------------------------------------------------------------------ GLM5Next router top-k

def _assert_ids_tie_aware(ids, ref_ids, score, tol=2e-6):
    for s in range(ids.shape[0]):
        if np.array_equal(ids[s], ref_ids[s]):
            continue
        a, b = score[s][ids[s]], score[s][ref_ids[s]]
        np.testing.assert_allclose(a, b, rtol=tol, atol=tol)


@pytest.mark.parametrize("gating,bias,norm,scale", [(O.GATING_SOFTMAX, False, False, 0.0),
                                                     (O.GATING_SOFTMAX, True, True, 0.0),
                                                     (O.GATING_SIGMOID, True, True, 2.5),
                                                     (O.GATING_SQRT_SOFTPLUS, False, True, 1.0)])
@pytest.mark.parametrize("E,K", [(128, 8), (256, 8), (160, 6), (700, 3)])
def test_glm5next_router_topk(gating, bias, norm, scale, E, K):
    import zeromoe_amd as Z

    S = 16
    rng = np.random.default_rng(E + K)
    lg = rng.standard_normal((S, E)).astype(np.float32)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32) if bias else None
    d_lg = torch.from_numpy(lg).cuda()
    ids, w = Z.glm5next_router_topk(d_lg, K, None if b is None else torch.from_numpy(b).cuda(), gating, norm, scale)
    torch.cuda.synchronize()
    row_ref, ids_ref, w_ref = O.glm5next_router_topk(lg, K, b, gating, norm, scale)
    ids, w, row = ids.cpu().numpy(), w.cpu().numpy(), d_lg.cpu().numpy()
    probs = O.glm5next_router_topk(lg, 0, None, gating)[0]  # the gated row alone
    score = probs + (b if b is not None else 0)
    _assert_ids_tie_aware(ids, ids_ref, score)
    same = np.all(ids == ids_ref, axis=1)
    np.testing.assert_allclose(w[same], w_ref[same], rtol=2e-6, atol=1e-7)
    neg = np.float32(-3.402823466e38)
    for s in np.nonzero(same)[0]:
        assert np.all(row[s, ids[s]] == neg)
    np.testing.assert_allclose(row[same], row_ref[same], rtol=2e-6, atol=1e-7)


def test_glm5next_router_topk_ties_and_nan():
    import zeromoe_amd as Z

    lg = np.zeros((2, 70), np.float32)
    lg[1, 0] = np.nan
    lg[1, 5] = 3.0
    ids, _ = Z.glm5next_router_topk(torch.from_numpy(lg).cuda(), 4, gating=O.GATING_SIGMOID)
    _, ref, _ = O.glm5next_router_topk(lg, 4, gating=O.GATING_SIGMOID)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref)
    assert list(ref[0]) == [0, 1, 2, 3] and list(ref[1][:2]) == [0, 5]


# ------------------------------------------------------------------ per-expert executor

@pytest.mark.parametrize("types", [(Q2, Q2, Q3), (Q4, Q4, Q4), (IQ2, IQ2, IQ2), (Q4, Q4, Q6), (Q5, Q5, Q6)])
@pytest.mark.parametrize("S", [1, 5])
def test_expert_executor(types, S):
    import zeromoe_amd as Z

    D, F = 1024, 512
    tg, tu, td = types
    Wg = O.random_blocks(tg, F, D, seed=1)
    Wu = O.random_blocks(tu, F, D, seed=2)
    Wd = O.random_blocks(td, D, F, seed=3)
    slab = np.concatenate([Wg.ravel(), Wu.ravel(), Wd.ravel()])
    up_off, down_off = Wg.size, Wg.size + Wu.size
    x = np.random.default_rng(S).standard_normal((S, D)).astype(np.float32)
    ex = Z.ExpertExecutor()
    try:
        out = ex.run(torch.from_numpy(slab).cuda(), up_off, down_off, types, x, D, F)
        assert list(ex.bad_counts()) == [0, 0]
        out2 = ex.run(torch.from_numpy(slab).cuda(), up_off, down_off, types, x, D, F)
    finally:
        ex.release()
    np.testing.assert_array_equal(out, out2)
    g = O.f32_matmul(tg, Wg, x).astype(np.float32)
    u = O.f32_matmul(tu, Wu, x).astype(np.float32)
    prod, _ = O.expert_swiglu(g, u)
    prod = prod.reshape(S, F)
    # gate/up differ from the oracle's by float rounding (<= 2e-5 of their
    # |w x| bound); propagated through silu' <= 1.1 and the down matmul
    gb = O.f32_matmul_absbound(tg, Wg, x)
    ub = O.f32_matmul_absbound(tu, Wu, x)
    dprod = 1.1 * MM_TOL * (gb * np.abs(u) + np.abs(g) * ub) + 1e-30
    ref = O.f32_matmul(td, Wd, prod)
    Wdd = O.dequantize(td, Wd, F).astype(np.float64)
    bound = O.f32_matmul_absbound(td, Wd, prod) * MM_TOL + dprod @ np.abs(Wdd).T
    assert np.all(np.abs(out - ref) <= bound * 1.5), float(np.max(np.abs(out - ref) / bound))
