"""The CPU lane of a hot/cold expert split (zm_cold_lane_*, the reference's
EarlyReadyLane, models/graph/early_ready_lane.hpp:75-211) against the oracle.

CPU tests: the lane's host computation equals the oracle's layer restricted
to the cold routes (ids' = cold_map[ids], w' = w * cold_mask[ids],
backends/ggml/moe_partial_route_ggml.hpp:21-35) bit for bit, with the AVX-512
and the scalar dots.  GPU test: fork -> hot layer on the GPU -> merge equals
the oracle's whole layer, and the lane's CPU work overlaps the GPU's."""
import threading
import time

import numpy as np
import pytest

import zm_oracle as O

Q2, Q3, Q4 = O.TYPE_Q2_K, O.TYPE_Q3_K, O.TYPE_Q4_K


def f32bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _split(E, n_cold, seed):
    """Cold experts in host slots (a permutation), the rest hot; masks with a
    zero and non-binary values."""
    rng = np.random.default_rng(seed)
    cold = rng.permutation(E)[:n_cold]
    cmap = np.full(E, -1, np.int32)
    cmap[cold] = np.arange(n_cold, dtype=np.int32)
    hmap = np.full(E, -1, np.int32)
    hot = np.setdiff1d(np.arange(E), cold)
    hmap[hot] = np.arange(len(hot), dtype=np.int32)
    cmask = np.where(cmap >= 0, rng.uniform(0.5, 1.5, E), 0.0).astype(np.float32)
    cmask[cold[0]] = 0.0
    hmask = (hmap >= 0).astype(np.float32)
    return cold, hot, cmap, cmask, hmap, hmask


def _cold_ref(x, ids, w, cmap, cmask, tg, td, Wg, Wu, Wd):
    ids_c = np.where(ids >= 0, cmap[np.maximum(ids, 0)], -1).astype(np.int32)
    w_c = (w * np.where(ids >= 0, cmask[np.maximum(ids, 0)], 0.0)).astype(np.float32)
    return O.moe_forward(x, ids_c, w_c, tg, tg, td, Wg, Wu, Wd, nthreads=4)


@pytest.mark.parametrize("types", [(Q2, Q3), (Q4, Q4), (Q2, Q2)])
@pytest.mark.parametrize("scalar", [False, True])
def test_cold_lane_host_bit_identical_to_oracle(types, scalar):
    import zeromoe_amd as Z

    tg, td = types
    H, F, E, K, S, n_cold = 1024, 512, 24, 8, 3, 9
    cold, _, cmap, cmask, _, _ = _split(E, n_cold, seed=5)
    Wg = O.random_blocks(tg, n_cold * F, H, seed=11).reshape(n_cold, F, -1)
    Wu = O.random_blocks(tg, n_cold * F, H, seed=12).reshape(n_cold, F, -1)
    Wd = O.random_blocks(td, n_cold * H, F, seed=13).reshape(n_cold, H, -1)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((S, H)).astype(np.float32)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(S)]).astype(np.int32)
    ids[1, 3] = -1
    ids[0, :3] = cold[:3]  # several cold routes, including the zero-mask one
    w = rng.uniform(0.05, 0.3, (S, K)).astype(np.float32)
    lane = Z.ColdLane(H, F, E, K, tg, tg, td, Wg, Wu, Wd, cmap, cmask, max_tokens=S, n_threads=4, scalar=scalar)
    if not scalar and not O.has_avx512():
        assert lane.stats()["vectorized"] == 0
    got = lane.compute_host(x, ids, w)
    ref = _cold_ref(x, ids, w, cmap, cmask, tg, td, Wg, Wu, Wd)
    np.testing.assert_array_equal(f32bits(got), f32bits(ref))
    # a token with no cold route gets zeros
    ids2 = np.array([[i for i in range(E) if cmap[i] < 0][:K]], np.int32)
    np.testing.assert_array_equal(lane.compute_host(x[:1], ids2, w[:1]), np.zeros((1, H), np.float32))
    lane.close()


def test_cold_lane_rejects_bad_descriptors():
    import zeromoe_amd as Z

    H, F = 512, 256
    W = O.random_blocks(O.TYPE_IQ2_XXS, 2 * F, H, seed=1).reshape(2, F, -1)
    with pytest.raises(RuntimeError, match="Q2_K, Q3_K and Q4_K"):
        Z.ColdLane(H, F, 4, 2, O.TYPE_IQ2_XXS, O.TYPE_IQ2_XXS, O.TYPE_IQ2_XXS, W, W, W, np.zeros(4, np.int32))
    Wq = O.random_blocks(Q4, 2 * F, H, seed=1).reshape(2, F, -1)
    with pytest.raises(RuntimeError, match="bad descriptor"):
        Z.ColdLane(H + 100, F, 4, 2, Q4, Q4, Q4, Wq, Wq, Wq, np.zeros(4, np.int32))


@pytest.mark.gpu
def test_cold_lane_fork_hot_merge_on_gpu():
    """c2-shaped layer (H=4096, F=1536, 128 experts, top-8, Q2_K/Q3_K) with 48
    experts cold in host memory and 80 hot in VRAM: router -> fork -> hot
    layer (zm_moe_forward with the hot slot table) -> merge.  The merged
    output is the hot output plus the lane's host result (bit for bit), the
    hot output matches the oracle's hot branch, and the lane finishes its CPU
    work while the GPU stream is still busy (it started on the fork event, not
    after the GPU work)."""
    import torch

    import zeromoe_amd as Z
    from moe_cases import assert_close_layer, dev_random_blocks

    Z.init()
    H, F, E, K, n_cold = 4096, 1536, 128, 8, 48
    cold, hot, cmap, cmask, hmap, hmask = _split(E, n_cold, seed=9)
    n_hot = len(hot)
    Wg_h = dev_random_blocks(Q2, n_hot * F, H, 21).view(n_hot, F, -1)
    Wu_h = dev_random_blocks(Q2, n_hot * F, H, 22).view(n_hot, F, -1)
    Wd_h = dev_random_blocks(Q3, n_hot * H, F, 23).view(n_hot, H, -1)
    Wg_c = O.random_blocks(Q2, n_cold * F, H, seed=31).reshape(n_cold, F, -1)
    Wu_c = O.random_blocks(Q2, n_cold * F, H, seed=32).reshape(n_cold, F, -1)
    Wd_c = O.random_blocks(Q3, n_cold * H, F, seed=33).reshape(n_cold, H, -1)
    rng = np.random.default_rng(3)
    for S in (1, 4):
        x_h = rng.standard_normal((S, H)).astype(np.float32)
        lg_h = rng.standard_normal((S, E)).astype(np.float32)
        lg_h[:, cold[1:4]] += 3.0  # make sure cold experts are routed
        x, lg = torch.from_numpy(x_h).cuda(), torch.from_numpy(lg_h).cuda()
        hot_layer = Z.MoELayer(H=H, F=F, n_experts=E, topk=K, type_gate=Q2, type_up=Q2, type_down=Q3, w_gate=Wg_h,
                               w_up=Wu_h, w_down=Wd_h, route_map=torch.from_numpy(hmap).cuda(),
                               route_mask=torch.from_numpy(hmask).cuda())
        lane = Z.ColdLane(H, F, E, K, Q2, Q2, Q3, Wg_c, Wu_c, Wd_c, cmap, cmask, max_tokens=S, n_threads=8)
        ids_g, w_g = Z.router(lg, K)  # router expert ids and weights (no slot table)
        out = torch.empty((S, H), device="cuda")
        lane.fork(x, ids_g, w_g)
        hot_layer.forward(x, lg, out=out)
        hot_only = out.clone()
        torch.cuda._sleep(100_000_000)  # keep the stream busy after the fork
        busy = torch.cuda.Event()
        busy.record()
        # host time at which the stream drained, seen by a poller started now
        drained = []

        def poll():
            while not busy.query():
                time.sleep(20e-6)
            drained.append(time.monotonic_ns())

        poller = threading.Thread(target=poll)
        poller.start()
        lane.merge(out)
        torch.cuda.synchronize()
        poller.join()
        assert hot_layer.status(S) == 0
        ids_h, w_h = ids_g.cpu().numpy(), w_g.cpu().numpy()
        assert (cmap[ids_h] >= 0).any() and (hmap[ids_h] >= 0).any()
        cold_h = lane.compute_host(x_h, ids_h, w_h)
        np.testing.assert_array_equal(f32bits(out.cpu().numpy()), f32bits(hot_only.cpu().numpy() + cold_h))
        # the hot branch against the oracle (hot experts only)
        ids_hot = np.where(hmap[ids_h] >= 0, hmap[ids_h], -1).astype(np.int32)
        w_hot = (w_h * hmask[ids_h]).astype(np.float32)
        used = sorted(set(int(v) for v in ids_hot.reshape(-1) if v >= 0))
        sel = torch.tensor(used, device="cuda")
        remap = {e: i for i, e in enumerate(used)}
        rid = np.array([[remap.get(int(v), -1) for v in row] for row in ids_hot], np.int32)
        ref_hot = O.moe_forward(x_h, rid, w_hot, Q2, Q2, Q3, Wg_h.index_select(0, sel).cpu().numpy(),
                                Wu_h.index_select(0, sel).cpu().numpy(), Wd_h.index_select(0, sel).cpu().numpy(),
                                nthreads=8)
        assert_close_layer(hot_only.cpu().numpy(), ref_hot)
        st = lane.stats()
        assert st["fork_ns"] <= st["compute_begin_ns"] <= st["compute_end_ns"] <= st["merge_ns"]
        # the lane starts on the fork's event, not after the GPU work: its CPU
        # work began while the stream was still busy (same monotonic clock)
        assert st["compute_begin_ns"] < drained[0], "the lane started only after the GPU stream drained"
        lane.close()
