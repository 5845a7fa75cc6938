"""zm_mul_mat_id_static (scratch in a device array compiled into the library,
no allocation, no bound workspace) against zm_mul_mat_id on the same inputs:
identical bits, on two calls in a row (the second smaller, so stale contents
of the shared array from the first call would show), and a clear decline for
shapes beyond the array."""
import ctypes as C

import numpy as np
import pytest
import torch

import zm_oracle as O

pytestmark = pytest.mark.gpu


def _descs(W, t, I, x, ids, y):
    from zeromoe_amd.ops import _tensor

    return [C.byref(d) for d in (_tensor(t, W, I), _tensor(0, x, None), _tensor(26, ids, None), _tensor(0, y, None))]


def _case(t, E, O_, I, S, n_ids, ne11, seed):
    rng = np.random.default_rng(seed)
    W = torch.from_numpy(O.random_blocks(t, E * O_, I, seed=seed).reshape(E, O_, -1)).cuda()
    x = torch.from_numpy(rng.standard_normal((S, ne11, I)).astype(np.float32)).cuda()
    ids = np.stack([rng.permutation(E)[:n_ids] for _ in range(S)]).astype(np.int32)
    ids[0, 0] = -1
    return W, x, torch.from_numpy(ids).cuda()


def test_static_scratch_entry_matches_workspace_entry():
    import zeromoe_amd as Z
    from zeromoe_amd._lib import lib

    Z.init()
    L = lib()
    # first a prefill-sized call on the MFMA path, then a smaller decode call
    for t, E, O_, I, S, n_ids, ne11, seed in [(O.TYPE_Q4_K, 16, 512, 2048, 96, 8, 1, 1),
                                              (O.TYPE_Q2_K, 32, 256, 4096, 1, 8, 1, 2),
                                              (O.TYPE_Q3_K, 12, 192, 1536, 3, 4, 4, 3)]:
        W, x, ids = _case(t, E, O_, I, S, n_ids, ne11, seed)
        ref = Z.mul_mat_id(W, t, I, x, ids)  # workspace entry point (binds its own workspace)
        y = torch.full_like(ref, float("nan"))
        d = _descs(W, t, I, x, ids, y)
        assert L.zm_mul_mat_id_static(*d, None, 0) == 1
        assert L.zm_mul_mat_id_static(*d, torch.cuda.current_stream().cuda_stream, 1) == 1, \
            L.zm_last_error().decode()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), ref.cpu().numpy())
        assert not np.isnan(ref.cpu().numpy()).any()


def test_static_scratch_entry_declines_oversize_shapes():
    import zeromoe_amd as Z
    from zeromoe_amd._lib import lib

    Z.init()
    L = lib()
    t, E, O_, I, S, n_ids = O.TYPE_Q4_K, 8, 64, 16384, 1024, 8  # Q8_K rows alone: 1024 x 18.7 KB
    W = torch.zeros((E, O_, (I // 256) * 144), dtype=torch.uint8, device="cuda")
    x = torch.zeros((S, 1, I), device="cuda")
    ids = torch.zeros((S, n_ids), dtype=torch.int32, device="cuda")
    y = torch.zeros((S, n_ids, O_), device="cuda")
    d = _descs(W, t, I, x, ids, y)
    assert L.zm_mul_mat_id_workspace_size(*d) > 16 << 20
    assert L.zm_mul_mat_id_static(*d, None, 0) == 0
    assert L.zm_mul_mat_id_static(*d, torch.cuda.current_stream().cuda_stream, 1) == 0
    assert b"16777216-byte device array" in L.zm_last_error()
