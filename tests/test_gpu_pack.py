"""Expert-record unpack (launch_ggml_moe_unpack[_scatter]) vs the numpy
restatement in oracle/zm_oracle.py (MI355X).  Byte work: every destination
byte must equal the oracle's, including the bytes the call must not touch
(destinations start filled with a canary)."""
import numpy as np
import pytest
import torch

import zm_oracle as O

pytestmark = pytest.mark.gpu

CANARY = 0x5A


@pytest.fixture(scope="module", autouse=True)
def _init():
    import zeromoe_amd as Z

    assert torch.cuda.is_available(), "GPU tests need a device"
    Z.init()
    yield


def _run(parts, strides, n_dst, count, src_stride, slots=None, seed=0, src_offset=0, dst_offset=0):
    import zeromoe_amd as Z

    print(f"unpack parts={parts} strides={strides} count={count} stride={src_stride} slots={slots is not None} "
          f"src_off={src_offset} dst_off={dst_offset}", flush=True)
    rng = np.random.default_rng(seed)
    src = rng.integers(0, 256, src_offset + max(count - 1, 0) * src_stride + sum(parts), dtype=np.uint8)
    dst = [np.full(dst_offset + n_dst * s + 64, CANARY, np.uint8) for s in strides]
    d_src = torch.from_numpy(src).cuda()
    d_dst = [torch.from_numpy(a).cuda() for a in dst]
    d_slots = None if slots is None else torch.from_numpy(np.asarray(slots, np.int32)).cuda()
    Z.moe_unpack(d_src[src_offset:], *(t[dst_offset:] for t in d_dst), count, src_stride, parts, strides,
                 slots=d_slots)
    torch.cuda.synchronize()
    want = [a.copy() for a in dst]
    O.moe_unpack(src[src_offset:], *(w[dst_offset:] for w in want), count, src_stride, parts, strides,
                 None if slots is None else np.asarray(slots))
    for p in range(3):
        np.testing.assert_array_equal(d_dst[p].cpu().numpy(), want[p], err_msg=f"part {p}")


def _c2_parts():
    H, F = 4096, 1536
    g = F * (H // 256) * 84
    return (g, g, H * (F // 256) * 110)


def test_unpack_c2_records_dense():
    """8 c2 experts (Q2_K gate/up, Q3_K down): 16-byte aligned vector path."""
    p = _c2_parts()
    _run(p, p, 8, 8, sum(p))


def test_unpack_single_record_into_expert_slot():
    """The reference's per-expert call: count 1, destinations offset to the
    expert (ggml_moe_transfer_manager.cpp:725-731)."""
    p = _c2_parts()
    _run(p, p, 4, 1, sum(p), dst_offset=3 * p[0])  # gate stride == gate bytes; the offset lands on expert 3


def test_unpack_scatter_padded_records_with_skips():
    p = _c2_parts()
    rs = sum(p) + 4096
    slots = [5, -1, 0, 7, -1, 2]
    _run(p, p, 8, len(slots), rs, slots=slots, seed=1)


@pytest.mark.parametrize("parts,strides,rs,src_off", [
    ((3, 2, 5), (4, 3, 6), 12, 0),               # tiny, byte path
    ((1000, 17, 33333), (1008, 32, 33344), 34400, 0),  # odd sizes: byte path for up/down
    ((16384 + 48, 16, 40000), (16448, 16, 40000), 56448, 0),  # aligned, tails and partial chunks
    ((16400, 16400, 16400), (16400, 16400, 16400), 49200, 4),  # src 4 bytes off: every part byte-copied
    ((4096, 0, 4096), (4096, 0, 4096), 8192, 0),  # empty up part
])
def test_unpack_alignment_and_tails(parts, strides, rs, src_off):
    _run(parts, strides, 5, 5, rs, src_offset=src_off, seed=2)
    _run(parts, strides, 5, 3, rs, slots=[4, 1, -1], src_offset=src_off, seed=3)


def test_unpack_rejects_bad_arguments():
    """NULL pointers and count <= 0 return hipErrorInvalidValue (1) and launch
    nothing, as the reference (ggml_moe_pack.cu:141-142,165-166)."""
    from zeromoe_amd._lib import lib

    t = torch.zeros(64, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    L = lib()
    assert L.launch_ggml_moe_unpack(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), 0, 16, 4, 4, 4, 4, 4, 4,
                                    s) == 1
    assert L.launch_ggml_moe_unpack(None, t.data_ptr(), t.data_ptr(), t.data_ptr(), 1, 16, 4, 4, 4, 4, 4, 4, s) == 1
    assert L.launch_ggml_moe_unpack_scatter(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), None, 1, 16, 4,
                                            4, 4, 4, 4, 4, s) == 1
    assert L.launch_ggml_moe_unpack(t.data_ptr(), t.data_ptr(), t.data_ptr(), t.data_ptr(), -3, 16, 4, 4, 4, 4, 4, 4,
                                    s) == 1
    torch.cuda.synchronize()
    assert int(t.sum().item()) == 0
