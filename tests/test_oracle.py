"""Pins the CPU oracle (oracle/zm_oracle.c) before it is trusted as the checker.

Each test is chosen so a plausible restatement mistake (wrong nibble/plane
order, wrong sub-block scale index, dropped mins term, wrong sign/parity,
wrong tie order, wrong rounding) fails it.  CPU only.
"""
import os

import numpy as np
import pytest

import zm_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_dots.npz")


def f32bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------------ golden vectors from the reference's own kernels

@pytest.mark.parametrize("name,t", [("q2_K", O.TYPE_Q2_K), ("q4_K", O.TYPE_Q4_K)])
def test_dot_bit_exact_vs_reference_golden(name, t):
    """oracle dot == ggml stock AVX2 Q2_K (bench/q2k_dot_bench.cpp:31-63) and the
    reference's Q4_K 512-bit dot (bench/q3k_q4k_dot_bench.cpp:73-125), bitwise."""
    g = np.load(GOLDEN, allow_pickle=False)
    for i, nb in enumerate(g[name + "_nb"]):
        w = np.ascontiguousarray(g[name + "_w"][i][: nb * O.BLOCK_BYTES[t]])
        q = np.ascontiguousarray(g[name + "_q8"][i][: nb * 292])
        got = O.vec_dot(t, w, q.view(O.Q8K_DTYPE))
        assert f32bits(got) == f32bits(g[name + "_dot"][i]), (name, i)


@pytest.mark.parametrize("t", [O.TYPE_Q2_K, O.TYPE_Q4_K])
def test_dot_bit_exact_vs_reference_live(t):
    # Looked up inside the test, not at collection: a GPU-only run never maps
    # the reference build.
    R = O.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    fn = R.zmref_dot_q2_K if t == O.TYPE_Q2_K else R.zmref_dot_q4_K
    rng = np.random.default_rng(7)
    for trial in range(300):
        n = 256 * int(rng.integers(1, 17))
        w = O.random_blocks(t, 1, n, seed=trial)[0]
        x = (rng.standard_normal(n) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        q = O.quantize_q8_K(x)
        assert f32bits(O.vec_dot(t, w, q)) == f32bits(fn(n, w.ctypes.data, q.ctypes.data))


# ------------------------------------------------------------------ dequant known answers

def _blank(t):
    return np.zeros(O.BLOCK_BYTES[t], np.uint8)


def _put_half(b, off, v):
    h = np.array([v], np.float16).view(np.uint16)[0]
    b[off] = h & 0xFF
    b[off + 1] = h >> 8


def test_q2_K_known_answer():
    """Single non-zero weight: qs byte 32h+l, bit-plane j (shift 2j) -> weight
    128h + 32j + l, scaled by scales[idx/16] (low nibble), min by the high nibble
    (kquant_matmul.cu:55-72)."""
    for h, j, l in [(0, 0, 0), (0, 3, 17), (1, 1, 5), (1, 2, 31)]:
        b = _blank(O.TYPE_Q2_K)
        _put_half(b, 80, 0.5)     # d
        _put_half(b, 82, 0.25)    # dmin
        idx = 128 * h + 32 * j + l
        b[16 + 32 * h + l] = 3 << (2 * j)
        b[idx // 16] = 6 | (2 << 4)  # scale 6, min 2 for the sub-block holding idx
        y = O.dequantize(O.TYPE_Q2_K, b, 256)[0]
        exp = np.zeros(256, np.float32)
        exp[(idx // 16) * 16:(idx // 16) * 16 + 16] = -0.25 * 2
        exp[idx] = 0.5 * 6 * 3 - 0.25 * 2
        np.testing.assert_array_equal(y, exp)


def test_q3_K_known_answer():
    """hmask bit set = no -4 offset; the hmask byte is hmask[l] for both halves
    (the pointer never advances, kquant_matmul.cu:186-200); scale index 8h+2j+(l>=16),
    6-bit signed (value-32): low nibble in scales[k] (k<8) / high nibble of
    scales[k-8], top 2 bits in scales[8 + k%4] at shift 2*(k/4)."""
    for h, j, l in [(0, 0, 3), (0, 2, 20), (1, 1, 9), (1, 3, 30)]:
        b = _blank(O.TYPE_Q3_K)
        _put_half(b, 108, 0.5)
        b[0:32] = 0xFF           # all high bits set: values q2 in 0..3
        idx = 128 * h + 32 * j + l
        k = idx // 16            # sub-block -> scale index
        sc6 = 32 + 5             # value 5
        lo, hi2 = sc6 & 15, sc6 >> 4
        sc = np.zeros(12, np.uint8)
        sc[:8] = 0x00
        # all other scales -> value -32 (raw 0): set raw 0 already; set k
        if k < 8:
            sc[k] |= lo
        else:
            sc[k - 8] |= lo << 4
        sc[8 + k % 4] |= hi2 << (2 * (k // 4))
        b[96:108] = sc
        b[32 + 32 * h + l] = 2 << (2 * j)
        y = O.dequantize(O.TYPE_Q3_K, b, 256)[0]
        exp = np.zeros(256, np.float32)
        exp[idx] = 0.5 * 5 * 2
        np.testing.assert_array_equal(y, exp)
        # clearing the hmask bit subtracts 4 (for every weight of plane j sharing hmask[l])
        b[l] &= ~np.uint8(1 << (4 * h + j))
        y2 = O.dequantize(O.TYPE_Q3_K, b, 256)[0]
        assert y2[idx] == 0.5 * 5 * (2 - 4)


def test_q4_K_known_answer():
    """qs byte 32c+l: low nibble -> weight 64c+l, high -> 64c+32+l; 6-bit
    (scale, min) of sub-block j from get_scale_min_k4 (kquant_matmul.cu:41-48)."""
    b = _blank(O.TYPE_Q4_K)
    _put_half(b, 0, 0.5)
    _put_half(b, 2, 0.125)
    sc = [1, 2, 3, 4, 5, 6, 7, 8]
    mn = [9, 10, 11, 12, 13, 14, 15, 3]
    raw = np.zeros(12, np.uint8)
    for j in range(4):
        raw[j] = sc[j]
        raw[j + 4] = mn[j]
    for j in range(4, 8):  # values < 16: high 2 bits zero
        raw[j + 4] = sc[j] | (mn[j] << 4)
    # put a 6-bit value in j=5: scale 5+32 -> high bits (>>4)=2 into raw[1]>>6
    raw[1] |= 2 << 6  # j-4 = 1 -> scale high bits of j=5
    sc[5] = 6 | 32
    b[4:16] = raw
    b[16 + 32 * 2 + 7] = 0x9 | (0x4 << 4)  # c=2, l=7: low 9 -> w[135] (sub 4), high 4 -> w[167] (sub 5)
    y = O.dequantize(O.TYPE_Q4_K, b, 256)[0]
    for i in range(256):
        j = i // 32
        q = 9 if i == 135 else (4 if i == 167 else 0)
        assert y[i] == np.float32(0.5 * sc[j]) * q - np.float32(0.125 * mn[j]), i


def test_q5_K_known_answer():
    """Q4_K nibbles and scales plus a fifth bit: bit 2c (low nibble) / 2c+1
    (high nibble) of qh[l] adds 16 to weight 64c+l / 64c+32+l
    (kquant_matmul.cu:94-117)."""
    b = _blank(O.TYPE_Q5_K)
    _put_half(b, 0, 0.5)
    _put_half(b, 2, 0.125)
    sc = [1, 2, 3, 4, 5, 6, 7, 8]
    mn = [9, 10, 11, 12, 13, 14, 15, 3]
    raw = np.zeros(12, np.uint8)
    for j in range(4):
        raw[j] = sc[j]
        raw[j + 4] = mn[j]
    for j in range(4, 8):
        raw[j + 4] = sc[j] | (mn[j] << 4)
    b[4:16] = raw
    qh, qs = 16, 48
    b[qs + 32 * 1 + 9] = 7 | (3 << 4)   # c=1, l=9: w[73] low 7, w[105] high 3
    b[qh + 9] = 1 << 2                   # bit 2c: +16 on w[73] only
    b[qh + 31] = 1 << 7                  # c=3 high half, l=31: w[255] = 16 with a zero nibble
    q = np.zeros(256)
    q[73], q[105], q[255] = 7 + 16, 3, 16
    y = O.dequantize(O.TYPE_Q5_K, b, 256)[0]
    for i in range(256):
        j = i // 32
        assert y[i] == np.float32(0.5 * sc[j]) * q[i] - np.float32(0.125 * mn[j]), i


def test_q6_K_known_answer():
    """Weight 128h+32g+l: low nibble of ql[64h+l] (g=0) / ql[64h+32+l] (g=1),
    high nibbles of the same bytes for g=2,3; two top bits at bit 2g of
    qh[32h+l]; value d*scales[t/16]*(q-32) with signed 8-bit scales
    (kquant_matmul.cu:119-140)."""
    b = _blank(O.TYPE_Q6_K)
    _put_half(b, 208, 0.25)
    scales = np.array([3, -5, 7, -9, 11, -13, 15, -17, 19, -21, 23, -25, 27, -29, 31, -128], np.int8)
    b[192:208] = scales.view(np.uint8)
    b[64 + 32 + 5] = 0xA << 4          # h=1, g=3, l=5 -> t=229: nibble 10
    b[128 + 32 + 5] = 2 << 6           # top bits 2 -> q=42
    b[17] = 3                           # h=0, g=0, l=17 -> t=17: nibble 3
    b[128 + 17] = 1                     # top bits 1 -> q=19
    b[0] = 0xF << 4                     # h=0, g=2, l=0 -> t=64: nibble 15
    b[128 + 0] = 3 << 4                 # top bits 3 -> q=63
    q = np.zeros(256)
    q[229], q[17], q[64] = 42, 19, 63
    y = O.dequantize(O.TYPE_Q6_K, b, 256)[0]
    for t in range(256):
        assert y[t] == np.float32(np.float32(0.25 * scales[t // 16]) * (q[t] - 32)), t


def test_iq4_xs_known_answer():
    """Sub-block ib: 6-bit scale = nibble (ib & 1) of scales_l[ib // 2] plus
    bits 2ib..2ib+1 of scales_h as bits 4-5, value ls - 32; qs byte 16ib + j:
    low nibble -> weight 32ib + j, high -> 32ib + 16 + j, through the table
    (kernels/quant/iq4xs_matmul.cu:80-99)."""
    t = O.iq4nl_table().astype(np.int64)
    b = _blank(O.TYPE_IQ4_XS)
    _put_half(b, 0, 0.5)
    ls = [32, 33, 31, 0, 63, 40, 20, 45]     # values 0, 1, -1, -32, 31, 8, -12, 13
    sh = 0
    for ib, v in enumerate(ls):
        b[4 + ib // 2] |= (v & 15) << (4 * (ib & 1))
        sh |= (v >> 4) << (2 * ib)
    b[2], b[3] = sh & 0xFF, sh >> 8
    b[8 + 16 * 3 + 5] = 0x9 | (0xE << 4)      # ib 3, j 5: w[101] = t[9], w[117] = t[14]
    b[8 + 16 * 6 + 0] = 0xF                   # ib 6, j 0: w[192] = t[15], w[208] = t[0]
    y = O.dequantize(O.TYPE_IQ4_XS, b, 256)[0]
    idx = np.zeros(256, np.int64)
    idx[101], idx[117], idx[192] = 9, 14, 15
    for i in range(256):
        assert y[i] == np.float32(np.float32(0.5 * (ls[i // 32] - 32)) * t[idx[i]]), i
    assert list(t[[0, 8, 15]]) == [-127, 1, 113] and np.all(np.diff(t) > 0)


def test_iq3_xxs_known_answer():
    """Sub-block ib, group l of 8 weights: grid entries qs[8ib + 2l] (weights
    0..3) and qs[8ib + 2l + 1] (4..7), byte j of an entry = weight j; the
    scales+signs word at 64 + 4ib: sign index (u >> 7l) & 127 through
    ksigns, scale d * (0.5 + (u >> 28)) * 0.5 (kernels/quant/iq3_matmul.cu:104-122)."""
    grid = O.iq3xxs_grid()
    b = _blank(O.TYPE_IQ3_XXS)
    _put_half(b, 0, 1.0)
    ib, l = 5, 2
    b[2 + 8 * ib + 2 * l] = 37
    b[2 + 8 * ib + 2 * l + 1] = 200
    sidx = 0b0000011                    # weights 0 and 1 negative (parity even)
    u = (sidx << (7 * l)) | (9 << 28)
    b[2 + 64 + 4 * ib:2 + 64 + 4 * ib + 4] = np.frombuffer(np.uint32(u).tobytes(), np.uint8)
    y = O.dequantize(O.TYPE_IQ3_XXS, b, 256)[0]
    g0 = [(int(grid[0]) >> (8 * j)) & 0xFF for j in range(4)]
    for s in range(8):
        scale = (0.5 + (9 if s == ib else 0)) * 0.5
        for ll in range(4):
            for j in range(8):
                i = 32 * s + 8 * ll + j
                if s == ib and ll == l:
                    e = int(grid[37 if j < 4 else 200]) >> (8 * (j & 3)) & 0xFF
                    exp = scale * e * (-1 if j in (0, 1) else 1)
                else:
                    exp = scale * g0[j & 3]
                assert y[i] == np.float32(exp), (s, ll, j)


def test_iq3_grid_stand_in_properties():
    g = O.iq3xxs_grid()
    assert len(set(g.tolist())) == 256
    levels = {4, 12, 20, 28, 36, 44, 52, 62}
    for v in g.tolist():
        assert {(v >> (8 * j)) & 0xFF for j in range(4)} <= levels


def test_iq2_xxs_known_answer():
    """value = d*(0.5+ls)*0.25*grid[idx][j]*sign, signs = ksigns[7-bit index]
    with the 8th sign = parity (iq2_matmul.cu:73-91, patches/ggml/0009...:69-75)."""
    grid = O.iq2xxs_grid()
    b = _blank(O.TYPE_IQ2_XXS)
    _put_half(b, 0, 1.0)
    ib, l = 3, 2
    gidx = 17
    sidx = 0b0000101  # two negatives -> parity 0
    aux0 = gidx << (8 * l)
    aux1 = (sidx << (7 * l)) | (6 << 28)
    qs = b[2:].view(np.uint16)
    qs[4 * ib + 0] = aux0 & 0xFFFF
    qs[4 * ib + 1] = aux0 >> 16
    qs[4 * ib + 2] = aux1 & 0xFFFF
    qs[4 * ib + 3] = aux1 >> 16
    y = O.dequantize(O.TYPE_IQ2_XXS, b, 256)[0]
    gb = [(int(grid[gidx]) >> (8 * j)) & 0xFF for j in range(8)]
    g0 = [(int(grid[0]) >> (8 * j)) & 0xFF for j in range(8)]
    for s in range(8):
        for ll in range(4):
            for j in range(8):
                i = 32 * s + 8 * ll + j
                if s == ib and ll == l:
                    sign = -1 if j in (0, 2) else 1
                    exp = 1.0 * (0.5 + 6) * 0.25 * gb[j] * sign
                elif s == ib:
                    exp = 1.0 * (0.5 + 6) * 0.25 * g0[j]
                else:
                    exp = 1.0 * 0.5 * 0.25 * g0[j]
                assert y[i] == np.float32(exp), (s, ll, j)
    # odd 7-bit pattern -> the 8th element is negative too
    assert O.ksigns()[1] == 0x81 and O.ksigns()[3] == 0x03 and O.ksigns()[127] == 0xFF


def test_iq2_grid_stand_in_properties():
    g = O.iq2xxs_grid()
    assert len(set(g.tolist())) == 256
    vals = {0x08: 0, 0x19: 1, 0x2B: 2}
    for v in g.tolist():
        digs = [vals[(v >> (8 * j)) & 0xFF] for j in range(8)]
        assert sum(digs) % 2 == 0
    assert int(g[0]) == 0x0808080808080808


# ------------------------------------------------------------------ integer block dots == brute force over dequant

@pytest.mark.parametrize("t", [O.TYPE_Q2_K, O.TYPE_Q3_K, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_IQ2_XXS,
                               O.TYPE_IQ3_XXS, O.TYPE_IQ4_XS])
def test_block_dots_equal_dequant_brute_force(t):
    """sum_j sc*dot - dmin*sum m*bsum per block equals dequant(w).dequant(q8)
    scaled by the block scales, exactly in float64 (integers < 2^53)."""
    rng = np.random.default_rng(3)
    n = 1024
    w = O.random_blocks(t, 1, n, seed=11)[0]
    x = rng.standard_normal(n).astype(np.float32)
    q = O.quantize_q8_K(x)
    isum, imin = O.block_dots(t, w, q)
    wd = O.dequantize(t, w, n)[0].astype(np.float64)
    qv = q["qs"].astype(np.float64).reshape(-1)
    blk = w.reshape(n // 256, O.BLOCK_BYTES[t])
    for b in range(n // 256):
        bb = blk[b]
        if t == O.TYPE_Q2_K:
            d = float(np.frombuffer(bb[80:82].tobytes(), np.float16)[0])
            dm = float(np.frombuffer(bb[82:84].tobytes(), np.float16)[0])
            exp = d * isum[b] - dm * imin[b]
        elif t == O.TYPE_Q3_K:
            exp = float(np.frombuffer(bb[108:110].tobytes(), np.float16)[0]) * isum[b]
        elif t in (O.TYPE_Q4_K, O.TYPE_Q5_K):
            d = float(np.frombuffer(bb[0:2].tobytes(), np.float16)[0])
            dm = float(np.frombuffer(bb[2:4].tobytes(), np.float16)[0])
            exp = d * isum[b] - dm * imin[b]
        elif t == O.TYPE_Q6_K:
            assert imin[b] == 0
            exp = float(np.frombuffer(bb[208:210].tobytes(), np.float16)[0]) * isum[b]
        elif t == O.TYPE_IQ4_XS:
            exp = float(np.frombuffer(bb[0:2].tobytes(), np.float16)[0]) * isum[b]
        elif t == O.TYPE_IQ3_XXS:
            exp = float(np.frombuffer(bb[0:2].tobytes(), np.float16)[0]) * isum[b] / 4.0
        else:
            exp = float(np.frombuffer(bb[0:2].tobytes(), np.float16)[0]) * isum[b] / 8.0
        got = float(np.dot(wd[256 * b:256 * b + 256], qv[256 * b:256 * b + 256]))
        assert abs(got - exp) <= 1e-9 * max(1.0, abs(exp)), (b, got, exp)


@pytest.mark.parametrize("t", [O.TYPE_Q2_K, O.TYPE_Q3_K, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K, O.TYPE_IQ2_XXS,
                               O.TYPE_IQ3_XXS, O.TYPE_IQ4_XS])
def test_vec_dot_matches_dequant_dot(t):
    rng = np.random.default_rng(5)
    n = 2048
    w = O.random_blocks(t, 4, n, seed=2)
    for r in range(4):
        x = rng.standard_normal(n).astype(np.float32)
        q = O.quantize_q8_K(x)
        ref = float(np.dot(O.dequantize(t, w[r], n)[0].astype(np.float64),
                           O.dequantize(O.TYPE_Q8_K, q, n)[0].astype(np.float64)))
        got = O.vec_dot(t, w[r], q)
        assert abs(got - ref) <= 1e-5 * max(1e-3, abs(ref)) + 1e-6


# ------------------------------------------------------------------ Q8_K quantization closed forms

def test_q8_K_closed_forms():
    x = np.zeros(256, np.float32)
    x[:6] = [-127, 0.5, 1.5, 2.5, -0.5, -1.5]   # max=-127 -> iscale = 1: round half even
    q = O.quantize_q8_K(x)[0]
    assert q["d"] == 1.0
    np.testing.assert_array_equal(q["qs"][:6], [-127, 0, 2, 2, 0, -2])
    assert q["bsums"][0] == -127 + 0 + 2 + 2 + 0 - 2
    # first maximal |x| wins the sign: [-2, 2] -> max = -2, iscale = 63.5
    x = np.zeros(256, np.float32)
    x[10], x[20] = -2.0, 2.0
    q = O.quantize_q8_K(x)[0]
    assert q["qs"][10] == -127 and q["qs"][20] == 127
    assert q["d"] == np.float32(1.0) / np.float32(-127.0 / -2.0)
    x[10], x[20] = 2.0, -2.0
    q = O.quantize_q8_K(x)[0]
    assert q["qs"][10] == -127 and q["qs"][20] == 127  # iscale = -63.5 now
    # all zero
    q = O.quantize_q8_K(np.zeros(256, np.float32))[0]
    assert q["d"] == 0 and not q["qs"].any() and not q["bsums"].any()
    # 16-sums of a random row
    x = np.random.default_rng(1).standard_normal(512).astype(np.float32)
    q = O.quantize_q8_K(x)
    for b in range(2):
        np.testing.assert_array_equal(q[b]["bsums"], q[b]["qs"].astype(np.int32).reshape(16, 16).sum(1))
        assert np.abs(q[b]["qs"]).max() == 127


def test_q8_K_matches_reference_rounding_restatement():
    """The reference's own statement of Q8_K rounding
    (tests/test_real_tensor_numerics.cpp:115-126: the signed value of largest
    magnitude, scale |max|/127, q = nearbyint(v / scale) clamped to +-127),
    evaluated here in float64: the oracle's d has that magnitude with the sign
    opposite to max (iscale = -127/max), and every q equals the reference's
    -q except where v/scale sits within float rounding of a half-integer."""
    rng = np.random.default_rng(12)
    for trial in range(40):
        x = (rng.standard_normal(256 * 4) * 10.0 ** rng.uniform(-4, 4)).astype(np.float32)
        q = O.quantize_q8_K(x)
        for b in range(4):
            v = x[256 * b: 256 * (b + 1)].astype(np.float64)
            i = int(np.argmax(np.abs(v)))  # first maximal magnitude
            mx = v[i]
            scale = abs(mx) / 127.0
            qr = np.clip(np.rint(v / scale), -127, 127)
            near_half = np.abs(np.abs(v / scale - np.floor(v / scale)) - 0.5) < 1e-4
            got = q[b]["qs"].astype(np.float64)
            # ggml's iscale = -127/max flips the sign when max > 0
            sgn = -1.0 if mx > 0 else 1.0
            ok = (got == sgn * qr) | near_half
            assert ok.all(), (trial, b, np.nonzero(~ok)[0][:5])
            assert abs(abs(float(q[b]["d"])) - scale) <= 1e-6 * scale
            assert np.sign(float(q[b]["d"])) == -np.sign(mx)


# ------------------------------------------------------------------ float helpers

def test_fp16_conversions_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.fp16_to_fp32(int(v)) for v in h[::97]], np.float32)
    np.testing.assert_array_equal(f32bits(got)[~np.isnan(ref[::97])], f32bits(ref[::97])[~np.isnan(ref[::97])])
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.uniform(-9, 5, 3000),
                         [65504, 65519.9, 65520, 6e-8, 2.9e-8, 3e-8, 0.0, -0.0]]).astype(np.float32)
    for v in xs:
        assert O.fp32_to_fp16(float(v)) == np.float16(v).view(np.uint16), v


def test_expf_accuracy():
    xs = np.linspace(-100, 88, 200001).astype(np.float32)
    got = np.array([O.expf(float(v)) for v in xs[::13]], np.float64)
    ref = np.exp(xs[::13].astype(np.float64))
    ok = ref > 1.2e-38  # normal range
    ulp = np.abs(got[ok] - ref[ok]) / np.spacing(ref[ok].astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 2.0, ulp.max()
    assert O.expf(0.0) == 1.0 and O.expf(-1000.0) == 0.0 and O.expf(1000.0) == np.inf


# ------------------------------------------------------------------ router / bucketing (brute force)

def _router_np(logits, K, gating, logit_bias=None, sel_bias=None, G=0, GU=0, norm=False, scale=0.0):
    S, E = logits.shape
    ids = np.zeros((S, K), np.int32)
    w = np.zeros((S, K), np.float32)
    for s in range(S):
        l = logits[s].astype(np.float32)
        if logit_bias is not None:
            l = (l + logit_bias).astype(np.float32)
        if gating == O.GATING_SOFTMAX:
            e = np.array([O.expf(float(v - l.max())) for v in l], np.float32)
            p = (e * np.float32(1.0 / e.astype(np.float64).sum())).astype(np.float32)
        else:
            p = np.array([1.0 / (1.0 + O.expf(float(-v))) for v in l], np.float32)
        sel = p if sel_bias is None else (p + sel_bias).astype(np.float32)
        sel = sel.copy()
        if G > 1 and 0 < GU < G:
            gs = E // G
            sc = []
            for g in range(G):
                v = sel[g * gs:(g + 1) * gs]
                o = sorted(range(gs), key=lambda j: (-v[j], j))
                sc.append(np.float32(v[o[0]] + v[o[1]]))
            keep = sorted(range(G), key=lambda g: (-sc[g], g))[:GU]
            for e_ in range(E):
                if e_ // gs not in keep:
                    sel[e_] = -np.inf
        order = sorted(range(E), key=lambda e_: (-sel[e_], e_))[:K]
        ids[s] = order
        w[s] = p[order]
        if norm:
            sm = np.float32(w[s].astype(np.float64).sum())
            w[s] = w[s] / max(sm, np.float32(6.103515625e-5))
        if scale not in (0.0, 1.0):
            w[s] = w[s] * np.float32(scale)
    return ids, w


@pytest.mark.parametrize("case", ["softmax", "softmax_bias", "sigmoid_groups", "ties"])
def test_router_brute_force(case):
    rng = np.random.default_rng(9)
    if case == "softmax":
        lg = rng.standard_normal((5, 128)).astype(np.float32)
        args = dict(K=8, gating=O.GATING_SOFTMAX)
    elif case == "softmax_bias":
        lg = rng.standard_normal((5, 128)).astype(np.float32)
        args = dict(K=8, gating=O.GATING_SOFTMAX, logit_bias=(rng.standard_normal(128) * 1.5).astype(np.float32),
                    norm=True)
    elif case == "sigmoid_groups":
        lg = rng.standard_normal((4, 256)).astype(np.float32)
        args = dict(K=8, gating=O.GATING_SIGMOID, sel_bias=(rng.standard_normal(256) * 0.1).astype(np.float32),
                    G=8, GU=4, norm=True, scale=2.5)
    else:
        lg = np.round(rng.standard_normal((6, 64)) * 2).astype(np.float32)  # many exact ties
        args = dict(K=6, gating=O.GATING_SOFTMAX)
    ids, w = O.router(lg, args["K"], args["gating"], args.get("logit_bias"), args.get("sel_bias"),
                      args.get("G", 0), args.get("GU", 0), args.get("norm", False), args.get("scale", 0.0))
    ri, rw = _router_np(lg, **args)
    np.testing.assert_array_equal(ids, ri)
    np.testing.assert_allclose(w, rw, rtol=2e-7, atol=0)


def test_bucket_is_stable_counting_sort():
    rng = np.random.default_rng(4)
    S, K, E = 200, 8, 40
    ids = rng.integers(-1, E, size=(S, K)).astype(np.int32)
    counts, offs, pairs = O.bucket(ids, E)
    flat = ids.reshape(-1)
    valid = np.nonzero(flat >= 0)[0]
    order = valid[np.argsort(flat[valid], kind="stable")]
    np.testing.assert_array_equal(pairs, order)
    np.testing.assert_array_equal(counts, np.bincount(flat[valid], minlength=E))
    np.testing.assert_array_equal(offs, np.concatenate([[0], np.cumsum(counts)]))


def test_slot_table():
    rmap = np.array([3, -1, 0, 1, -1, 2], np.int32)
    ids = np.array([[0, 1, 2], [5, 4, 3]], np.int32)
    w = np.array([[0.5, 0.25, 0.25], [0.1, 0.2, 0.7]], np.float32)
    i2, w2 = O.apply_slot_table(rmap, ids, w)
    np.testing.assert_array_equal(i2, [[3, -1, 0], [2, -1, 1]])
    np.testing.assert_array_equal(w2, np.array([[0.5, 0.0, 0.25], [0.1, 0.0, 0.7]], np.float32))


# ------------------------------------------------------------------ op semantics

@pytest.mark.parametrize("t", [O.TYPE_Q2_K, O.TYPE_Q3_K, O.TYPE_Q4_K, O.TYPE_IQ2_XXS])
def test_mul_mat_id_semantics(t):
    """dst[t,id] = vec_dot(W[ids], q8(x[id % ne11])); id < 0 -> zeros
    (patches/ggml/0002...:46-58); ids like bench/mmid_exact_check.cpp:41."""
    I, O_, E, n_ids, S = 512, 8, 24, 10, 2
    W = O.random_blocks(t, E * O_, I, seed=t).reshape(E, O_, -1)
    rng = np.random.default_rng(11)
    ids = np.array([[3, -1, 17, -1, -1, 8, -1, -1, -1, 21], [0, 1, 2, 3, 4, 5, 6, 7, 23, -1]], np.int32)
    for ne11 in (1, n_ids):
        x = rng.standard_normal((S, ne11, I)).astype(np.float32)
        y = O.mul_mat_id(t, W, x, ids)
        for s in range(S):
            for k in range(n_ids):
                e = ids[s, k]
                if e < 0:
                    assert not y[s, k].any()
                    continue
                q = O.quantize_q8_K(x[s, k % ne11])
                for r in range(O_):
                    assert f32bits(y[s, k, r]) == f32bits(O.vec_dot(t, W[e, r], q))
    # multithreaded == single threaded, bitwise
    x = rng.standard_normal((S, 1, I)).astype(np.float32)
    np.testing.assert_array_equal(O.mul_mat_id(t, W, x, ids, 1), O.mul_mat_id(t, W, x, ids, 4))


def test_moe_forward_composition():
    """moe_forward == mul_mat_id(gate/up) -> swiglu -> mul_mat_id(down) ->
    ((w0*y0 + w1*y1) + ...) with float32 rounding at every step."""
    H, F, E, K, S = 512, 256, 6, 3, 2
    tg, td = O.TYPE_Q4_K, O.TYPE_Q3_K
    Wg = O.random_blocks(tg, E * F, H, 1).reshape(E, F, -1)
    Wu = O.random_blocks(tg, E * F, H, 2).reshape(E, F, -1)
    Wd = O.random_blocks(td, E * H, F, 3).reshape(E, H, -1)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((S, H)).astype(np.float32)
    ids = np.array([[1, 4, -1], [5, 0, 2]], np.int32)
    w = np.array([[0.5, 0.3, 0.2], [0.6, 0.25, 0.15]], np.float32)
    out = O.moe_forward(x, ids, w, tg, tg, td, Wg, Wu, Wd)
    g = O.mul_mat_id(tg, Wg, x[:, None, :], ids)
    u = O.mul_mat_id(tg, Wu, x[:, None, :], ids)
    a = O.swiglu(g, u)
    d = O.mul_mat_id(td, Wd, a, ids)
    ref = np.zeros((S, H), np.float32)
    for s in range(S):
        acc = (w[s, 0] * d[s, 0]).astype(np.float32)
        for k in range(1, K):
            acc = (acc + (w[s, k] * d[s, k]).astype(np.float32)).astype(np.float32)
        ref[s] = acc
    np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("t,tol", [(O.TYPE_Q2_K, 0.40), (O.TYPE_Q3_K, 0.20), (O.TYPE_Q4_K, 0.09),
                                   (O.TYPE_Q5_K, 0.045), (O.TYPE_Q6_K, 0.025), (O.TYPE_IQ2_XXS, 0.40),
                                   (O.TYPE_IQ4_XS, 0.12), (O.TYPE_IQ3_XXS, 0.3)])
def test_quantizer_round_trip(t, tol):
    x = O.fill_normal(42, 8 * 1024, 0.0, 0.02).reshape(8, 1024)
    y = O.dequantize(t, O.quantize(t, x), 1024)
    rel = np.sqrt(((x - y) ** 2).mean() / (x ** 2).mean())
    assert rel < tol, rel


def _f16_bytes(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def _q2_K_block(d, dmin, sc, m, q):
    """GGUF block_q2_K from its fields (scales: low nibble sc, high nibble m;
    q of weight l at bits 2j of qs[32*(l // 128) + l % 32], j = (l % 128) // 32)."""
    b = np.zeros(84, np.uint8)
    b[0:16] = (sc & 15) | ((m & 15) << 4)
    for l in range(256):
        half, r = divmod(l, 128)
        j, ll = divmod(r, 32)
        b[16 + 32 * half + ll] |= (q[l] & 3) << (2 * j)
    b[80:82], b[82:84] = _f16_bytes(d), _f16_bytes(dmin)
    return b


def _q3_K_block(d, sc, q):
    """GGUF block_q3_K: q in [-4, 3] (low 2 bits in qs as for Q2_K, hmask bit
    l // 32 of byte l % 32 set when q >= 0), 6-bit scales sc (value sc - 32)."""
    b = np.zeros(110, np.uint8)
    u = q + 4
    for l in range(256):
        half, r = divmod(l, 128)
        j, ll = divmod(r, 32)
        b[32 + 32 * half + ll] |= (u[l] & 3) << (2 * j)
        if u[l] & 4:
            b[ll] |= 1 << (l // 32)
    for j in range(16):
        b[96 + (j % 8)] |= (sc[j] & 15) << (4 * (j // 8))
        b[96 + 8 + j % 4] |= (sc[j] >> 4) << (2 * (j // 4))
    b[108:110] = _f16_bytes(d)
    return b


def _q4_K_block(d, dmin, sc, m, q):
    """GGUF block_q4_K: 6-bit (sc, m) packed as get_scale_min_k4 reads them,
    sub-blocks 2i / 2i+1 in the low / high nibbles of qs[32i .. 32i+31]."""
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = _f16_bytes(d), _f16_bytes(dmin)
    for j in range(8):
        if j < 4:
            b[4 + j] = sc[j]
            b[8 + j] = m[j]
        else:
            b[12 + j - 4] = (sc[j] & 15) | ((m[j] & 15) << 4)
            b[4 + j - 4] |= (sc[j] >> 4) << 6
            b[8 + j - 4] |= (m[j] >> 4) << 6
    for i in range(4):
        b[16 + 32 * i:48 + 32 * i] = q[64 * i:64 * i + 32] | (q[64 * i + 32:64 * i + 64] << 4)
    return b


@pytest.mark.parametrize("t", [O.TYPE_Q2_K, O.TYPE_Q3_K, O.TYPE_Q4_K])
def test_quantizer_reproduces_representable_blocks(t):
    """A block built from chosen fields is exactly representable; quantizing its
    dequantized values must give back the identical values.  Each sub-block
    holds both ends of its quant range and the largest scale and min sit at the
    top of their field (Q3_K: the largest-magnitude scale is -32 and every
    sub-block holds q = -4, the value the quantizer maps to the scale), so the
    optimal scales are unique: a wrong scale search, rounding or packing in the
    restated ggml quantizers fails here."""
    rng = np.random.default_rng(100 + t)
    for _ in range(60):
        d, dmin = (float(np.float16(rng.uniform(1e-4, 1e-3))) for _ in range(2))
        if t == O.TYPE_Q2_K:
            sc, m = rng.integers(1, 16, 16), rng.integers(0, 16, 16)
            sc[rng.integers(16)] = 15
            m[rng.integers(16)] = 15
            q = rng.integers(0, 4, 256)
            q[0::16], q[1::16] = 0, 3
            blk = _q2_K_block(d, dmin, sc, m, q)
        elif t == O.TYPE_Q3_K:
            v = rng.integers(1, 32, 16) * rng.choice([-1, 1], 16)
            v[rng.integers(16)] = -32
            q = rng.integers(-4, 4, 256)
            q[0::16] = -4
            blk = _q3_K_block(d, v + 32, q)
        else:
            sc, m = rng.integers(1, 64, 8), rng.integers(0, 64, 8)
            sc[rng.integers(8)] = 63
            m[rng.integers(8)] = 63
            q = rng.integers(0, 16, 256)
            q[0::32], q[1::32] = 0, 15
            blk = _q4_K_block(d, dmin, sc, m, q)
        x = O.dequantize(t, blk[None, :], 256)
        np.testing.assert_array_equal(O.dequantize(t, O.quantize(t, x), 256), x)


# ------------------------------------------------------------------ FP32-activation path restatements


@pytest.mark.parametrize("t", [O.TYPE_Q2_K, O.TYPE_Q3_K, O.TYPE_Q4_K, O.TYPE_IQ2_XXS])
def test_f32_matmul_equals_integer_dot_on_exact_activations(t):
    """With x = q * 2^-7 (int8 q, |q| = 127 present in every block) the Q8_K
    quantization is exact, so ggml's integer block dot (pinned by the
    reference's golden vectors above) and the f32 dequant dot must agree to
    float rounding: a wrong dequant plane, scale index or sign fails."""
    rng = np.random.default_rng(31)
    I, Orows, S = 1024, 6, 3
    W = O.random_blocks(t, Orows, I, seed=5)
    q = rng.integers(-127, 128, size=(S, I)).astype(np.float32)
    q[:, ::256] = 127.0
    x = q * np.float32(2.0 ** -7)
    y = O.f32_matmul(t, W, x)
    bound = O.f32_matmul_absbound(t, W, x)
    for s in range(S):
        xq = O.quantize_q8_K(x[s])
        for o in range(Orows):
            ref = O.vec_dot(t, W[o], xq)
            assert abs(y[s, o] - ref) <= 2e-6 * bound[s, o] + 1e-30, (s, o, y[s, o], ref)


def test_f32_matmul_is_linear_in_x():
    W = O.random_blocks(O.TYPE_Q3_K, 4, 512, seed=2)
    rng = np.random.default_rng(3)
    a, b = rng.standard_normal((2, 512)).astype(np.float32)
    ya, yb, yab = O.f32_matmul(O.TYPE_Q3_K, W, a), O.f32_matmul(O.TYPE_Q3_K, W, b), O.f32_matmul(O.TYPE_Q3_K, W, a + b)
    np.testing.assert_allclose(yab, ya + yb, rtol=1e-6, atol=1e-6)


def test_expert_swiglu_closed_forms():
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 5.0, 2.0, np.nan, np.inf, 1.0], np.float32)
    u = np.array([3.0, 0.0, 2.0, 1.0, 1.0, 5.0, -9.0, 1.0, 1.0, -np.inf], np.float32)
    out, bad = O.expert_swiglu(g, u)
    assert bad == [1, 2]
    assert out[0] == 0.0 and out[1] == 0.0
    np.testing.assert_allclose(out[2], -2.0 / (1.0 + np.e), rtol=1e-6)
    np.testing.assert_allclose(out[3], 30.0, rtol=1e-6)  # silu(30) = 30 (to f32)
    assert abs(out[4]) < 1e-11
    # unclamped default == the layer oracle's SwiGLU, bit for bit
    fin = np.isfinite(g) & np.isfinite(u)
    np.testing.assert_array_equal(f32bits(out[fin]), f32bits(O.swiglu(g[fin], u[fin])))
    # default clamp acts on the product; fused clamp on the inputs
    oc, _ = O.expert_swiglu(g[:7], u[:7], clamp=7.0)
    np.testing.assert_allclose(oc[5], 7.0)           # silu(5)*5 = 24.8 -> 7
    np.testing.assert_allclose(oc[6], -7.0)          # silu(2)*(-9) = -15.9 -> -7
    of, _ = O.expert_swiglu(g[:7], u[:7], clamp=4.0, fused=True)
    np.testing.assert_allclose(of[5], 4.0 / (1.0 + np.exp(-4.0)) * 4.0, rtol=1e-6)  # min(g,4), clamp(u,4)
    np.testing.assert_allclose(of[6], 2.0 / (1.0 + np.exp(-2.0)) * -4.0, rtol=1e-6)
    # fused without a clamp is the plain SwiGLU
    o0, _ = O.expert_swiglu(g[:7], u[:7], fused=True)
    np.testing.assert_array_equal(f32bits(o0), f32bits(out[:7]))


def test_scatter_accum_brute_force():
    rng = np.random.default_rng(4)
    n, D, S = 9, 33, 6
    src = rng.standard_normal((n, D)).astype(np.float32)
    tok = np.array([3, 0, 5, -1, 6, 1, 2, 4, 100], np.int32)  # -1, 6, 100: skipped
    w = rng.random(n).astype(np.float32)
    dst0 = rng.standard_normal((S, D)).astype(np.float32)
    got = O.scatter_accum(src, tok, dst0, w)
    want = dst0.astype(np.float64).copy()
    for i in range(n):
        if 0 <= tok[i] < S:
            want[tok[i]] += float(w[i]) * src[i].astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(got[[i for i in range(S) if i not in tok]], dst0[[i for i in range(S) if i not in tok]])
    plain = O.scatter_accum(src, tok, dst0)
    np.testing.assert_allclose(plain[3], dst0[3] + src[0], rtol=1e-6)


@pytest.mark.parametrize("gating,bias,norm,scale", [(O.GATING_SOFTMAX, False, False, 0.0),
                                                     (O.GATING_SOFTMAX, True, True, 0.0),
                                                     (O.GATING_SIGMOID, True, True, 2.5),
                                                     (O.GATING_SQRT_SOFTPLUS, False, True, 1.0)])
def test_glm_router_matches_layer_router(gating, bias, norm, scale):
    """Two independent restatements of the same router (glm5next_router.cu's
    scan and moe_routed's select/gather, the latter pinned by brute force
    above) must choose the same ids and weights."""
    rng = np.random.default_rng(12)
    S, E, K = 7, 96, 6
    lg = rng.standard_normal((S, E)).astype(np.float32)
    b = (rng.standard_normal(E) * 0.5).astype(np.float32) if bias else None
    row, ids, w = O.glm5next_router_topk(lg, K, b, gating, norm, scale)
    ri, rw = O.router(lg, K, gating, None, b, 0, 0, norm, scale)
    np.testing.assert_array_equal(ids, ri)
    np.testing.assert_allclose(w, rw, rtol=2e-6)
    # the row left behind: probabilities with the chosen ones at -FLT_MAX
    for s in range(S):
        assert np.all(row[s, ids[s]] == np.float32(-3.402823466e38))
        rest = np.delete(row[s], ids[s])
        assert np.all((rest >= 0) & (rest <= 1.5 if gating != O.GATING_SOFTMAX else rest <= 1))
    if gating == O.GATING_SOFTMAX:
        p = row.copy()
        for s in range(S):
            p[s, ids[s]] = w[s] if not norm else 0
        if not norm:
            np.testing.assert_allclose(p.sum(1), 1.0, rtol=1e-5)


def test_glm_router_ties_and_nan():
    lg = np.zeros((1, 10), np.float32)
    _, ids, w = O.glm5next_router_topk(lg, 4)
    assert list(ids[0]) == [0, 1, 2, 3]  # equal scores: lower index first
    lg = np.array([[np.nan, 5, 4, 3]], np.float32)
    _, ids, _ = O.glm5next_router_topk(lg, 2, gating=O.GATING_SIGMOID)
    assert list(ids[0]) == [0, 1]  # a NaN at expert 0 seeds the scan and is never displaced
    lg = np.array([[1, np.nan, 4, 3]], np.float32)
    _, ids, _ = O.glm5next_router_topk(lg, 3, gating=O.GATING_SIGMOID)
    assert list(ids[0]) == [2, 3, 0]  # a NaN elsewhere is never chosen


# ------------------------------------------------------------------ expert records

def test_moe_unpack_known_answer():
    """Two 10-byte records [g g g | u u | d d d d d] + 2 bytes padding: the
    hand-written destination bytes (kernels/math/ggml_moe_pack.cu:39-60)."""
    src = np.arange(24, dtype=np.uint8)
    g, u, d = (np.full(n, 255, np.uint8) for n in (8, 6, 12))
    O.moe_unpack(src, g, u, d, 2, 12, (3, 2, 5), dst_strides=(4, 3, 6))
    np.testing.assert_array_equal(g, [0, 1, 2, 255, 12, 13, 14, 255])
    np.testing.assert_array_equal(u, [3, 4, 255, 15, 16, 255])
    np.testing.assert_array_equal(d, [5, 6, 7, 8, 9, 255, 17, 18, 19, 20, 21, 255])


def test_moe_unpack_inverts_pack_and_scatter_skips():
    """pack (rows concatenated per expert) then scatter-unpack into fresh
    tensors gives back exactly the packed experts' bytes; slot -1 records and
    the bytes between experts stay untouched."""
    rng = np.random.default_rng(3)
    parts, strides, E = (1344, 1344, 1760), (1408, 1344, 1792), 6
    planar = [rng.integers(0, 256, E * s, dtype=np.uint8) for s in strides]
    experts = [4, 0, 5, 2]
    rs = sum(parts) + 48
    src = O.moe_pack(*planar, experts, rs, parts, strides, fill=0xAB)
    slots = np.array([4, -1, 5, 2], np.int32)
    out = [np.full(E * s, 7, np.uint8) for s in strides]
    O.moe_unpack(src, *out, 4, rs, parts, strides, slots)
    for p in range(3):
        for e in range(E):
            lo, hi = e * strides[p], e * strides[p] + parts[p]
            want = planar[p][lo:hi] if e in (4, 5, 2) else np.full(parts[p], 7, np.uint8)
            np.testing.assert_array_equal(out[p][lo:hi], want)
            np.testing.assert_array_equal(out[p][hi:(e + 1) * strides[p]], 7)


# ------------------------------------------------------------------ AVX-512 CPU baseline

@pytest.mark.parametrize("t", [O.TYPE_Q2_K, O.TYPE_Q3_K])
def test_avx512_dots_bit_identical_to_oracle(t):
    """The CPU baseline's VNNI dots equal the oracle dots bit for bit (random
    blocks over a wide range of scales, every hmask / scale pattern); Q2_K
    also against the reference's golden vectors."""
    if not O.has_avx512():
        pytest.skip("host without AVX-512 VNNI")
    rng = np.random.default_rng(30 + t)
    for trial in range(200):
        nb = int(rng.integers(1, 17))
        w = O.random_blocks(t, 1, 256 * nb, seed=1000 + trial)[0]
        x = (rng.standard_normal(256 * nb) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
        q = O.quantize_q8_K(x)
        assert f32bits(O.vec_dot_fast(t, w, q)) == f32bits(O.vec_dot(t, w, q)), trial
    if t == O.TYPE_Q2_K:
        g = np.load(GOLDEN, allow_pickle=False)
        for i, nb in enumerate(g["q2_K_nb"]):
            w = np.ascontiguousarray(g["q2_K_w"][i][: nb * O.BLOCK_BYTES[t]])
            q = np.ascontiguousarray(g["q2_K_q8"][i][: nb * 292]).view(O.Q8K_DTYPE)
            assert f32bits(O.vec_dot_fast(t, w, q)) == f32bits(g["q2_K_dot"][i]), i


def test_avx512_layer_bit_identical_to_oracle():
    """zmo_moe_forward_fast (the CPU baseline: two parallel regions, serial
    Q8_K) equals zmo_moe_forward on a c2-shaped layer with a skipped route."""
    rng = np.random.default_rng(3)
    H, F, E, K = 1024, 512, 6, 4
    Wg = O.random_blocks(O.TYPE_Q2_K, E * F, H, seed=1).reshape(E, F, -1)
    Wu = O.random_blocks(O.TYPE_Q2_K, E * F, H, seed=2).reshape(E, F, -1)
    Wd = O.random_blocks(O.TYPE_Q3_K, E * H, F, seed=3).reshape(E, H, -1)
    x = rng.standard_normal((2, H)).astype(np.float32)
    ids = np.array([[3, 0, 5, 1], [2, -1, 4, 0]], np.int32)
    w = rng.uniform(0.1, 0.4, (2, K)).astype(np.float32)
    ref = O.moe_forward(x, ids, w, O.TYPE_Q2_K, O.TYPE_Q2_K, O.TYPE_Q3_K, Wg, Wu, Wd, nthreads=4)
    got = O.moe_forward(x, ids, w, O.TYPE_Q2_K, O.TYPE_Q2_K, O.TYPE_Q3_K, Wg, Wu, Wd, nthreads=4, fast=True)
    np.testing.assert_array_equal(f32bits(got), f32bits(ref))
