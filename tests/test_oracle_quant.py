"""CPU pins of the oracle's quantization layer (f16, q8_row, q4_tiled, q4tp)
and of its exact / a8w8 matvecs, against known answers, closed forms and
brute force -- not against a retyped copy of the oracle's own formulas."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc

DT_Q8ROW, DT_Q4T, DT_Q4TP = 3, 11, 15


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _dequant(t):
    L = orc.lib()
    rows, cols = t["rows"], t["cols"]
    out = np.empty(rows * cols, dtype=np.float32)
    if t["dtype"] == DT_Q8ROW:
        return t["q"].astype(np.float32) * t["row_scale"][:, None]
    b = np.ascontiguousarray(t["bytes"], dtype=np.uint8)
    if t["dtype"] == DT_Q4T:
        L.or_dequant_q4t(_p(b), rows * cols, _p(out))
    else:
        L.or_dequant_q4tp(_p(b), rows, cols, _p(out))
    return out.reshape(rows, cols)


# ---------------------------------------------------------------- f16 ----
def test_f16_known_answers():
    """quant.rs:872-891 known answers (subnormals and the smallest normal)."""
    L = orc.lib()
    cases = {0x0001: 5.9604645e-8, 0x03FF: 6.097555e-5, 0x812B: -1.7821789e-5, 0x0400: 6.1035156e-5,
             0x3C00: 1.0, 0xC000: -2.0, 0x7BFF: 65504.0}
    for h, v in cases.items():
        assert L.or_f16_to_f32(h) == np.float32(v), hex(h)


def test_f16_exhaustive_against_ieee():
    """every finite half decodes to the IEEE binary16 value and round-trips"""
    L = orc.lib()
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(x)) for x in h], dtype=np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin], ref[fin])
    back = np.array([L.or_f32_to_f16(float(v)) for v in ref[fin]], dtype=np.uint16)
    same = back == h[fin]
    # +0 / -0 are the only halves allowed to map onto each other
    assert np.all(same | (ref[fin] == 0))


def test_f32_to_f16_rounds_to_nearest_even():
    L = orc.lib()
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(20000) * np.exp2(rng.integers(-20, 14, 20000))).astype(np.float32)
    got = np.array([L.or_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


# ------------------------------------------------------------- layouts ----
def test_q8_row_layout_closed_form():
    """disk q8_row: rows*cols int8 row-major, then one f16 scale per row"""
    rows, cols = 3, 5
    q = np.array([[1, -2, 3, -4, 127], [0, 0, 0, 0, 0], [-127, 5, 6, 7, 8]], dtype=np.int8)
    s = np.array([0.5, 2.0, -0.25], dtype=np.float16)
    b = np.concatenate([q.view(np.uint8).ravel(), s.view(np.uint8)])
    out = np.empty(rows * cols, dtype=np.float32)
    orc.lib().or_dequant_q8_row(_p(b), rows, cols, _p(out))
    assert np.array_equal(out.reshape(rows, cols), q.astype(np.float32) * s.astype(np.float32)[:, None])


def _q4t_tile(scale, nibbles):
    """18-byte tile: f16 scale, then 16 bytes with element 2k in the low nibble"""
    n = np.asarray(nibbles, dtype=np.uint8)
    return np.concatenate([np.array([scale], dtype=np.float16).view(np.uint8),
                           (n[0::2] | (n[1::2] << 4)).astype(np.uint8)])


def test_q4t_tile_closed_form():
    nib = np.arange(32) % 16
    b = np.concatenate([_q4t_tile(0.5, nib), _q4t_tile(-3.0, nib[::-1])])
    out = np.empty(64, dtype=np.float32)
    orc.lib().or_dequant_q4t(_p(b), 64, _p(out))
    want = np.concatenate([(nib - 8) * 0.5, (nib[::-1] - 8) * -3.0]).astype(np.float32)
    assert np.array_equal(out, want)


def _q4tp_bytes(nibs, lo, step, codes):
    """rows x gpr tiles: [16 B nibbles per tile] [f16 lo, f16 step per row]
    [5-bit codes, LSB first, ceil(gpr*5/8) bytes per row]"""
    rows, gpr = codes.shape
    nib = np.concatenate([(n[0::2] | (n[1::2] << 4)).astype(np.uint8) for n in nibs.reshape(-1, 32)])
    params = np.stack([np.asarray(lo, np.float16), np.asarray(step, np.float16)], axis=1).view(np.uint8).ravel()
    stride = (gpr * 5 + 7) // 8
    cb = np.zeros((rows, stride), dtype=np.uint8)
    for r in range(rows):
        bits = 0
        for g in range(gpr):
            bits |= int(codes[r, g]) << (5 * g)
        cb[r] = np.frombuffer(bits.to_bytes(stride, "little"), dtype=np.uint8)
    return np.concatenate([nib, params, cb.ravel()])


def test_q4tp_ladder_closed_form():
    """lo = 0, step = 1 gives the exact ladder 2^c; codes spanning byte edges"""
    rows, gpr = 2, 7
    rng = np.random.default_rng(1)
    nibs = rng.integers(0, 16, (rows, gpr, 32)).astype(np.uint8)
    codes = np.array([[0, 31, 7, 13, 1, 30, 16], [5, 5, 0, 22, 9, 31, 2]])
    b = _q4tp_bytes(nibs, [0.0, -1.0], [1.0, 1.0], codes)
    L = orc.lib()
    stride = (gpr * 5 + 7) // 8
    off = rows * gpr * 16 + rows * 4
    for r in range(rows):
        for g in range(gpr):
            assert L.or_q4tp_code(_p(b[off + r * stride:]), stride, g) == codes[r, g]
    out = np.empty(rows * gpr * 32, dtype=np.float32)
    L.or_dequant_q4tp(_p(b), rows, gpr * 32, _p(out))
    scale = np.exp2(codes + np.array([[0.0], [-1.0]]))
    want = (nibs.astype(np.float32) - 8.0) * scale[:, :, None]
    assert np.array_equal(out.reshape(rows, gpr, 32), want.astype(np.float32))


def test_q4tp_put_code_roundtrip():
    L = orc.lib()
    rng = np.random.default_rng(2)
    for gpr in (1, 3, 8, 13, 128):
        codes = rng.integers(0, 32, gpr)
        buf = np.zeros((gpr * 5 + 7) // 8, dtype=np.uint8)
        for g, c in enumerate(codes):
            L.or_q4tp_put_code(_p(buf), g, int(c))
        assert [L.or_q4tp_code(_p(buf), len(buf), g) for g in range(gpr)] == codes.tolist()


def test_q4tp_step0_equals_q4t():
    """tests/gpu_q4tp_batch.rs:23-48: step 0, any code == q4t at scale 2^lo"""
    rows, gpr = 3, 4
    rng = np.random.default_rng(4)
    nibs = rng.integers(0, 16, (rows, gpr, 32)).astype(np.uint8)
    lo = np.array([-2.0, -5.0, 1.0])
    b = _q4tp_bytes(nibs, lo, [0.0] * rows, rng.integers(0, 32, (rows, gpr)))
    out = np.empty(rows * gpr * 32, dtype=np.float32)
    orc.lib().or_dequant_q4tp(_p(b), rows, gpr * 32, _p(out))
    tiles = np.concatenate([_q4t_tile(2.0 ** lo[r], nibs[r, g]) for r in range(rows) for g in range(gpr)])
    ref = np.empty_like(out)
    orc.lib().or_dequant_q4t(_p(tiles), rows * gpr * 32, _p(ref))
    assert np.array_equal(out, ref)


# ------------------------------------------------------------ matvecs ----
def _tensors():
    from cmf_amd import synth
    return [synth.q8_uniform(5, 37, 320), synth.q4t_uniform(6, 40, 256), synth.q4tp_uniform(7, 24, 384),
            synth.q8_normal(8, 16, 96), synth.q4t_normal(9, 20, 160)]


@pytest.mark.parametrize("i", range(5))
def test_exact_matmat_bruteforce(i):
    """qtensor.rs:10702-10733: |y - f64 dot| <= 1e-5 * sum|w x|"""
    from cmf_amd import synth
    t = _tensors()[i]
    W = _dequant(t).astype(np.float64)
    xs = synth.normal(100 + i, 3 * t["cols"]).reshape(3, t["cols"])
    y = orc.matmat(t, xs, threads=2)
    ref = xs.astype(np.float64) @ W.T
    bound = 1e-5 * (np.abs(xs.astype(np.float64)) @ np.abs(W).T)
    assert np.all(np.abs(y - ref) <= bound + 1e-30)


@pytest.mark.parametrize("i", range(3))
def test_a8w8_matvec_bound(i):
    """qtensor.rs:10446-10481: a8w8 within rel-L2 0.05 of the exact result"""
    from cmf_amd import synth
    t = _tensors()[i]
    x = synth.normal(200 + i, t["cols"])
    ex = orc.matmat(t, x, threads=2)[0]
    a8 = orc.matmat(t, x, threads=2, a8w8=True)[0]
    assert np.linalg.norm(a8 - ex) / np.linalg.norm(ex) < 0.05


def test_split_act_reconstructs():
    """split_act: x = sx * xq except the outliers, which are kept exactly"""
    from cmf_amd import synth
    n = 512
    x = synth.normal(9, n)
    x[[3, 100, 411]] = [40.0, -55.0, 33.0]  # beyond 8 * rms: outliers
    xq = np.empty(n, dtype=np.int8)
    sx = np.zeros(1, dtype=np.float32)
    oi = np.empty(n, dtype=np.int32)
    ov = np.empty(n, dtype=np.float32)
    xsum = np.zeros(1, dtype=np.int32)
    no = orc.lib().or_split_act(_p(x), n, _p(xq), _p(sx), _p(oi), _p(ov), _p(xsum))
    assert sorted(oi[:no].tolist()) == [3, 100, 411]
    assert np.array_equal(np.sort(ov[:no]), np.sort(x[[3, 100, 411]]))
    inl = np.ones(n, bool)
    inl[oi[:no]] = False
    assert np.all(xq[~inl] == 0)
    assert np.max(np.abs(xq[inl].astype(np.float32) * sx[0] - x[inl])) <= 0.5 * sx[0] * (1 + 1e-6)
    assert xsum[0] == int(xq.astype(np.int64).sum())
