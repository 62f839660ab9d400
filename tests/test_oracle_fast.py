"""CPU pins of the oracle's a8w8 batch arm and of its AVX-512 VNNI timing arm
(oracle/fast.c, the reference's x86 kernels qtensor.rs:4204-4228,
4312-4361, 4616-4641, 8921-8990).

- The VNNI arm returns the scalar a8w8 arm's values bit for bit, for every
  format, batch size (the four-input q4t blocks and the remainder rows),
  ragged q8 widths (the 64-byte tail) and activations with outliers.
- The scalar arm's four-input q4t order is pinned independently: with
  power-of-two tile scales and small activations every float step is exact,
  so both orders must equal the brute-force int64 dot; with random data both
  orders stay within f32 rounding of the f64 dot of the same integers.
- The batched verify forward (or_forward_rows) equals per-position forwards
  bit for bit under the exact contract, and a decode through the VNNI arm
  equals the scalar a8w8 decode token for token and state for state.
"""
import numpy as np
import pytest

from oracle import oracle as orc

vnni = pytest.mark.skipif(not orc.fast_supported(), reason="host has no AVX-512 VNNI")


def _acts(seed, b, cols, outliers):
    from cmf_amd import synth
    xs = synth.normal(seed, b * cols).reshape(b, cols)
    if outliers:
        rng = np.random.default_rng(seed)
        for i in range(b):
            j = rng.choice(cols, 3, replace=False)
            xs[i, j] = rng.choice([-1, 1], 3) * 40.0
    return xs


def _tensors():
    from cmf_amd import synth
    return [("q8", synth.q8_uniform(5, 96, 4096)), ("q8 ragged", synth.q8_uniform(6, 80, 1000)),
            ("q4t", synth.q4t_uniform(7, 96, 2048)), ("q4tp", synth.q4tp_uniform(8, 64, 2048))]


@vnni
@pytest.mark.parametrize("b", [1, 3, 4, 5, 9])
@pytest.mark.parametrize("outliers", [False, True])
def test_vnni_arm_equals_scalar_arm(b, outliers):
    for name, t in _tensors():
        xs = _acts(100 + b, b, t["cols"], outliers)
        ref = orc.matmat(t, xs, threads=3, a8w8=True)
        got = orc.matmat(t, xs, threads=5, fast=True)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (name, b, outliers)


def _q4t_ints(t):
    """codes (nibble - 8) [rows][cols] and f32 tile scales [rows][gpr]"""
    rows, cols = t["rows"], t["cols"]
    gpr = cols // 32
    raw = np.asarray(t["bytes"], np.uint8).reshape(rows, gpr, 18)
    sc = raw[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    nib = raw[:, :, 2:]
    codes = np.stack([(nib & 15).astype(np.int64) - 8, (nib >> 4).astype(np.int64) - 8], axis=-1)
    return codes.reshape(rows, cols), sc


def _set_scales(t, fn):
    rows, gpr = t["rows"], t["cols"] // 32
    raw = np.asarray(t["bytes"], np.uint8).reshape(rows, gpr, 18).copy()
    s = fn(rows, gpr).astype(np.float16)
    raw[:, :, :2] = s.reshape(rows, gpr, 1).view(np.uint8)
    u = dict(t)
    u["bytes"] = raw.reshape(-1)
    return u


def test_q4t_blocked_order_exact_case():
    """power-of-two tile scales 2^-2..2^1 over 16 tiles: every partial sum is
    a multiple of 2^-2 below 2^22, so each float step of either order (the
    four-input blocks, rows 0-3, and the per-tile order, row 4) is exact and
    the result is the brute-force int64 dot times sx, rounded once"""
    from cmf_amd import synth
    t = synth.q4t_uniform(21, 40, 512)
    rng = np.random.default_rng(3)
    t = _set_scales(t, lambda r, g: 2.0 ** rng.integers(-2, 2, (r, g)))
    codes, sc = _q4t_ints(t)
    # activations that quantize to themselves: amax 1.0, sx = 1/127, xq = xi
    xi = rng.integers(-127, 128, (5, 512))
    xi[:, 0] = 127
    xs = (xi / 127.0).astype(np.float32)
    out = orc.matmat(t, xs, threads=2, a8w8=True)
    sx = np.float64(np.float32(1.0) / np.float32(127.0))
    W = codes * sc.repeat(32, axis=1).astype(np.float64)
    for i in range(5):
        ref = ((W @ xi[i].astype(np.float64)) * sx).astype(np.float32)
        assert np.array_equal(out[i], ref), i


def test_q4t_blocked_order_random_bound():
    """random data: the four-input rows (blocked order) and the fifth (per
    tile order) both within 1e-5 relative of the f64 dot of the integer
    codes and quantized activations"""
    from cmf_amd import synth
    t = synth.q4t_uniform(22, 64, 4096)
    codes, sc = _q4t_ints(t)
    xs = synth.normal(9, 5 * 4096).reshape(5, 4096)
    out = orc.matmat(t, xs, threads=2, a8w8=True)
    W = codes * sc.repeat(32, axis=1).astype(np.float64)
    for i in range(5):
        xq = np.empty(4096, np.int8)
        sx = np.empty(1, np.float32)
        oi = np.empty(4096, np.int32)
        ov = np.empty(4096, np.float32)
        xsum = np.empty(1, np.int32)
        no = orc.lib().or_split_act(orc._p(np.ascontiguousarray(xs[i])), 4096, orc._p(xq), orc._p(sx),
                                    orc._p(oi), orc._p(ov), orc._p(xsum))
        ref = (W @ xq.astype(np.float64)) * float(sx[0])
        for o in range(no):
            ref += W[:, oi[o]] * float(ov[o])
        rel = np.abs(out[i] - ref) / np.abs(ref).max()
        assert rel.max() < 1e-5, (i, rel.max())


def test_batch_forward_equals_positions_exact():
    from cmf_amd import synth
    cfg = dict(n_layers=2, hidden=128, n_heads=4, n_kv=2, head_dim=32, inter=256, vocab=512, max_seq=64,
               rope_theta=1e6, eps=1e-6)
    sm = synth.synth_model(cfg, seed=4, norm_noise=0.1, sigma=0.05)
    prompt = np.array([3, 17, 99, 4, 250, 7, 8, 12, 41, 300], np.int32)
    outs = []
    for bv in (False, True):
        o = orc.OracleModel(sm, threads=2, batch_verify=bv)
        toks, st = o.generate(prompt, 12, spec=True, k=4)
        outs.append((toks, [o.kv(li) for li in range(2)], o.kv(-1)))
    assert np.array_equal(outs[0][0], outs[1][0])
    for (ka, va), (kb, vb) in zip(outs[0][1], outs[1][1]):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    assert np.array_equal(outs[0][2][0], outs[1][2][0])


@vnni
def test_vnni_decode_equals_scalar_a8w8_decode():
    from cmf_amd import synth
    cfg = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=64, inter=512, vocab=1024, max_seq=64,
               rope_theta=1e6, eps=1e-6)
    sm = synth.synth_model(cfg, seed=5, norm_noise=0.1, sigma=0.05)
    prompt = np.array([3, 17, 99, 4, 250, 7, 8, 12], np.int32)
    res = []
    for fast in (False, True):
        o = orc.OracleModel(sm, threads=3, a8w8=True, fast=fast, batch_verify=True)
        toks, st = o.generate(prompt, 10, spec=True, k=4)
        res.append((toks, st.accepted, [o.kv(li) for li in range(2)]))
    assert np.array_equal(res[0][0], res[1][0]) and res[0][1] == res[1][1]
    for (ka, va), (kb, vb) in zip(res[0][2], res[1][2]):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
