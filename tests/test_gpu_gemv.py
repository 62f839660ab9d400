"""GPU parity of the dequant GEMV / skinny GEMM family against the CPU oracle
(the reference's exact contract, qtensor.rs).  Tolerance: relative L2 1e-3
(BASELINE north star); observed errors are ~1e-6."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _x(seed, b, cols):
    from cmf_amd import synth
    return synth.normal(seed, b * cols).reshape(b, cols)


def _check(gpu, t, xs, tol=TOL):
    w = gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
    got = gpu.matmul(w, xs)
    ref = orc.matmat(t, xs, threads=16)
    err = rel_l2(got, ref)
    print(f"dtype {t['dtype']} {t['rows']}x{t['cols']} b={xs.shape[0]}: rel-L2 {err:.3e}", flush=True)
    assert err < tol
    # every row and batch element individually
    for i in range(xs.shape[0]):
        assert rel_l2(got[i], ref[i]) < tol
    return got, ref


def test_q8_config1(gpu):
    from cmf_amd import synth
    t = synth.q8_uniform(11, 4096, 4096)
    _check(gpu, t, _x(12, 1, 4096))


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 16])
def test_q8_batches(gpu, m):
    from cmf_amd import synth
    t = synth.q8_normal(21 + m, 1024, 2048)
    _check(gpu, t, _x(22 + m, m, 2048))


@pytest.mark.parametrize("shape", [(12288, 4096), (4096, 12288)])
@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_q4t_config2(gpu, shape, m):
    from cmf_amd import synth
    t = synth.q4t_uniform(31 + shape[0], shape[0], shape[1])
    _check(gpu, t, _x(32 + m, m, shape[1]))


def test_q8_config5_projection(gpu):
    """BASELINE config 5's q8 4096x2048 attention projection at M=5"""
    from cmf_amd import synth
    t = synth.q8_uniform(5003, 4096, 2048)
    _check(gpu, t, _x(5004, 5, 2048))


@pytest.mark.parametrize("shape", [(12288, 4096), (4096, 12288)])
def test_q4tp_config3(gpu, shape):
    from cmf_amd import synth
    t = synth.q4tp_uniform(41 + shape[0], shape[0], shape[1])
    _check(gpu, t, _x(42, 5, shape[1]))


@pytest.mark.parametrize("m", [1, 3, 7, 13])
def test_q4tp_batches_small(gpu, m):
    from cmf_amd import synth
    t = synth.q4tp_uniform(51 + m, 512, 1024)
    _check(gpu, t, _x(52 + m, m, 1024))


def test_ragged_shapes(gpu):
    """rows not a multiple of 16, cols not a multiple of the K step"""
    from cmf_amd import synth
    _check(gpu, synth.q8_normal(61, 37, 80), _x(62, 3, 80))
    _check(gpu, synth.q4t_uniform(63, 45, 96), _x(64, 2, 96))
    _check(gpu, synth.q4tp_uniform(65, 19, 160), _x(66, 4, 160))
    _check(gpu, synth.q4t_uniform(67, 1, 32), _x(68, 1, 32))


def test_large_batch_split(gpu):
    """q8 with b > 16 is served as GEMV launches of 16"""
    from cmf_amd import synth
    _check(gpu, synth.q8_normal(71, 256, 512), _x(72, 37, 512))


@pytest.mark.parametrize("b", [17, 64, 130])
@pytest.mark.parametrize("fmt", ["q4t", "q4tp"])
def test_gemm_large_batch(gpu, fmt, b):
    """q4 with b > 16: the MFMA GEMM (ragged batch tiles and row blocks)"""
    from cmf_amd import synth
    mk = synth.q4t_uniform if fmt == "q4t" else synth.q4tp_uniform
    _check(gpu, mk(73 + b, 272, 640), _x(74 + b, b, 640))


@pytest.mark.parametrize("shape", [(12288, 4096), (4096, 12288)])
def test_gemm_config2_prefill(gpu, shape):
    """config 2 shapes at a prefill-sized batch (256 rows)"""
    from cmf_amd import synth
    _check(gpu, synth.q4t_uniform(75, *shape), _x(76, 256, shape[1]))


def test_q8_matvec_range(gpu):
    from cmf_amd import synth
    t = synth.q8_normal(81, 300, 256)
    w = gpu.Weight(t["dtype"], 300, 256, q=t["q"], row_scale=t["row_scale"])
    x = _x(82, 1, 256)
    out = np.zeros((1, 37), np.float32)
    assert gpu.q8_matvec_range(w, 5, x, 37, 256, out)
    ref = orc.matmat(t, x)[:, 5:42]
    assert rel_l2(out, ref) < TOL


def test_seam_declines_other_codec(gpu):
    from cmf_amd import synth
    t = synth.q4t_uniform(91, 64, 64)
    w = gpu.Weight(t["dtype"], 64, 64, payload=t["bytes"])
    out = np.zeros((1, 64), np.float32)
    assert gpu.q8_matmat(w, _x(92, 1, 64), 1, 64, 64, out) is False
    assert gpu.q4tp_matvec(w, _x(92, 1, 64), 64, 64, out) is False
    assert gpu.q4t_matvec(w, _x(92, 1, 64), 64, 64, out) is True


def test_q4tp_step0_equals_q4t(gpu):
    """A q4tp tensor whose ladder is flat (step 0) and a q4t tensor with the
    same nibbles and scale 2^lo give identical products."""
    from cmf_amd import synth
    rows, cols = 64, 256
    tp = synth.q4tp_uniform(101, rows, cols)
    gpr = cols // 32
    b = tp["bytes"].copy()
    params = b[rows * gpr * 16: rows * gpr * 16 + rows * 4].view(np.uint16).reshape(rows, 2)
    params[:, 1] = 0  # step = 0 -> every rung equals 2^lo
    q4t = np.empty(rows * gpr * 18, np.uint8).reshape(rows, gpr, 18)
    lo = params[:, 0].view(np.float16).astype(np.float32)
    s16 = np.exp2(lo).astype(np.float16)
    q4t[:, :, 0:2] = np.repeat(s16.view(np.uint8).reshape(rows, 1, 2), gpr, axis=1)
    q4t[:, :, 2:] = b[: rows * gpr * 16].reshape(rows, gpr, 16)
    ttp = dict(tp, bytes=b)
    tt = synth.tensor(synth.DT_Q4T, rows, cols, payload=q4t.reshape(-1))
    x = _x(102, 3, cols)
    if np.all(np.exp2(lo).astype(np.float16).astype(np.float32) == np.exp2(lo).astype(np.float32)):
        a = gpu.matmul(gpu.Weight(synth.DT_Q4TP, rows, cols, payload=b), x)
        c = gpu.matmul(gpu.Weight(synth.DT_Q4T, rows, cols, payload=tt["bytes"]), x)
        assert rel_l2(a, c) < 1e-6
    else:
        a = gpu.matmul(gpu.Weight(synth.DT_Q4TP, rows, cols, payload=b), x)
        assert rel_l2(a, orc.matmat(ttp, x)) < TOL


def test_ffn(gpu):
    """gpu.rs:1773 q4t_ffn: down(silu(gate x) * up x)"""
    from cmf_amd import synth
    H, I = 256, 512
    g, u, d = synth.q4t_normal(111, I, H), synth.q4t_normal(112, I, H), synth.q4t_normal(113, H, I)
    x = _x(114, 3, H)
    W = lambda t: gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"])
    out = np.zeros((3, H), np.float32)
    assert gpu.ffn(W(g), W(u), W(d), x, 3, H, I, out)
    gg, uu = orc.matmat(g, x), orc.matmat(u, x)
    act = (gg / (1 + np.exp(-gg))) * uu
    ref = orc.matmat(d, act.astype(np.float32))
    assert rel_l2(out, ref) < TOL
