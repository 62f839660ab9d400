"""GPU parity of the a8w8 mode (cmf_matmat_a8w8) against the oracle's a8w8
arm (split_act + integer tile dots + exact outliers, qtensor.rs:9237-9281,
8921-8933, 4106-4130, 4405-4413, 4517-4544, 4666-4671).  The integer tile
dots are exact on both sides, so only the f32 order of the tile sums
differs: tolerance relative L2 1e-5 per row, far below what a dropped or
misplaced outlier term (|x| > 8 rms) would cost."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _xs(seed, b, cols, outliers):
    from cmf_amd import synth
    xs = synth.normal(seed, b * cols).reshape(b, cols).copy()
    if outliers:
        rng = np.random.default_rng(seed)
        for i in range(b):
            n = 1 + i % 4
            idx = rng.choice(cols, n, replace=False)
            xs[i, idx] = rng.choice([-1.0, 1.0], n) * (40.0 + 10.0 * rng.random(n))
    return xs


def _tensor(fmt, rows, cols, seed):
    from cmf_amd import synth
    if fmt == "q8":
        return synth.q8_uniform(seed, rows, cols)
    if fmt == "q4t":
        return synth.q4t_uniform(seed, rows, cols)
    return synth.q4tp_uniform(seed, rows, cols)


def _check(gpu, t, xs):
    w = gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
    got = gpu.matmul_a8w8(w, xs)
    ref = orc.matmat(t, xs, threads=16, a8w8=True)
    errs = [rel_l2(got[i], ref[i]) for i in range(xs.shape[0])]
    print(f"a8w8 dtype {t['dtype']} {t['rows']}x{t['cols']} b={xs.shape[0]}: max row rel-L2 {max(errs):.3e}",
          flush=True)
    assert max(errs) < TOL
    w.free()


@pytest.mark.parametrize("fmt,rows,cols", [("q8", 4096, 4096), ("q4t", 12288, 4096), ("q4tp", 4096, 12288)])
@pytest.mark.parametrize("b", [1, 5])
@pytest.mark.parametrize("outliers", [False, True])
def test_a8w8_configs(gpu, fmt, rows, cols, b, outliers):
    _check(gpu, _tensor(fmt, rows, cols, 300 + b), _xs(31 + b, b, cols, outliers))


@pytest.mark.parametrize("fmt,rows,cols", [("q8", 777, 1000), ("q4t", 1000, 480), ("q4tp", 333, 224)])
def test_a8w8_ragged_and_split_batches(gpu, fmt, rows, cols):
    """rows / cols off the 16-row and 64/128-column blocks; b = 17 runs as
    two launches of the 16-row operand"""
    _check(gpu, _tensor(fmt, rows, cols, 7), _xs(8, 17, cols, True))


def test_a8w8_outliers_change_result(gpu):
    """the outlier terms are live: zeroing the planted outliers changes the
    result by far more than the tolerance"""
    t = _tensor("q4t", 1024, 2048, 5)
    xs = _xs(6, 2, 2048, True)
    w = gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
    a = gpu.matmul_a8w8(w, xs)
    xz = xs.copy()
    xz[np.abs(xz) > 30.0] = 0.0
    z = gpu.matmul_a8w8(w, xz)
    assert rel_l2(a, z) > 100 * TOL
    w.free()
