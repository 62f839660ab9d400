"""cmf_gemv_dev_noalloc: the GEMV on device pointers whose operand workspace
is the library's static device array (no allocation in the call).  Its
output equals cmf_prep_dev + cmf_gemv_prepared with a caller workspace
(the same kernels: bit-equal) and the oracle's exact contract (relative L2
1e-3), on two calls in a row, the second with a smaller input; a weight
whose operand exceeds the workspace is rejected with an error."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _gemv_prepared(gpu, w, dx, ldx, b, rows):
    import ctypes as C
    L = gpu.lib()
    pl = gpu.DevBuf(L.cmf_prep_bytes(w.h))
    xs = gpu.DevBuf(64 * 4)
    dy = gpu.DevBuf(b * rows * 4)
    gpu.check(L.cmf_prep_dev(w.h, dx.p, ldx, b, pl.p, xs.p))
    gpu.check(L.cmf_gemv_prepared(w.h, pl.p, xs.p, b, dy.p, rows, 0))
    gpu.check(L.cmf_sync())
    y = dy.download((b, rows))
    for d in (pl, xs, dy):
        d.free()
    return y


def _noalloc(gpu, w, dx, ldx, b, rows):
    L = gpu.lib()
    dy = gpu.DevBuf(b * rows * 4)
    gpu.check(L.cmf_gemv_dev_noalloc(w.h, dx.p, ldx, b, dy.p, rows))
    gpu.check(L.cmf_sync())
    y = dy.download((b, rows))
    dy.free()
    return y


def _weights():
    from cmf_amd import synth
    return [synth.q8_normal(71, 1024, 2048, 0.05), synth.q4t_normal(72, 3072, 1024, 0.05),
            synth.q4tp_uniform(73, 512, 4096), synth.q4t_uniform(74, 4096, 12288)]


@pytest.mark.parametrize("wi", [0, 1, 2, 3])
def test_noalloc_equals_workspace_entry(gpu, wi):
    from cmf_amd import synth
    t = _weights()[wi]
    w = gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
    rows, cols = t["rows"], t["cols"]
    # first call: 9 rows; second: 3 rows of another input (smaller), ldx > cols
    for b, seed, ldx in ((9, 81, cols), (3, 82, cols + 64)):
        x = np.zeros((b, ldx), np.float32)
        x[:, :cols] = synth.normal(seed, b * cols).reshape(b, cols)
        dx = gpu.DevBuf(x.nbytes)
        dx.upload(x)
        got = _noalloc(gpu, w, dx, ldx, b, rows)
        want = _gemv_prepared(gpu, w, dx, ldx, b, rows)
        ref = orc.matmat(t, x[:, :cols], threads=16)
        print(f"dtype {t['dtype']} {rows}x{cols} b={b}: equal to the workspace entry "
              f"{np.array_equal(got, want)}, rel-L2 vs oracle {rel_l2(got, ref):.2e}", flush=True)
        assert np.array_equal(got, want)
        assert rel_l2(got, ref) < 1e-3
        dx.free()
    w.free()


def test_noalloc_rejects_oversized_operand(gpu):
    from cmf_amd import synth
    t = synth.q4t_uniform(75, 16, 32768)
    w = gpu.Weight(t["dtype"], 16, 32768, payload=t["bytes"])
    dx = gpu.DevBuf(32768 * 4)
    dy = gpu.DevBuf(16 * 4)
    rc = gpu.lib().cmf_gemv_dev_noalloc(w.h, dx.p, 32768, 1, dy.p, 16)
    msg = gpu.lib().cmf_last_error().decode()
    print("rc", rc, msg, flush=True)
    assert rc < 0 and "workspace" in msg
    for d in (dx, dy):
        d.free()
    w.free()
