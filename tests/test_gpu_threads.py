"""Seam ops called from several host threads at once.  Each thread runs on
its own HIP stream with its own seam and GEMM scratch (the reference's GPU
gate is thread-local, gpu.rs:18-46, 978-1000), so concurrent matvecs, GEMMs
(b > 16) and FFNs of different threads neither race nor see each other's
operands: every result equals the one computed alone and the oracle's."""
import threading

import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def test_concurrent_seam_calls(gpu):
    from cmf_amd import synth
    n_threads, iters = 4, 12
    work = []
    for i in range(n_threads):
        t = synth.q4t_uniform(300 + i, 1024 + 64 * i, 512) if i % 2 == 0 else synth.q8_normal(300 + i, 768, 1024)
        w = gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
        b = (1, 5, 33)[i % 3]  # 33 > 16: the MFMA GEMM and its per-thread scratch
        x = synth.normal(400 + i, b * t["cols"]).reshape(b, t["cols"])
        ref = orc.matmat(t, x, threads=8)
        work.append((w, x, ref, gpu.matmul(w, x)))
    H, I = 256, 512
    ffn_w = [synth.q4t_uniform(500 + j, *s) for j, s in enumerate([(I, H), (I, H), (H, I)])]
    fw = [gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"]) for t in ffn_w]
    fx = synth.normal(510, 3 * H).reshape(3, H)
    f_alone = np.empty((3, H), np.float32)
    assert gpu.ffn(*fw, fx, 3, H, I, f_alone)
    errors = []

    def run(i):
        try:
            w, x, ref, alone = work[i]
            for _ in range(iters):
                got = gpu.matmul(w, x)
                if not np.array_equal(got, alone) or rel_l2(got, ref) > 1e-3:
                    errors.append(f"thread {i}: differs (rel {rel_l2(got, ref):.2e})")
                    return
                out = np.empty((3, H), np.float32)
                gpu.ffn(*fw, fx, 3, H, I, out)
                if not np.array_equal(out, f_alone):
                    errors.append(f"thread {i}: ffn differs")
                    return
        except Exception as e:  # noqa: BLE001
            errors.append(f"thread {i}: {e!r}")

    ths = [threading.Thread(target=run, args=(i,)) for i in range(n_threads)]
    for t in ths:
        t.start()
    for t in ths:
        t.join(timeout=120)
    print(errors, flush=True)
    assert not errors
    for w, *_ in work:
        w.free()
    for w in fw:
        w.free()
