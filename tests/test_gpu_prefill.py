"""Prefill on the large-batch MFMA GEMMs (prefill_batch, pipeline.rs:5100-5108):
256-position chunks, each weight read once per chunk by the q8 (attention,
eh_proj) and q4t (FFN) GEMMs with the RMSNorm / SwiGLU / MTP-concat operand
producers, residual adds in the GEMM epilogue.  The trunk KV of every layer,
the MTP KV of the (h_p, id_{p+1}) warm pairs and the tip hidden equal the
oracle's per-position forwards within relative L2 1e-4, over three chunks
(256 + 256 + 88 rows)."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096,
           max_seq=640, rope_theta=1e6, eps=1e-6)


def test_prefill_chunks_equal_oracle(gpu):
    import time
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = synth.synth_model(CFG, seed=21, norm_noise=0.1, sigma=0.05)
    g = Model(sm)
    prompt = synth.ids(22, 600, CFG["vocab"])
    t0 = time.perf_counter()
    g.prefill(prompt)
    dt = time.perf_counter() - t0
    pos, tip = g.state()
    assert pos == 600
    o = orc.OracleModel(sm)
    otip = o.prefill(prompt)
    print(f"prefill 600 positions: {dt * 1e3:.1f} ms (first call, includes buffer setup); "
          f"tip rel {rel_l2(tip, otip):.2e}", flush=True)
    assert rel_l2(tip, otip) < 1e-4
    for li in list(range(CFG["n_layers"])) + [-1]:
        n = 600 if li >= 0 else 599
        k, v = g.kv_export(li, n)
        rk, rv = o.kv(li)
        ek, ev = rel_l2(k, rk), rel_l2(v, rv)
        # and the rows of the last chunk on their own
        ek2 = rel_l2(k[:, 512:], rk[:, 512:])
        print(f"layer {li}: K rel {ek:.2e} V rel {ev:.2e} (last chunk K {ek2:.2e})", flush=True)
        assert ek < 1e-4 and ev < 1e-4 and ek2 < 1e-4
    # the decode continues on the prefilled state like the oracle
    gt, _ = g.decode(6, spec=True, k=4)
    ot, _ = o.decode(otip, 600, prompt, 6, spec=True, k=4)
    assert gt.tolist() == ot.tolist()
    g.free()
