"""Prefill on the large-batch MFMA GEMMs (prefill_batch, pipeline.rs:5100-5108):
chunks of up to 2048 positions (CMF_PREFILL_CHUNK), each weight read once per
chunk by the q8 (attention, eh_proj) and q4t (FFN) GEMMs with the RMSNorm /
SwiGLU / MTP-concat operand producers, residual adds in the GEMM epilogue.
The trunk KV of every layer, the MTP KV of the (h_p, id_{p+1}) warm pairs and
the tip hidden equal the oracle's per-position forwards within relative L2
1e-4, in one chunk and (child processes with smaller chunks) over two and
three chunks (256 + 256 + 88 rows)."""
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


CFG4 = dict(n_layers=2, hidden=1024, n_heads=16, n_kv=8, head_dim=128, inter=3072, vocab=4096,
            max_seq=2304, rope_theta=1e6, eps=1e-6)


def test_prefill_config4_block_shape_equals_oracle(gpu):
    """BASELINE config 4's block shape (hidden 1024, 16 query / 8 KV heads of
    128, FFN 3072) at its 2048-position context: one 2048-row chunk on the
    GEMMs and the tiled prefill attention with one KV head per XCD, the
    same kernels config 4 runs.  The KV of both layers, the MTP KV of the
    warm pairs and the tip equal the oracle's per-position forwards; every
    chunk's rows and every KV head are checked on their own, and greedy
    K = 4 rounds continue from the prefilled state (the XCD-partitioned
    decode blocks) with the oracle's tokens.  The tip is also measured
    against an f64 numpy forward of the 2048 positions: the GPU must be as
    close to it as the f32 oracle is (both sum 2048-long attention rows in
    f32, in different orders)."""
    import time
    from cmf_amd import synth
    from cmf_amd.model import Model
    from test_oracle_model import _np_forward
    sm = synth.synth_model(CFG4, seed=24, norm_noise=0.1, sigma=0.02)
    g = Model(sm)
    n = 2048
    prompt = synth.ids(25, n, CFG4["vocab"])
    g.prefill(prompt)
    pos, tip = g.state()
    assert pos == n
    t1 = time.perf_counter()
    o = orc.OracleModel(sm, threads=16)
    otip = o.prefill(prompt)
    t2 = time.perf_counter()
    ftip = _np_forward(sm, prompt)[-1]
    print(f"oracle {t2 - t1:.1f} s, f64 {time.perf_counter() - t2:.1f} s; tip: gpu-oracle {rel_l2(tip, otip):.2e}, "
          f"gpu-f64 {rel_l2(tip, ftip):.2e}, oracle-f64 {rel_l2(otip, ftip):.2e}", flush=True)
    errs = []
    for li in list(range(CFG4["n_layers"])) + [-1]:
        rows = n if li >= 0 else n - 1
        k, v = g.kv_export(li, rows)
        rk, rv = o.kv(li)
        ek, ev = rel_l2(k, rk), rel_l2(v, rv)
        worst = 0.0
        for c0 in range(0, rows, 256):
            c1 = min(rows, c0 + 256)
            worst = max(worst, rel_l2(k[:, c0:c1], rk[:, c0:c1]), rel_l2(v[:, c0:c1], rv[:, c0:c1]))
        # each KV head on its own (one per XCD in the prefill attention)
        heads = max(max(rel_l2(k[h], rk[h]), rel_l2(v[h], rv[h])) for h in range(CFG4["n_kv"]))
        print(f"layer {li}: K rel {ek:.2e} V rel {ev:.2e}; worst chunk {worst:.2e}, worst head {heads:.2e}",
              flush=True)
        errs.append(max(ek, ev, worst, heads))
    assert max(errs) < 1e-4
    assert rel_l2(tip, ftip) < 2.0 * rel_l2(otip, ftip) + 1e-5
    assert rel_l2(tip, otip) < 3e-4
    assert gpu.lib().cmf_model_fused_blocks(g.h) == 1  # the config-4 decode blocks
    gt, _ = g.decode(10, spec=True, k=4)
    ot, _ = o.decode(otip, n, prompt, 10, spec=True, k=4)
    assert gt.tolist() == ot.tolist()
    g.free()


_PLACEMENT_CHILD = r"""
import sys, json
sys.path.insert(0, sys.argv[1])
import numpy as np
import cmf_amd
from cmf_amd import synth
from cmf_amd.model import Model
from oracle import oracle as orc
cmf_amd.init(0)
cfg = dict(n_layers=1, hidden=256, n_heads=16, n_kv=8, head_dim=128, inter=512, vocab=2048, max_seq=320,
           rope_theta=1e6, eps=1e-6)
sm = synth.synth_model(cfg, seed=27, norm_noise=0.1, sigma=0.05)
g = Model(sm)
prompt = synth.ids(28, 300, cfg["vocab"])
g.prefill(prompt)
o = orc.OracleModel(sm, threads=8)
otip = o.prefill(prompt)
_, tip = g.state()
k, v = g.kv_export(0, 300)
rk, rv = o.kv(0)
rel = lambda a, b: float(np.linalg.norm(a - b) / np.linalg.norm(b))
print(json.dumps({"xcd": cmf_amd.lib().cmf_model_prefill_xcd(g.h), "tip": rel(tip, otip), "k": rel(k, rk),
                  "v": rel(v, rv)}))
"""


@pytest.mark.parametrize("forced", [False, True])
def test_prefill_placement_check_falls_back(gpu, forced):
    """The XCD-placed prefill attention (8 kv heads) checks that every
    (query block, kv head) was served once; a failed check (forced from the
    host here: CMF_PREFILL_PLACEMENT_FAIL=1) re-runs the prefill on the
    grid-indexed variant, whose results equal the oracle's as well"""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, CMF_PREFILL_PLACEMENT_FAIL="1" if forced else "0")
    r = subprocess.run([sys.executable, "-c", _PLACEMENT_CHILD, root], env=env, capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["xcd"] == (0 if forced else 1)
    assert res["tip"] < 1e-4 and res["k"] < 1e-4 and res["v"] < 1e-4


_CHUNK_CHILD = r"""
import sys, json
sys.path.insert(0, sys.argv[1])
import numpy as np
import cmf_amd
from cmf_amd import synth
from cmf_amd.model import Model
from oracle import oracle as orc
cmf_amd.init(0)
cfg = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096, max_seq=640,
           rope_theta=1e6, eps=1e-6)
sm = synth.synth_model(cfg, seed=21, norm_noise=0.1, sigma=0.05)
g = Model(sm)
prompt = synth.ids(22, 600, cfg["vocab"])
g.prefill(prompt)
o = orc.OracleModel(sm, threads=8)
otip = o.prefill(prompt)
_, tip = g.state()
rel = lambda a, b: float(np.linalg.norm(a - b) / np.linalg.norm(b))
out = {"tip": rel(tip, otip)}
for li in (0, 1, -1):
    k, v = g.kv_export(li, 600 if li >= 0 else 599)
    rk, rv = o.kv(li)
    out[f"k{li}"], out[f"v{li}"] = rel(k, rk), rel(v, rv)
    out[f"klast{li}"] = rel(k[:, 512:], rk[:, 512:])
gt, _ = g.decode(6, spec=True, k=4)
ot, _ = o.decode(otip, 600, prompt, 6, spec=True, k=4)
out["tokens_equal"] = gt.tolist() == ot.tolist()
print(json.dumps(out))
"""


@pytest.mark.parametrize("chunk", [256, 512])
def test_prefill_multi_chunk(gpu, chunk):
    """The 600-position prefill in chunks of 256 (three: 256 + 256 + 88) and
    512 (two): the chunk boundaries (positions, the causal attention over the
    cached rows, the MTP warm pair across a boundary) give the oracle's KV,
    tip and decode tokens (a child process: the chunk size is read once per
    process)"""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, CMF_PREFILL_CHUNK=str(chunk))
    r = subprocess.run([sys.executable, "-c", _CHUNK_CHILD, root], env=env, capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res.pop("tokens_equal")
    assert max(res.values()) < 1e-4, res
