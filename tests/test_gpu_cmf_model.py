"""A model read from a .cmf file (cmf_amd.loader over the native container
reader) runs on the GPU exactly as the same weights handed over in memory,
and its tokens equal the CPU oracle's (tied and untied embedding tables,
f16 and bf16 norms, q8 / q4t / q4tp matrices)."""
import numpy as np
import pytest

import cmf_writer as W
from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096,
             max_seq=256, rope_theta=1e6, eps=1e-6)


def _model(seed, untied=False):
    from cmf_amd import synth
    sm = synth.synth_model(SMALL, seed=seed, norm_noise=0.1, sigma=0.05)
    if untied:
        sm["embed"] = synth.q8_normal(seed + 100, SMALL["vocab"], SMALL["hidden"], 0.05)
        sm["layers"][1]["down"] = synth.q4tp_uniform(seed + 101, SMALL["hidden"], SMALL["inter"], sigma=0.002)
    return W.f16_model(sm)


@pytest.mark.parametrize("untied", [False, True])
def test_file_model_equals_memory_model_and_oracle(gpu, tmp_path, untied):
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = _model(11 + untied, untied)
    p = tmp_path / "m.cmf"
    W.write_model(p, sm)
    print(f"untied={untied}: {p.stat().st_size} bytes", flush=True)
    gf = Model.from_cmf(str(p))
    gm = Model(sm)
    ids = synth.ids(17, 10, SMALL["vocab"])
    hf, lf = gf.forward_batch(ids, 0)
    hm, lm = gm.forward_batch(ids, 0)
    assert np.array_equal(hf, hm) and np.array_equal(lf, lm)  # same weights, same kernels
    o = orc.OracleModel(sm)
    for i, t in enumerate(ids):
        h = o.forward(int(t), i)
        assert rel_l2(hf[i], h) < 1e-4
        assert int(np.argmax(lf[i])) == int(np.argmax(o.logits(h)))
    gf.free()
    gm.free()


def test_file_model_greedy_spec_tokens_equal_oracle(gpu, tmp_path):
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = _model(13)
    p = tmp_path / "g.cmf"
    W.write_model(p, sm, norm_dtype=2)  # bf16 norms in the file
    g = Model.from_cmf(str(p))
    from cmf_amd import loader
    sm_file = loader.load(str(p))  # the weights as the file holds them (bf16-rounded norms)
    prompt = synth.ids(19, 16, SMALL["vocab"])
    g.prefill(prompt)
    gt, gst = g.decode(20, spec=True, k=4)
    ot, ost = orc.OracleModel(sm_file).generate(prompt, 20, spec=True, k=4)
    n = min(len(gt), len(ot))
    print("gpu", gt[:n].tolist(), "cpu", ot[:n].tolist(), flush=True)
    assert n >= 20 and gt[:n].tolist() == ot[:n].tolist()
    g.free()


def test_file_moe_model_equals_memory_model_and_oracle(gpu, tmp_path):
    """a Qwen3-MoE file (f16 router, q4t experts) through the loader: the
    same hidden rows as the in-memory model, tokens equal to the oracle's"""
    from cmf_amd import synth
    from cmf_amd.model import Model
    moe = dict(n_experts=8, top_k=2, inter=128, layers=[0], router_dtype="f16")
    sm = W.f16_model(synth.synth_model(SMALL, seed=15, norm_noise=0.3, sigma=0.08, moe=moe))
    p = tmp_path / "moe.cmf"
    W.write_model(p, sm)
    gf = Model.from_cmf(str(p))
    gm = Model(sm)
    ids = synth.ids(18, 8, SMALL["vocab"])
    hf, _ = gf.forward_batch(ids, 0)
    hm, _ = gm.forward_batch(ids, 0)
    assert np.array_equal(hf, hm)
    prompt = synth.ids(20, 16, SMALL["vocab"])
    gf.prefill(prompt)
    gt, _ = gf.decode(12, spec=True, k=4)
    ot, _ = orc.OracleModel(sm).generate(prompt, 12, spec=True, k=4)
    print("gpu", gt.tolist(), "cpu", ot.tolist(), flush=True)
    assert gt.tolist() == ot.tolist()
    gf.free()
    gm.free()
