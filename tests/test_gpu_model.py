"""GPU parity of the decode engine (verify forward, speculative decode)
against the CPU oracle's restatement of the reference pipeline."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096,
             max_seq=256, rope_theta=1e6, eps=1e-6)


@pytest.fixture(scope="module")
def small(gpu):
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = synth.synth_model(SMALL, seed=5, norm_noise=0.1, sigma=0.05)
    return sm, Model(sm)


def test_forward_batch_matches_oracle(small):
    sm, g = small
    from cmf_amd import synth
    ids = synth.ids(7, 12, SMALL["vocab"])
    hid, lg = g.forward_batch(ids, 0)
    o = orc.OracleModel(sm)
    for i, t in enumerate(ids):
        h = o.forward(int(t), i)
        print(f"row {i}: hidden rel {rel_l2(hid[i], h):.2e}", flush=True)
        assert rel_l2(hid[i], h) < 1e-4
        ol = o.logits(h)
        assert rel_l2(lg[i], ol) < 1e-4
        assert int(np.argmax(lg[i])) == int(np.argmax(ol))


def test_verify_block_is_causal(small):
    """a batch of b rows equals b single-row forwards (causal mask inside the
    verify block, KV appended for every row)"""
    sm, g = small
    from cmf_amd import synth
    ids = synth.ids(9, 6, SMALL["vocab"])
    hb, lb = g.forward_batch(ids, 0)
    rows = []
    for i, t in enumerate(ids):
        h1, l1 = g.forward_batch(ids[i:i + 1], i)
        rows.append(h1[0])
    assert rel_l2(np.stack(rows), hb) < 1e-5


@pytest.mark.parametrize("b", [1, 3, 5])
def test_small_batches_match_oracle(small, b):
    """verify-sized batches (1 + K rows) against the oracle, row by row"""
    sm, g = small
    from cmf_amd import synth
    ids = synth.ids(11, b, SMALL["vocab"])
    hid, lg = g.forward_batch(ids, 0)
    o = orc.OracleModel(sm)
    for i, t in enumerate(ids):
        h = o.forward(int(t), i)
        e = rel_l2(hid[i], h)
        print(f"b={b} row {i}: hidden rel {e:.2e}", flush=True)
        assert e < 1e-4
        assert rel_l2(lg[i], o.logits(h)) < 1e-4


def _gen_pair(sm, g, prompt, n, spec, k, sampler_gpu=None, sampler_or=None, seed=0):
    g.prefill(prompt)
    gt, gst = g.decode(n, sampler=sampler_gpu, seed=seed, spec=spec, k=k)
    o = orc.OracleModel(sm)
    ot, ost = o.generate(prompt, n, spec=spec, k=k, sampler=sampler_or, seed=seed)
    return gt, gst, ot, ost


@pytest.mark.parametrize("k", [1, 4])
def test_greedy_spec_tokens_equal_oracle(small, k):
    sm, g = small
    from cmf_amd import synth
    prompt = synth.ids(13, 20, SMALL["vocab"])
    gt, gst, ot, ost = _gen_pair(sm, g, prompt, 24, True, k)
    print("gpu", gt.tolist(), "acc", gst.accepted, "rounds", gst.rounds, flush=True)
    print("cpu", ot.tolist(), "acc", ost.accepted, flush=True)
    n = min(len(gt), len(ot))
    assert n >= 24
    assert gt[:n].tolist() == ot[:n].tolist()
    assert gst.accepted == ost.accepted


def test_greedy_spec_equals_vanilla(small):
    """pipeline.rs:11543 speculative_equals_vanilla_greedy, on the GPU"""
    sm, g = small
    from cmf_amd import synth
    prompt = synth.ids(17, 16, SMALL["vocab"])
    g.prefill(prompt)
    a, _ = g.decode(30, spec=True, k=4)
    g.prefill(prompt)
    b, _ = g.decode(30, spec=False)
    assert a[:30].tolist() == b[:30].tolist()


def test_sampling_spec_tokens_equal_oracle(small):
    """temperature 0.8 with the default chain (top_k 40, top_p 0.9, min_p
    0.05), repetition penalty 1: same seeded uniforms -> same tokens"""
    sm, g = small
    import cmf_amd
    from cmf_amd import synth
    prompt = synth.ids(19, 20, SMALL["vocab"])
    sg = cmf_amd.SamplerConfig(temperature=0.8, repetition_penalty=1.0)
    so = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0)
    gt, gst, ot, ost = _gen_pair(sm, g, prompt, 24, True, 4, sg, so, seed=1234)
    print("gpu", gt.tolist(), gst.accepted, flush=True)
    print("cpu", ot.tolist(), ost.accepted, flush=True)
    n = min(len(gt), len(ot))
    assert gt[:n].tolist() == ot[:n].tolist()


@pytest.mark.parametrize("sampling", [False, True])
def test_captured_rounds_equal_eager_and_oracle(small, sampling, monkeypatch):
    """decode_rounds(n > 1) replays one captured round n - 1 times; two such
    calls in a row (the second replaying the graph kept from the first, with a
    host state read in between) give the eagerly launched tokens and the
    oracle's"""
    sm, g = small
    import cmf_amd
    from cmf_amd import synth
    from cmf_amd.model import Model
    prompt = synth.ids(23, 18, SMALL["vocab"])
    sg = cmf_amd.SamplerConfig(temperature=0.8, repetition_penalty=1.0) if sampling else None
    so = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0) if sampling else None
    monkeypatch.setenv("CMF_DECODE_GRAPH", "0")
    eager = Model(sm)
    runs = []
    for m in (g, eager):
        m.prefill(prompt)
        m.decode_begin(sampler=sg, seed=77)
        m.decode_rounds(5, spec=True, k=3)
        st = m.state()
        m.decode_rounds(4, spec=True, k=3)
        runs.append(m.tokens())
        print("graph" if m is g else "eager", runs[-1].tolist(), "pos", st[0], flush=True)
    eager.free()
    assert runs[0].tolist() == runs[1].tolist()
    o = orc.OracleModel(sm)
    ot, _ = o.generate(prompt, len(runs[0]) + 8, spec=True, k=3, sampler=so, seed=77)
    assert runs[0].tolist() == ot[:len(runs[0])].tolist()
