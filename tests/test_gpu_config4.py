"""BASELINE config 4 on the GPU: the synthetic Qwen3-0.6B-arch model (28
layers, hidden 1024, 16Q/8KV x 128, FFN 3072, vocab 151936, attention q8,
FFN q4t, lm_head/embedding q8, one MTP layer) after a 2048-token prefill,
speculative decode with K=4, greedy and temperature 0.8, against the CPU
oracle decoding from the same state (the GPU's prefilled KV imported into
the oracle; the prefill itself is pinned by the smaller forward tests).
Also the device sampler's sparse distribution at the full vocabulary (38
selection slices of 4096 logits, cross-slice merge and denominator)
against the oracle's sparse_distribution_into."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CTX = 2048
N_TOK = 8


@pytest.fixture(scope="module")
def full(gpu):
    from cmf_amd import synth
    from cmf_amd.model import Model
    cfg = dict(synth.QWEN3_06B, max_seq=CTX + 64)
    sm = synth.synth_model(cfg, seed=1)
    g = Model(sm)
    prompt = synth.ids(2024, CTX, cfg["vocab"])
    o = orc.OracleModel(sm, threads=16)
    yield sm, g, o, prompt
    g.free()


def _prefill_both(sm, g, o, prompt):
    g.prefill(prompt)
    pos, hid = g.state()
    assert pos == CTX
    o.reset()
    for li in range(sm["cfg"]["n_layers"]):
        o.import_kv(li, *g.kv_export(li, CTX))
    o.import_kv(-1, *g.kv_export(-1, CTX - 1))
    return hid


@pytest.mark.parametrize("sampling", [False, True])
def test_config4_spec_decode_tokens_equal_oracle(full, sampling):
    import cmf_amd
    sm, g, o, prompt = full
    hid = _prefill_both(sm, g, o, prompt)
    sg = cmf_amd.SamplerConfig(temperature=0.8, repetition_penalty=1.0) if sampling else None
    so = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0) if sampling else None
    gt, gst = g.decode(N_TOK, sampler=sg, seed=4242, spec=True, k=4)
    ot, ost = o.decode(hid, CTX, prompt, N_TOK, spec=True, k=4, sampler=so, seed=4242)
    print(f"sampling={sampling}: gpu {gt.tolist()} acc {gst.accepted}/{gst.drafted} | "
          f"oracle {ot.tolist()} acc {ost.accepted}/{ost.drafted}", flush=True)
    assert gt.tolist() == ot.tolist()
    assert gst.accepted == ost.accepted


@pytest.mark.parametrize("seed,scale", [(1, 1.0), (2, 4.0), (3, 12.0)])
def test_sparse_distribution_full_vocab(gpu, seed, scale):
    """logits N(0, scale^2) over 151936 ids at T=0.8, top_k 40, top_p 0.9,
    min_p 0.05: ids equal, probabilities within 1e-5 relative"""
    import ctypes as C
    import cmf_amd
    from cmf_amd import synth
    from cmf_amd.model import Model
    V = 151936
    cfg = dict(n_layers=1, hidden=128, n_heads=1, n_kv=1, head_dim=128, inter=128, vocab=V, max_seq=16,
               rope_theta=1e6, eps=1e-6)
    sm = synth.synth_model(cfg, seed=9, mtp=False)
    g = Model(sm)
    sg = cmf_amd.SamplerConfig(temperature=0.8, repetition_penalty=1.0)
    so = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0)
    lg = (synth.normal(100 + seed, V) * scale).astype(np.float32)
    # the winners spread over many slices, one of them in the last (ragged) slice
    lg[V - 3] = lg.max() + 0.5
    ids, pr = g.sparse_distribution(lg, sg)
    g.free()
    oid = np.empty(4 * 256 + 64, np.uint32)
    opr = np.empty(4 * 256 + 64, np.float32)
    P = lambda a: a.ctypes.data_as(C.c_void_p)
    n = orc.lib().or_sparse_distribution(P(lg), V, C.byref(so), None, 0, P(oid), P(opr))
    print(f"seed {seed} scale {scale}: device n={len(ids)} oracle n={n}; slices "
          f"{sorted(set((ids // 4096).tolist()))}", flush=True)
    assert ids.tolist() == oid[:n].astype(np.int32).tolist()
    assert np.allclose(pr, opr[:n], rtol=1e-5, atol=1e-7)
    assert V - 3 in ids.tolist()


@pytest.mark.parametrize("levels,k,tp", [(2, 40, 1.0), (8, 40, 1.0), (8, 40, 0.9), (64, 40, 1.0), (8, 64, 0.9)])
def test_sparse_distribution_tied_logits(gpu, levels, k, tp):
    """logits on a coarse grid over 151936 ids, ties at the k-th value:
    levels 8 (about 200 ids share the top value), 64 (a few share the k-th),
    2 (tens of thousands tied: the 4 k + 64 cap, first in index order).
    par_topk keeps every entry tied with the k-th (sampler.rs:515-600), so
    the ids equal the oracle's or_sparse_distribution and the
    probabilities agree within 1e-5"""
    import ctypes as C
    import cmf_amd
    from cmf_amd import synth
    from cmf_amd.model import Model
    V = 151936
    cfg = dict(n_layers=1, hidden=128, n_heads=1, n_kv=1, head_dim=128, inter=128, vocab=V, max_seq=16,
               rope_theta=1e6, eps=1e-6)
    sm = synth.synth_model(cfg, seed=9, mtp=False)
    g = Model(sm)
    sg = cmf_amd.SamplerConfig(temperature=1.0, top_k=k, top_p=tp, min_p=0.0, repetition_penalty=1.0)
    so = orc.SamplerCfg(1.0, tp, k, 1.0, 0.0, 0.0)
    lg = np.floor(synth.normal(7 + levels, V) * (levels / 8)).astype(np.float32)
    ids, pr = g.sparse_distribution(lg, sg)
    g.free()
    oid = np.empty(4 * 256 + 64, np.uint32)
    opr = np.empty(4 * 256 + 64, np.float32)
    P = lambda a: a.ctypes.data_as(C.c_void_p)
    n = orc.lib().or_sparse_distribution(P(lg), V, C.byref(so), None, 0, P(oid), P(opr))
    kth = np.sort(lg)[::-1][k - 1]
    print(f"levels {levels} k {k} top_p {tp}: k-th value {kth}, {int((lg >= kth).sum())} ids >= it; "
          f"device n={len(ids)} oracle n={n}", flush=True)
    assert (lg >= kth).sum() > k
    assert ids.tolist() == oid[:n].astype(np.int32).tolist()
    assert np.allclose(pr, opr[:n], rtol=1e-5, atol=1e-7)
