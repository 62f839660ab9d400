"""CPU pins of the oracle's model path: the C forward against an f64 numpy
forward of the same Qwen3-arch block (dequantized weights, plain softmax
attention), and greedy speculative decode == vanilla greedy
(pipeline.rs:11543-11564)."""
import numpy as np
import pytest

from oracle import oracle as orc

TINY = dict(n_layers=2, hidden=128, n_heads=4, n_kv=2, head_dim=32, inter=256, vocab=512, max_seq=64,
            rope_theta=1e6, eps=1e-6)


@pytest.fixture(scope="module")
def tiny():
    from cmf_amd import synth
    return synth.synth_model(TINY, seed=3, norm_noise=0.1, sigma=0.05)


def _dq(t):
    from cmf_amd import synth
    return synth.dequant(t).astype(np.float64)


def _rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def _rope(x, pos, theta):
    hd = x.shape[-1]
    inv = theta ** (-np.arange(0, hd, 2) / hd)
    ang = pos * inv
    a, b = x[..., : hd // 2], x[..., hd // 2:]
    return np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)], axis=-1)


def _np_forward(sm, toks):
    """f64 forward of every position; returns the final hidden rows (before the final norm)"""
    c = sm["cfg"]
    H, nh, nkv, hd, eps = c["hidden"], c["n_heads"], c["n_kv"], c["head_dim"], c["eps"]
    E = _dq(sm.get("embed", sm["lm_head"]))
    hs = np.stack([E[t] for t in toks])
    for l in sm["layers"]:
        Wq, Wk, Wv, Wo = _dq(l["wq"]), _dq(l["wk"]), _dq(l["wv"]), _dq(l["wo"])
        Wg, Wu, Wd = _dq(l["gate"]), _dq(l["up"]), _dq(l["down"])
        n = len(toks)
        x = np.stack([_rms(h, l["input_norm"], eps) for h in hs])
        q = (x @ Wq.T).reshape(n, nh, hd)
        k = (x @ Wk.T).reshape(n, nkv, hd)
        v = (x @ Wv.T).reshape(n, nkv, hd)
        q = np.stack([[_rope(_rms(q[p, h], l["q_norm"], eps), p, c["rope_theta"]) for h in range(nh)]
                      for p in range(n)])
        k = np.stack([[_rope(_rms(k[p, g], l["k_norm"], eps), p, c["rope_theta"]) for g in range(nkv)]
                      for p in range(n)])
        att = np.zeros((n, nh, hd))
        for p in range(n):
            for h in range(nh):
                g = h // (nh // nkv)
                s = k[: p + 1, g] @ q[p, h] / np.sqrt(hd)
                w = np.exp(s - s.max())
                att[p, h] = (w / w.sum()) @ v[: p + 1, g]
        hs = hs + att.reshape(n, nh * hd) @ Wo.T
        x2 = np.stack([_rms(h, l["post_norm"], eps) for h in hs])
        gg, uu = x2 @ Wg.T, x2 @ Wu.T
        hs = hs + (gg / (1 + np.exp(-gg)) * uu) @ Wd.T
    return hs


def test_forward_matches_f64_numpy(tiny):
    from cmf_amd import synth
    toks = synth.ids(4, 6, TINY["vocab"])
    o = orc.OracleModel(tiny, threads=2)
    got = np.stack([o.forward(int(t), i) for i, t in enumerate(toks)])
    ref = _np_forward(tiny, toks)
    rel = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert rel.max() < 1e-5, rel
    # the tied lm_head logits of the last row
    lg = o.logits(got[-1])
    E = _dq(tiny["lm_head"])
    ref_lg = E @ _rms(ref[-1], tiny["final_norm"], TINY["eps"])
    assert np.linalg.norm(lg - ref_lg) / np.linalg.norm(ref_lg) < 1e-5


def test_untied_embedding_matches_f64_numpy(tiny):
    """an embedding table of its own (loader.rs:714-724): rows come from it,
    logits from lm_head"""
    from cmf_amd import synth
    sm = dict(tiny, embed=synth.q8_normal(91, TINY["vocab"], TINY["hidden"], 0.05))
    toks = synth.ids(5, 4, TINY["vocab"])
    o = orc.OracleModel(sm, threads=2)
    got = np.stack([o.forward(int(t), i) for i, t in enumerate(toks)])
    ref = _np_forward(sm, toks)
    assert (np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)).max() < 1e-5
    tied = np.stack([orc.OracleModel(tiny, threads=2).forward(int(toks[0]), 0)])
    assert np.linalg.norm(tied[0] - got[0]) > 1e-3 * np.linalg.norm(got[0])  # the table matters
    lg = o.logits(got[-1])
    ref_lg = _dq(tiny["lm_head"]) @ _rms(ref[-1], tiny["final_norm"], TINY["eps"])
    assert np.linalg.norm(lg - ref_lg) / np.linalg.norm(ref_lg) < 1e-5


@pytest.mark.parametrize("k", [1, 3])
def test_spec_greedy_equals_vanilla(tiny, k):
    from cmf_amd import synth
    prompt = synth.ids(5, 9, TINY["vocab"])
    a, _ = orc.OracleModel(tiny, threads=2).generate(prompt, 20, spec=True, k=k)
    b, _ = orc.OracleModel(tiny, threads=2).generate(prompt, 20, spec=False)
    assert a[:20].tolist() == b[:20].tolist()


def test_spec_sampling_is_seed_deterministic(tiny):
    from cmf_amd import synth
    prompt = synth.ids(6, 7, TINY["vocab"])
    sc = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0)
    a, sa = orc.OracleModel(tiny, threads=2).generate(prompt, 16, spec=True, k=3, sampler=sc, seed=7)
    b, sb = orc.OracleModel(tiny, threads=4).generate(prompt, 16, spec=True, k=3, sampler=sc, seed=7)
    assert a.tolist() == b.tolist() and sa.accepted == sb.accepted
