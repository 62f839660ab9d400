"""CPU pins of the oracle's model path: the C forward against an f64 numpy
forward of the same Qwen3-arch block (dequantized weights, plain softmax
attention), and greedy speculative decode == vanilla greedy
(pipeline.rs:11543-11564)."""
import ctypes as C

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
        if "moe" not in l:
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
        if "moe" in l:  # softmax router, top-k renormalised, weighted expert sum
            mo = l["moe"]
            r = mo["router"]
            R = np.ascontiguousarray(r["bytes"]).view(np.float16).astype(np.float64).reshape(r["rows"], r["cols"]) \
                if r["dtype"] == 1 else _dq(r)
            for p in range(n):
                lg = R @ x2[p]
                pr = np.exp(lg - lg.max())
                pr /= pr.sum()
                top = sorted(range(len(pr)), key=lambda e: (-pr[e], e))[:mo["top_k"]]
                ws = pr[top] / (pr[top].sum() if mo.get("norm_topk", True) else 1.0) * mo.get("routed_scaling", 1.0)
                for e, w in zip(top, ws):
                    ex = mo["experts"][e]
                    g, u = _dq(ex["gate"]) @ x2[p], _dq(ex["up"]) @ x2[p]
                    hs[p] = hs[p] + w * (_dq(ex["down"]) @ (g / (1 + np.exp(-g)) * u))
            continue
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


MOE = dict(n_experts=8, top_k=3, inter=64, layers=[1])


@pytest.mark.parametrize("router", ["q8", "f16"])
def test_moe_layer_matches_f64_numpy(router):
    """a decoder whose layer 1 is a routed MoE FFN (Qwen3-MoE: softmax router
    over the normed row, top-k renormalised, weighted expert SwiGLUs;
    pipeline.rs:10868-11045) against the f64 numpy forward; the routing
    differs per position (more than top_k experts used over the rows)"""
    from cmf_amd import synth
    sm = synth.synth_model(TINY, seed=4, norm_noise=0.1, sigma=0.05, moe=dict(MOE, router_dtype=router))
    toks = synth.ids(6, 6, TINY["vocab"])
    o = orc.OracleModel(sm, threads=2)
    got = np.stack([o.forward(int(t), i) for i, t in enumerate(toks)])
    ref = _np_forward(sm, toks)
    rel = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert rel.max() < 1e-5, rel
    # the MoE layer matters: the dense twin of layer 1 gives other rows
    dense = synth.synth_model(TINY, seed=4, norm_noise=0.1, sigma=0.05)
    d = np.stack([orc.OracleModel(dense, threads=2).forward(int(toks[0]), 0)])
    assert np.linalg.norm(d[0] - got[0]) > 1e-3 * np.linalg.norm(got[0])


def test_moe_model_spec_greedy_equals_vanilla():
    from cmf_amd import synth
    sm = synth.synth_model(TINY, seed=4, norm_noise=0.1, sigma=0.05, moe=MOE)
    prompt = synth.ids(8, 9, TINY["vocab"])
    a, _ = orc.OracleModel(sm, threads=2).generate(prompt, 16, spec=True, k=3)
    b, _ = orc.OracleModel(sm, threads=2).generate(prompt, 16, spec=False)
    assert a[:16].tolist() == b[:16].tolist()


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


# ---------------------------------------------------------------------------
# The accept / commit / re-warm branch of graph_spec_step, pinned on models
# whose drafts get accepted.
# ---------------------------------------------------------------------------
ACC_PROMPT_SEED = 23  # greedy K=4 rounds accept 0, 1, 3 and 4 drafts on TINY / SMALL


@pytest.fixture(scope="module")
def acc():
    from cmf_amd import synth
    return synth.accept_model(TINY)


def _reference_state(sm, toks):
    """trunk KV of positions [0, n) and MTP KV rows [0, n-1) built by plain
    forwards and (h_p, t_{p+1}) warms — what every committed round must
    leave (pipeline.rs:2275-2318 prefill warm, 4120-4176 re-warm)"""
    o = orc.OracleModel(sm, threads=2)
    o.prefill(np.asarray(toks))
    return o


def _assert_state_equal(o, ref, n_layers):
    for li in list(range(n_layers)) + [-1]:
        k, v = o.kv(li)
        rk, rv = ref.kv(li)
        if li < 0:  # plain steps after the last round do not warm the head
            assert k.shape[1] <= rk.shape[1]
            rk, rv = rk[:, :k.shape[1]], rv[:, :k.shape[1]]
        assert k.shape == rk.shape, (li, k.shape, rk.shape)
        assert np.array_equal(k, rk) and np.array_equal(v, rv), li


def test_spec_accepts_constant_oracle():
    """pipeline.rs:11567-11587: constant lm_head -> every logit ties -> the
    trunk and the draft head both pick the highest id: 100% acceptance and
    one repeated token"""
    from cmf_amd import synth
    sm = synth.constant_head_model(TINY)
    prompt = synth.ids(4, 4, TINY["vocab"])
    toks, st = orc.OracleModel(sm, threads=2).generate(prompt, 10, spec=True, k=4)
    assert st.drafted > 0
    assert st.accepted == st.drafted
    assert st.hist[4] == st.rounds
    assert set(toks.tolist()) == {TINY["vocab"] - 1}


@pytest.mark.parametrize("k", [1, 4])
def test_spec_greedy_equals_vanilla_with_acceptance(acc, k):
    """speculative_equals_vanilla_greedy (pipeline.rs:11543-11564) with the
    evidence the reference's test asks for: drafts are accepted, and for
    K = 4 rounds end at 0 < a < K (partial commits)"""
    from cmf_amd import synth
    prompt = synth.ids(ACC_PROMPT_SEED, 20, TINY["vocab"])
    o = orc.OracleModel(acc, threads=2)
    a, st = o.generate(prompt, 40, spec=True, k=k)
    b, _ = orc.OracleModel(acc, threads=2).generate(prompt, 40, spec=False)
    assert a[:40].tolist() == b[:40].tolist()
    assert st.accepted > 0
    if k == 4:
        assert sum(st.hist[1:4]) > 0, list(st.hist)
        assert st.hist[0] > 0 and st.hist[4] > 0
    # committed state == plain forwards + (h_p, t_{p+1}) warms
    n = o.kvs[0].len
    assert n - 1 - k <= o.st.mtp.len <= n - 1
    ref = _reference_state(acc, np.concatenate([prompt, a])[:n])
    _assert_state_equal(o, ref, TINY["n_layers"])


def test_spec_sampling_accepts_and_commits(acc):
    """temperature 0.8: drafts are accepted (some rounds partially), the run
    is seed-deterministic and the committed state is the plain-forward one"""
    from cmf_amd import synth
    prompt = synth.ids(19, 20, TINY["vocab"])
    sc = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0)
    o = orc.OracleModel(acc, threads=2)
    a, st = o.generate(prompt, 40, spec=True, k=4, sampler=sc, seed=1234)
    b, st2 = orc.OracleModel(acc, threads=4).generate(prompt, 40, spec=True, k=4, sampler=sc, seed=1234)
    assert a.tolist() == b.tolist() and st.accepted == st2.accepted
    assert st.accepted > 0 and sum(st.hist[1:4]) > 0, list(st.hist)
    n = o.kvs[0].len
    ref = _reference_state(acc, np.concatenate([prompt, a])[:n])
    _assert_state_equal(o, ref, TINY["n_layers"])


def test_spec_accept_hand_computed_toy():
    """spec_accept_or_correct_sparse (sampler.rs:683-711) on a 3-token toy,
    by hand, over SplitMix64 seed 0's published uniforms 0.8833108,
    0.43152797, 0.026433766:
      p = {0: .5, 1: .3, 2: .2}, q = {0: .2, 1: .8}
      d = 0: r = .8833; r*q_d = .1767 < p_d = .5       -> accept
      d = 1: r = .4315; r*q_d = .3452 >= p_d = .3      -> reject;
             residual max(0, p - q) = {0: .3, 2: .2} -> {0: .6, 2: .4};
             r = .0264 < .6                            -> correction 0
    and with caller uniforms [.9, .7]: d = 1 rejected, .7 >= .6 -> 2"""
    L = orc.lib()
    pid, pp = np.array([0, 1, 2], np.uint32), np.array([0.5, 0.3, 0.2], np.float32)
    qid, qp = np.array([0, 1], np.uint32), np.array([0.2, 0.8], np.float32)
    P = lambda a: a.ctypes.data_as(C.c_void_p)
    r = orc.Rng(0)
    assert L.or_spec_accept_sparse(P(pid), P(pp), 3, P(qid), P(qp), 2, 0, C.byref(r)) == -1
    assert L.or_spec_accept_sparse(P(pid), P(pp), 3, P(qid), P(qp), 2, 1, C.byref(r)) == 0
    u = np.array([0.9, 0.7], np.float32)
    r = orc.Rng(0, P(u), 2, 0)
    assert L.or_spec_accept_sparse(P(pid), P(pp), 3, P(qid), P(qp), 2, 1, C.byref(r)) == 2
    assert r.used == 2
    # three uniforms of seed 0 consumed by the first two calls
    r = orc.Rng(0)
    L.or_spec_accept_sparse(P(pid), P(pp), 3, P(qid), P(qp), 2, 0, C.byref(r))
    L.or_spec_accept_sparse(P(pid), P(pp), 3, P(qid), P(qp), 2, 1, C.byref(r))
    r0 = orc.Rng(0)
    for _ in range(3):
        L.or_rng_next_u64(C.byref(r0))
    assert r.state == r0.state


def _vanilla(sm, prompt, n):
    toks, _ = orc.OracleModel(sm, threads=2).generate(prompt, n, spec=False)
    return toks


@pytest.mark.parametrize("a_want", [0, 1, 2, 3, 4])
def test_verify_step_greedy_chosen_drafts(acc, a_want):
    """or_verify_step with drafts = the next a_want vanilla tokens and then a
    wrong one: a == a_want, the next token and the row picks are the vanilla
    ones, and the committed trunk / MTP caches equal plain forwards"""
    from cmf_amd import synth
    K = 4
    prompt = synth.ids(7, 12, TINY["vocab"])
    s = _vanilla(acc, prompt, K + 2)  # s[0] = t_next
    toks = [int(t) for t in s[:a_want + 1]]
    while len(toks) < K + 1:
        toks.append((int(s[len(toks)]) + 1) % TINY["vocab"])
    o = orc.OracleModel(acc, threads=2)
    tip = o.prefill(prompt)
    a, nxt, h, am, lg = o.verify_step(tip, len(prompt), toks, past=np.concatenate([prompt, s[:1]]))
    assert a == a_want
    assert nxt == int(s[a + 1])
    assert am[:a + 1].tolist() == [int(t) for t in s[1:a + 2]]
    assert o.kvs[0].len == len(prompt) + a + 1 and o.st.mtp.len == len(prompt) + a
    ref = _reference_state(acc, np.concatenate([prompt, s[:a + 1]]))
    _assert_state_equal(o, ref, TINY["n_layers"])
    # the hidden row a is the plain forward's tip
    ref2 = orc.OracleModel(acc, threads=2)
    hp = ref2.prefill(np.concatenate([prompt, s[:a + 1]]))
    assert np.array_equal(h, hp)


def test_verify_step_sampled_shared_uniforms(acc):
    """the sampled verify under caller uniforms: draft i = the vanilla
    argmax token with q = {d: 1}; uniforms 0 accept every draft inside
    supp(p); a draft outside the top-k is rejected (p_d = 0) and the
    correction is p's inverse CDF at the next uniform"""
    from cmf_amd import synth
    K = 4
    V = TINY["vocab"]
    prompt = synth.ids(7, 12, V)
    s = _vanilla(acc, prompt, K + 2)
    sc = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0)
    o0 = orc.OracleModel(acc, threads=2)
    tip0 = o0.prefill(prompt)
    _, _, _, _, lg = o0.verify_step(tip0, len(prompt), s[:K + 1], past=np.concatenate([prompt, s[:1]]))
    # a token outside every row's top-40
    far = int(np.argmin(lg[2]))
    toks = [int(s[0]), int(s[1]), int(s[2]), far, int(s[4])]
    qi = np.zeros((K, 64), np.uint32)
    qp = np.zeros((K, 64), np.float32)
    qi[:, 0] = toks[1:]
    qp[:, 0] = 1.0
    qn = np.ones(K, np.int32)
    u_c = 0.37
    o = orc.OracleModel(acc, threads=2)
    tip = o.prefill(prompt)
    a, nxt, h, am, lg2 = o.verify_step(tip, len(prompt), toks, sampler=sc, q=(qi, qp, qn),
                                       uniforms=[0.0, 0.0, 0.0, u_c], past=np.concatenate([prompt, s[:1]]))
    assert a == 2 and o.rng_used == 4
    # p of row 2 (the stream holds the accepted drafts) at u_c
    ids = np.empty(4 * 256 + 64, np.uint32)
    pr = np.empty(4 * 256 + 64, np.float32)
    past = np.concatenate([prompt, s[:3]]).astype(np.uint32)
    P = lambda x: x.ctypes.data_as(C.c_void_p)
    m = orc.lib().or_sparse_distribution(P(np.ascontiguousarray(lg2[2])), V, C.byref(sc), P(past), len(past),
                                         P(ids), P(pr))
    assert far not in ids[:m].tolist()
    cdf = np.cumsum(pr[:m].astype(np.float32), dtype=np.float32)
    assert nxt == int(ids[int(np.argmax(u_c < cdf))])
    ref = _reference_state(acc, np.concatenate([prompt, s[:3]]))
    _assert_state_equal(o, ref, TINY["n_layers"])


def test_a8w8_contract_switch(tiny):
    """OracleModel(a8w8=True) routes the forward's quantized matvecs through
    the a8w8 contract (split_act + integer dots, qtensor.rs:9237-9281): the
    hidden state moves by the contract's activation rounding (~1e-2), and the
    exact model is untouched by the switch"""
    he = orc.OracleModel(tiny, threads=2).forward(5, 0)
    ha = orc.OracleModel(tiny, threads=2, a8w8=True).forward(5, 0)
    he2 = orc.OracleModel(tiny, threads=2, a8w8=False).forward(5, 0)
    rel = np.linalg.norm(he - ha) / np.linalg.norm(he)
    assert 1e-4 < rel < 5e-2
    assert np.array_equal(he, he2)


def _np_block(l, xs, c):
    """f64 dense decoder block over rows xs at positions 0..n-1 (its own
    causal KV): the per-layer body of _np_forward"""
    H, nh, nkv, hd, eps = c["hidden"], c["n_heads"], c["n_kv"], c["head_dim"], c["eps"]
    Wq, Wk, Wv, Wo = _dq(l["wq"]), _dq(l["wk"]), _dq(l["wv"]), _dq(l["wo"])
    Wg, Wu, Wd = _dq(l["gate"]), _dq(l["up"]), _dq(l["down"])
    hs = np.array(xs, np.float64)
    n = len(hs)
    x = np.stack([_rms(h, l["input_norm"], eps) for h in hs])
    q = (x @ Wq.T).reshape(n, nh, hd)
    k = (x @ Wk.T).reshape(n, nkv, hd)
    v = (x @ Wv.T).reshape(n, nkv, hd)
    q = np.stack([[_rope(_rms(q[p, h], l["q_norm"], eps), p, c["rope_theta"]) for h in range(nh)] for p in range(n)])
    k = np.stack([[_rope(_rms(k[p, g], l["k_norm"], eps), p, c["rope_theta"]) for g in range(nkv)] for p in range(n)])
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
    return hs + (gg / (1 + np.exp(-gg)) * uu) @ Wd.T


def test_mtp_step_matches_f64_numpy(tiny):
    """or_mtp_step (mtp_step_hl, pipeline.rs:3051-3160) with a random,
    non-zero hidden half of eh_proj: x = eh_proj [rms(embed(t_{p+1}), enorm);
    rms(h_p, hnorm)] with h_p the trunk output BEFORE the final norm (the
    decode loop's `hidden`, pipeline.rs:2563-2571), one block over the MTP's
    own KV at positions 0..p, logits = lm_head rms(block(x), mtp norm).  The
    f64 restatement pins the block output and the logits at every position;
    the plausible mistakes (no hnorm, the post-final-norm hidden fed, the
    halves swapped) each land far outside the tolerance."""
    from cmf_amd import synth
    c = TINY
    H, eps = c["hidden"], c["eps"]
    mtp = tiny["mtp"]
    Weh = _dq(mtp["eh_proj"])
    assert np.abs(Weh[:, H:]).max() > 0.0  # the hidden half takes part
    E = _dq(tiny["lm_head"])
    toks = synth.ids(12, 7, c["vocab"])
    hs = _np_forward(tiny, toks)  # pre-final-norm trunk rows (f64)
    o = orc.OracleModel(tiny, threads=2)
    hid = [o.forward(int(t), i) for i, t in enumerate(toks)]
    got_lg, got_h = [], []
    for p in range(len(toks) - 1):
        lg = np.empty(c["vocab"], np.float32)
        ho = np.empty(H, np.float32)
        orc.lib().or_mtp_step(C.byref(o.m), C.byref(o.st), orc._p(hid[p]), int(toks[p + 1]), p, orc._p(lg), orc._p(ho))
        got_lg.append(lg)
        got_h.append(ho)

    def ref(variant):
        xs = []
        for p in range(len(toks) - 1):
            e = _rms(E[toks[p + 1]], mtp["enorm"], eps)
            h = hs[p]
            if variant == "post_norm":
                h = _rms(h, tiny["final_norm"], eps)
            hh = h if variant == "no_hnorm" else _rms(h, mtp["hnorm"], eps)
            xs.append(Weh @ (np.concatenate([hh, e]) if variant == "swapped" else np.concatenate([e, hh])))
        outs = _np_block(mtp["layer"], xs, c)
        return outs, [E @ _rms(x, mtp["norm"], eps) for x in outs]

    rh, rl = ref("exact")
    for p in range(len(got_h)):
        eh = np.linalg.norm(got_h[p] - rh[p]) / np.linalg.norm(rh[p])
        el = np.linalg.norm(got_lg[p] - rl[p]) / np.linalg.norm(rl[p])
        assert eh < 1e-5 and el < 1e-5, (p, eh, el)
    for variant in ("no_hnorm", "post_norm", "swapped"):
        wh, _ = ref(variant)
        d = max(np.linalg.norm(got_h[p] - wh[p]) / np.linalg.norm(wh[p]) for p in range(len(got_h)))
        assert d > 1e-2, (variant, d)
