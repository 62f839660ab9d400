"""GPU parity of the speculative ACCEPT path: the greedy and sampled
acceptance with a > 0, the commit of hidden row a, the trunk KV rollback of
rejected rows and the MTP re-warm of accepted pairs, against the CPU oracle.

The models accept drafts by construction: `synth.accept_model` (an MTP head
that repeats its input token over a trunk that emits runs of one token;
greedy K=4 rounds end at a = 0, 1, 3 and 4 on this prompt) and
`synth.constant_head_model` (the reference's
speculative_accepts_constant_oracle, pipeline.rs:11567-11587).

Checked: tokens and accepted counts equal the oracle's; the committed trunk
KV rows [0, next_pos) and MTP KV rows [0, next_pos - 1) equal plain
forwards of the emitted stream plus (h_p, t_{p+1}) warms, within relative
L2 1e-4 (the batched verify sums in another order than per-row forwards);
cmf_verify_step with chosen drafts (a = 0..K, greedy and under shared
uniforms) equals the oracle's or_verify_step."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096,
             max_seq=256, rope_theta=1e6, eps=1e-6)
GREEDY_PROMPT = 23   # oracle K=4 rounds by accepted count: [7, 2, 0, 2, 4]
SAMPLE_PROMPT = 19   # T=0.8 seed 1234, K=4: [6, 1, 1, 0, 6]
KV_TOL = 1e-4


@pytest.fixture(scope="module")
def acc(gpu):
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = synth.accept_model(SMALL)
    return sm, Model(sm)


def _sampler():
    import cmf_amd
    return (cmf_amd.SamplerConfig(temperature=0.8, repetition_penalty=1.0),
            orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0))


def _check_state(sm, g, seq, mtp_rows):
    """GPU trunk KV [0, len(seq)) and MTP KV [0, mtp_rows) against the
    oracle's plain forwards of seq with (h_p, t_{p+1}) warms"""
    ref = orc.OracleModel(sm)
    ref.prefill(np.asarray(seq))
    n = len(seq)
    for li in range(sm["cfg"]["n_layers"]):
        k, v = g.kv_export(li, n)
        rk, rv = ref.kv(li)
        ek, ev = rel_l2(k, rk), rel_l2(v, rv)
        print(f"  trunk layer {li}: rows {n} K rel {ek:.2e} V rel {ev:.2e}", flush=True)
        assert ek < KV_TOL and ev < KV_TOL
    k, v = g.kv_export(-1, mtp_rows)
    rk, rv = ref.kv(-1)
    ek, ev = rel_l2(k, rk[:, :mtp_rows]), rel_l2(v, rv[:, :mtp_rows])
    print(f"  MTP: rows {mtp_rows} K rel {ek:.2e} V rel {ev:.2e}", flush=True)
    assert ek < KV_TOL and ev < KV_TOL


@pytest.mark.parametrize("k", [1, 4])
def test_greedy_accepts_like_oracle(acc, k):
    """the whole decode loop (cmf_decode: rounds launched one at a time, plain
    steps at the end): tokens and accepted count equal the oracle's, > 0"""
    sm, g = acc
    from cmf_amd import synth
    prompt = synth.ids(GREEDY_PROMPT, 20, SMALL["vocab"])
    g.prefill(prompt)
    gt, gst = g.decode(40, spec=True, k=k)
    ot, ost = orc.OracleModel(sm).generate(prompt, 40, spec=True, k=k)
    print(f"k={k} gpu accepted {gst.accepted}/{gst.drafted} oracle {ost.accepted}/{ost.drafted} "
          f"hist {list(ost.hist)[:k + 1]}", flush=True)
    assert gt.tolist() == ot.tolist()
    assert gst.accepted == ost.accepted and gst.drafted == ost.drafted
    assert gst.accepted > 0
    if k == 4:
        assert sum(ost.hist[1:4]) > 0


@pytest.mark.parametrize("graph", [True, False])
@pytest.mark.parametrize("sampling", [False, True])
def test_rounds_commit_state(acc, graph, sampling, monkeypatch):
    """decode_rounds (captured HIP graph or eager launches): the emitted
    tokens are the oracle's, drafts were accepted, and the committed trunk and
    MTP caches are the plain-forward ones"""
    sm, g = acc
    from cmf_amd import synth
    from cmf_amd.model import Model
    sg, so = _sampler() if sampling else (None, None)
    prompt = synth.ids(SAMPLE_PROMPT if sampling else GREEDY_PROMPT, 20, SMALL["vocab"])
    m = g
    if not graph:
        monkeypatch.setenv("CMF_DECODE_GRAPH", "0")
        m = Model(sm)
    m.prefill(prompt)
    m.decode_begin(sampler=sg, seed=1234)
    st1 = m.decode_rounds(4, spec=True, k=4)
    st2 = m.decode_rounds(3, spec=True, k=4)
    toks = m.tokens()
    pos, _ = m.state()
    print(f"graph={graph} sampling={sampling}: accepted {st1.accepted}+{st2.accepted} of "
          f"{st1.drafted}+{st2.drafted}, next_pos {pos}, tokens {toks.tolist()}", flush=True)
    assert st1.drafted == 16 and st2.drafted == 12
    ot, _ = orc.OracleModel(sm).generate(prompt, len(toks) + 6, spec=True, k=4, sampler=so, seed=1234)
    assert toks.tolist() == ot[:len(toks)].tolist()
    assert st1.accepted + st2.accepted > 0
    assert len(toks) == 7 + st1.accepted + st2.accepted
    assert pos == len(prompt) + len(toks)
    _check_state(sm, m, np.concatenate([prompt, toks]), pos - 1)
    if m is not g:
        m.free()


def test_constant_head_accepts_everything(gpu):
    """pipeline.rs:11567-11587 on the device: every logit ties, the trunk and
    the draft head both pick the highest id, every draft is accepted"""
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = synth.constant_head_model(SMALL)
    g = Model(sm)
    g.prefill(synth.ids(4, 4, SMALL["vocab"]))
    toks, st = g.decode(10, spec=True, k=4)
    g.free()
    print("constant head:", toks.tolist(), st.accepted, st.drafted, flush=True)
    assert st.drafted > 0 and st.accepted == st.drafted
    assert set(toks.tolist()) == {SMALL["vocab"] - 1}


def _vanilla(sm, prompt, n):
    toks, _ = orc.OracleModel(sm).generate(prompt, n, spec=False)
    return toks


@pytest.mark.parametrize("a_want", [0, 1, 2, 3, 4])
def test_verify_step_greedy(acc, a_want):
    """cmf_verify_step with drafts = the next a_want vanilla tokens, then a
    wrong one: a, the next token, the row picks and the committed caches
    equal the oracle's or_verify_step"""
    sm, g = acc
    from cmf_amd import synth
    K, V = 4, SMALL["vocab"]
    prompt = synth.ids(7, 12, V)
    s = _vanilla(sm, prompt, K + 2)
    toks = [int(t) for t in s[:a_want + 1]]
    while len(toks) < K + 1:
        toks.append((int(s[len(toks)]) + 1) % V)
    g.prefill(prompt)
    a, nxt, am, lg = g.verify_step(toks, len(prompt), want_logits=True)
    o = orc.OracleModel(sm)
    tip = o.prefill(prompt)
    oa, onxt, _, oam, olg = o.verify_step(tip, len(prompt), toks, past=np.concatenate([prompt, s[:1]]))
    print(f"a_want {a_want}: gpu a={a} next={nxt} argmax={am.tolist()} | oracle a={oa} next={onxt} "
          f"argmax={oam.tolist()} | logits rel {rel_l2(lg, olg):.2e}", flush=True)
    assert oa == a_want and a == oa and nxt == onxt
    assert am.tolist() == oam.tolist()
    assert rel_l2(lg, olg) < 1e-4
    pos, _ = g.state()
    assert pos == len(prompt) + a + 1
    _check_state(sm, g, np.concatenate([prompt, s[:a + 1]]), pos - 1)
    # the decode continues from the committed state like the oracle's vanilla stream
    g.decode_begin(seed=0)
    g.decode_rounds(2, spec=False)
    cont = g.tokens()
    want = _vanilla(sm, prompt, a + 4)[a + 1:a + 3]
    assert cont.tolist() == want.tolist()


def test_verify_step_sampled_uniforms(acc):
    """the sampled verify under shared uniforms: drafts with q = {d: 1}; the
    third draft is outside every top-k (p_d = 0) and is rejected; uniforms
    [0, 0, 0, .37] give a = 2 and the correction drawn from row 2 at .37,
    equal to the oracle's"""
    sm, g = acc
    from cmf_amd import synth
    K, V = 4, SMALL["vocab"]
    sg, so = _sampler()
    prompt = synth.ids(7, 12, V)
    s = _vanilla(sm, prompt, K + 2)
    o0 = orc.OracleModel(sm)
    tip0 = o0.prefill(prompt)
    _, _, _, _, lg = o0.verify_step(tip0, len(prompt), s[:K + 1])
    far = int(np.argmin(lg[2]))
    toks = [int(s[0]), int(s[1]), int(s[2]), far, int(s[4])]
    qi = np.zeros((K, 64), np.int32)
    qp = np.zeros((K, 64), np.float32)
    qi[:, 0] = toks[1:]
    qp[:, 0] = 1.0
    qn = np.ones(K, np.int32)
    for u_c in (0.37, 0.93):
        g.prefill(prompt)
        a, nxt, _, _ = g.verify_step(toks, len(prompt), sampler=sg, q=(qi, qp, qn), uniforms=[0.0, 0.0, 0.0, u_c])
        o = orc.OracleModel(sm)
        tip = o.prefill(prompt)
        oa, onxt, _, _, _ = o.verify_step(tip, len(prompt), toks, sampler=so, q=(qi.astype(np.uint32), qp, qn),
                                          uniforms=[0.0, 0.0, 0.0, u_c], past=np.concatenate([prompt, s[:1]]))
        print(f"u_c {u_c}: gpu a={a} next={nxt} | oracle a={oa} next={onxt}", flush=True)
        assert a == oa == 2 and nxt == onxt
        pos, _ = g.state()
        _check_state(sm, g, np.concatenate([prompt, s[:3]]), pos - 1)
    # every draft accepted: the bonus token is drawn from row K at the last uniform
    toks2 = [int(t) for t in s[:K + 1]]
    qi[:, 0] = toks2[1:]
    g.prefill(prompt)
    a, nxt, _, _ = g.verify_step(toks2, len(prompt), sampler=sg, q=(qi, qp, qn), uniforms=[0.0] * K + [0.5])
    o = orc.OracleModel(sm)
    tip = o.prefill(prompt)
    oa, onxt, _, _, _ = o.verify_step(tip, len(prompt), toks2, sampler=so, q=(qi.astype(np.uint32), qp, qn),
                                      uniforms=[0.0] * K + [0.5], past=np.concatenate([prompt, s[:1]]))
    print(f"all accepted: gpu a={a} next={nxt} | oracle a={oa} next={onxt}", flush=True)
    assert a == oa == K and nxt == onxt


def test_kv_truncate_then_append(acc):
    """kv_cache.rs:883 truncate_last on the device: forward 6 tokens, roll
    back 3, forward 2 others at the cut; the cache equals plain forwards of
    the surviving stream"""
    sm, g = acc
    from cmf_amd import synth
    V = SMALL["vocab"]
    first = synth.ids(31, 6, V)
    other = synth.ids(32, 2, V)
    g.forward_batch(first, 0, want_logits=False)
    assert g.state()[0] == 6
    g.kv_truncate(3)
    pos, _ = g.state()
    assert pos == 3
    g.forward_batch(other, pos, want_logits=False)
    assert g.state()[0] == 5
    seq = np.concatenate([first[:3], other])
    ref = orc.OracleModel(sm)
    for p, t in enumerate(seq):
        ref.forward(int(t), p)
    for li in range(SMALL["n_layers"]):
        k, v = g.kv_export(li, 5)
        rk, rv = ref.kv(li)
        print(f"layer {li}: K rel {rel_l2(k, rk):.2e} V rel {rel_l2(v, rv):.2e}", flush=True)
        assert rel_l2(k, rk) < KV_TOL and rel_l2(v, rv) < KV_TOL
