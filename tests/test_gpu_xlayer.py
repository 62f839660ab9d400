"""GPU parity of the XCD-partitioned decoder blocks (xlayer.hip: attention
and FFN of a block as two launches whose per-XCD workgroups exchange tagged
partials through the XCD's L2) against the CPU oracle and against the
six-launch blocks of the same model (CMF_XL=0 at model creation).

The model has config 4's block shape (hidden 1024, 16 query / 8 KV heads of
128, FFN 3072, q8 attention, q4t FFN) over 2 layers and a 4096-token
vocabulary, so the oracle runs in seconds; `synth.accept_model` with
sigma 0.02 drafts tokens the trunk accepts (greedy K=4 rounds on prompt 23
end at a = 0, 1, 2 and 4; T=0.8 on prompt 19 with seed 7 at a = 0..4), so
the commit, rollback and MTP re-warm run through the new launches too.

Checked: verify-batch hidden rows (1, 5, 9 and 16 rows: one MFMA for hi and
lo planes up to 8 rows, two beyond) within 3e-4 relative L2 of the oracle
and 5e-5 of the six-launch blocks, the same argmax; greedy and sampled
tokens and accepted counts equal to the oracle's, eager and graph-captured;
the committed trunk and MTP caches equal to plain forwards; at contexts of
1000, 2300 and 2900 positions (the attention launch's three tile counts) the
verify rows and new K / V rows equal the six-launch blocks'."""
import os

import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

XL = dict(n_layers=2, hidden=1024, n_heads=16, n_kv=8, head_dim=128, inter=3072, vocab=4096, max_seq=512,
          rope_theta=1e6, eps=1e-6)
GREEDY_PROMPT = 23   # oracle K=4 rounds by accepted count: [14, 1, 2, 0, 4]
SAMPLE_PROMPT = 19   # T=0.8 seed 7, K=4: [7, 2, 1, 1, 4]
SAMPLE_SEED = 7
HID_TOL, PATH_TOL, KV_TOL = 3e-4, 5e-5, 3e-4


def _model(sm, xl=True):
    from cmf_amd.model import Model
    old = os.environ.get("CMF_XL")
    if xl:
        os.environ.pop("CMF_XL", None)
    else:
        os.environ["CMF_XL"] = "0"
    try:
        return Model(sm)
    finally:
        if old is None:
            os.environ.pop("CMF_XL", None)
        else:
            os.environ["CMF_XL"] = old


@pytest.fixture(scope="module")
def xl(gpu):
    from cmf_amd import synth
    sm = synth.accept_model(XL, sigma=0.02, eh_noise=10.0)
    g, six = _model(sm), _model(sm, xl=False)
    # on an MI355X (256 CUs) this block shape takes the XCD-partitioned launches
    assert gpu.lib().cmf_model_fused_blocks(g.h) == 1
    assert gpu.lib().cmf_model_fused_blocks(six.h) == 0
    yield sm, g, six
    g.free()
    six.free()


def _sampler():
    import cmf_amd
    return (cmf_amd.SamplerConfig(temperature=0.8, repetition_penalty=1.0),
            orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0))


def _check_state(sm, g, seq, mtp_rows):
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


@pytest.mark.parametrize("b", [1, 5, 9, 16])
def test_forward_batch_matches_oracle(xl, b):
    sm, g, six = xl
    from cmf_amd import synth
    ids = synth.ids(7, b, XL["vocab"])
    h1, l1 = g.forward_batch(ids, 0)
    h0, l0 = six.forward_batch(ids, 0)
    o = orc.OracleModel(sm)
    for i, t in enumerate(ids):
        h = o.forward(int(t), i)
        ol = o.logits(h)
        print(f"b={b} row {i}: hidden rel {rel_l2(h1[i], h):.2e} (six-launch {rel_l2(h0[i], h):.2e}, "
              f"between {rel_l2(h1[i], h0[i]):.2e}) logits rel {rel_l2(l1[i], ol):.2e}", flush=True)
        assert rel_l2(h1[i], h) < HID_TOL
        assert rel_l2(h1[i], h0[i]) < PATH_TOL
        assert int(np.argmax(l1[i])) == int(np.argmax(ol))


@pytest.mark.parametrize("k", [1, 4])
def test_greedy_accepts_like_oracle(xl, k):
    sm, g, _ = xl
    from cmf_amd import synth
    prompt = synth.ids(GREEDY_PROMPT, 20, XL["vocab"])
    g.prefill(prompt)
    gt, gst = g.decode(40, spec=True, k=k)
    ot, ost = orc.OracleModel(sm).generate(prompt, 40, spec=True, k=k)
    print(f"k={k}: gpu accepted {gst.accepted}/{gst.drafted} oracle {ost.accepted}/{ost.drafted} "
          f"hist {list(ost.hist)[:k + 1]}", flush=True)
    assert gt.tolist() == ot.tolist()
    assert gst.accepted == ost.accepted and gst.drafted == ost.drafted
    assert gst.accepted > 0
    if k == 4:
        assert sum(ost.hist[1:4]) > 0


@pytest.mark.parametrize("sampling", [False, True])
def test_graph_rounds_commit_state(xl, sampling):
    """rounds replayed from a captured HIP graph: tokens are the oracle's,
    drafts were accepted, the committed caches are the plain-forward ones"""
    sm, g, _ = xl
    from cmf_amd import synth
    sg, so = _sampler() if sampling else (None, None)
    seed = SAMPLE_SEED if sampling else 0
    prompt = synth.ids(SAMPLE_PROMPT if sampling else GREEDY_PROMPT, 20, XL["vocab"])
    g.prefill(prompt)
    g.decode_begin(sampler=sg, seed=seed)
    st1 = g.decode_rounds(5, spec=True, k=4)
    st2 = g.decode_rounds(4, spec=True, k=4)
    toks = g.tokens()
    pos, _ = g.state()
    print(f"sampling={sampling}: accepted {st1.accepted}+{st2.accepted} of {st1.drafted}+{st2.drafted}, "
          f"tokens {toks.tolist()}", flush=True)
    ot, _ = orc.OracleModel(sm).generate(prompt, len(toks) + 6, spec=True, k=4, sampler=so, seed=seed)
    assert toks.tolist() == ot[:len(toks)].tolist()
    assert st1.accepted + st2.accepted > 0
    assert pos == len(prompt) + len(toks)
    _check_state(sm, g, np.concatenate([prompt, toks]), pos - 1)


def test_sampled_decode_like_oracle(xl):
    sm, g, _ = xl
    from cmf_amd import synth
    sg, so = _sampler()
    prompt = synth.ids(SAMPLE_PROMPT, 20, XL["vocab"])
    g.prefill(prompt)
    gt, gst = g.decode(40, sampler=sg, seed=SAMPLE_SEED, spec=True, k=4)
    ot, ost = orc.OracleModel(sm).generate(prompt, 40, spec=True, k=4, sampler=so, seed=SAMPLE_SEED)
    print(f"T=0.8: gpu accepted {gst.accepted}/{gst.drafted} oracle {ost.accepted}/{ost.drafted}", flush=True)
    assert gt.tolist() == ot.tolist()
    assert gst.accepted == ost.accepted and gst.accepted > 0


XL_LONG = dict(XL, max_seq=3072)


@pytest.fixture(scope="module")
def xl_long(gpu):
    from cmf_amd import synth
    sm = synth.accept_model(XL_LONG, sigma=0.02, eh_noise=10.0)
    g, six = _model(sm), _model(sm, xl=False)
    assert gpu.lib().cmf_model_fused_blocks(g.h) == 1
    yield sm, g, six
    g.free()
    six.free()


@pytest.mark.parametrize("pos0", [1000, 2300, 2900])
def test_long_context_matches_six_launch(xl_long, pos0):
    """the attention launch is instantiated for 4, 5 and 6 position tiles
    per workgroup, picked from the call's position bound (pos0 + b: 63, 145
    and 182 tiles over 32 workgroups); after the same prefill, the verify
    rows and the appended K / V rows equal the six-launch blocks' (whose
    attention the oracle pins at short context)"""
    sm, g, six = xl_long
    from cmf_amd import synth
    prompt = synth.ids(31, pos0, XL["vocab"])
    ids = synth.ids(37, 5, XL["vocab"])
    g.prefill(prompt)
    six.prefill(prompt)
    h1, l1 = g.forward_batch(ids, pos0)
    h0, l0 = six.forward_batch(ids, pos0)
    for i in range(len(ids)):
        e = rel_l2(h1[i], h0[i])
        print(f"pos0={pos0} row {i}: hidden rel {e:.2e}", flush=True)
        assert e < PATH_TOL
        assert int(np.argmax(l1[i])) == int(np.argmax(l0[i]))
    n = pos0 + len(ids)
    for li in range(XL["n_layers"]):
        k1, v1 = g.kv_export(li, n)
        k0, v0 = six.kv_export(li, n)
        ek, ev = rel_l2(k1[:, pos0:], k0[:, pos0:]), rel_l2(v1[:, pos0:], v0[:, pos0:])
        print(f"  layer {li}: new K rel {ek:.2e} V rel {ev:.2e}", flush=True)
        assert ek < PATH_TOL and ev < PATH_TOL


_FALLBACK_CHILD = r"""
import sys, json
sys.path.insert(0, sys.argv[1])
import numpy as np
import cmf_amd
from cmf_amd import synth
from cmf_amd.model import Model
from oracle import oracle as orc
cmf_amd.init(0)
XL = dict(n_layers=2, hidden=1024, n_heads=16, n_kv=8, head_dim=128, inter=3072, vocab=4096, max_seq=512,
          rope_theta=1e6, eps=1e-6)
sm = synth.accept_model(XL, sigma=0.02, eh_noise=10.0)
g = Model(sm)
fused0 = cmf_amd.lib().cmf_model_fused_blocks(g.h)
prompt = synth.ids(23, 40, XL["vocab"])
g.prefill(prompt)
g.decode_begin(seed=0)
st = g.decode_rounds(4, spec=True, k=4)
got = g.tokens()
ot, _ = orc.OracleModel(sm).generate(prompt, len(got) + 6, spec=True, k=4)
print(json.dumps({"fused0": fused0, "fused1": cmf_amd.lib().cmf_model_fused_blocks(g.h),
                  "fallbacks": cmf_amd.lib().cmf_model_xl_fallbacks(g.h), "accepted": st.accepted,
                  "gpu": got.tolist(), "cpu": ot[:len(got)].tolist()}))
"""


def test_failed_check_falls_back_to_six_launch_blocks(gpu):
    """A call whose XCD-partitioned blocks fail their check (forced from the
    host here: CMF_XL_FORCE_FAIL=1 reports one failure after the first
    call) switches the model to the six-launch blocks and runs again from
    the decode state before it: the tokens (greedy K = 4 rounds with drafts
    accepted, replayed from a captured graph) still equal the oracle's"""
    import json
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, CMF_XL_FORCE_FAIL="1")
    r = subprocess.run([sys.executable, "-c", _FALLBACK_CHILD, root], env=env, capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["fused0"] == 1 and res["fused1"] == 0 and res["fallbacks"] == 1
    assert res["accepted"] > 0
    assert res["gpu"] == res["cpu"]
