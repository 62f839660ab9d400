"""Sampled speculative decode over tied logits on the GPU against the oracle.

The model's tied q8 lm_head has two groups of identical rows (ids 0..2047
and 2048..4095), so every logit takes one of two values and the larger one
is shared by 2048 ids: par_topk keeps the top k and every tie of the k-th
value, the first 4 k + 64 in index order (sampler.rs:515-600), so each
sparse distribution holds 224 entries (top_k 40), and the trunk and the
MTP head can favour different groups, so drafts are rejected and the
correction is drawn from the residual.  The device chain runs those lists
over several 64-entry blocks; its tokens (draws, acceptances, corrections)
equal the oracle's under the same seeded stream."""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096, max_seq=256,
           rope_theta=1e6, eps=1e-6)


def _two_group_model():
    from cmf_amd import synth
    sm = synth.synth_model(CFG, seed=11, norm_noise=0.1, sigma=0.05)
    lm = sm["lm_head"]
    q = lm["q"].reshape(CFG["vocab"], CFG["hidden"])
    q[1:2048] = q[0]
    q[2049:] = q[2048]
    lm["row_scale"][1:2048] = lm["row_scale"][0]
    lm["row_scale"][2049:] = lm["row_scale"][2048]
    return sm


@pytest.mark.parametrize("k", [1, 4])
def test_sampled_decode_over_tied_logits_equals_oracle(gpu, k):
    import cmf_amd
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = _two_group_model()
    g = Model(sm)
    prompt = synth.ids(12, 10, CFG["vocab"])
    sg = cmf_amd.SamplerConfig(temperature=1.0, top_k=40, top_p=1.0, min_p=0.0, repetition_penalty=1.0)
    so = orc.SamplerCfg(1.0, 1.0, 40, 1.0, 0.0, 0.0)
    g.prefill(prompt)
    gt, gst = g.decode(30, sampler=sg, seed=5, spec=True, k=k)
    ot, ost = orc.OracleModel(sm).generate(prompt, 30, spec=True, k=k, sampler=so, seed=5)
    g.free()
    print(f"k={k}: gpu {gt.tolist()} accepted {gst.accepted}/{gst.drafted}", flush=True)
    print(f"k={k}: cpu {ot.tolist()} accepted {ost.accepted}", flush=True)
    n = min(len(gt), len(ot))
    assert n >= 30
    assert gt[:n].tolist() == ot[:n].tolist()
    assert gst.accepted == ost.accepted
    # the draws come from the 224-entry lists of both groups
    assert max(gt.tolist()) >= 2048 or min(gt.tolist()) < 224
