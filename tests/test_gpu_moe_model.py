"""A decoder with routed-expert (Qwen3-MoE) FFN blocks in the device model:
the router GEMV over the block's normed rows, device routing and the grouped
expert GEMVs, h += their weighted sum (moe_ffn, pipeline.rs:10868-10915;
GraphFfn::Moe, gpu.rs:1248-1361), in the verify forward, the decode loop
and the chunked prefill.  Against the CPU oracle: hidden rows and logits
within relative L2 1e-4, speculative and plain decode tokens equal."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=3, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096,
           max_seq=320, rope_theta=1e6, eps=1e-6)
MOE = dict(n_experts=16, top_k=4, inter=128, layers=[0, 2])


@pytest.fixture(scope="module", params=["q4t-f16router", "q8-q8router"])
def moe_model(gpu, request):
    """q4t experts with an f16 router (the reference converter's choice,
    convert.rs force_f16), q8 experts with a q8 router"""
    from cmf_amd import synth
    from cmf_amd.model import Model
    dt = synth.DT_Q4T if request.param.startswith("q4t") else synth.DT_Q8ROW
    moe = dict(MOE, router_dtype="f16" if "f16" in request.param else "q8")
    sm = synth.synth_model(CFG, seed=31, norm_noise=0.3, sigma=0.08, moe=moe, ffn_dtype=dt)
    g = Model(sm)
    yield sm, g
    g.free()


def test_moe_forward_batch_matches_oracle(moe_model):
    sm, g = moe_model
    from cmf_amd import synth
    ids = synth.ids(33, 9, CFG["vocab"])
    hid, lg = g.forward_batch(ids, 0)
    o = orc.OracleModel(sm)
    for i, t in enumerate(ids):
        h = o.forward(int(t), i)
        e = rel_l2(hid[i], h)
        print(f"row {i}: hidden rel {e:.2e}", flush=True)
        assert e < 1e-4
        assert rel_l2(lg[i], o.logits(h)) < 1e-4


@pytest.mark.parametrize("spec", [True, False])
def test_moe_decode_tokens_equal_oracle(moe_model, spec):
    """prefill (the MoE blocks of the chunk in 16-row batches) + decode"""
    sm, g = moe_model
    from cmf_amd import synth
    prompt = synth.ids(34, 40, CFG["vocab"])
    g.prefill(prompt)
    gt, gst = g.decode(20, spec=spec, k=4)
    ot, ost = orc.OracleModel(sm).generate(prompt, 20, spec=spec, k=4)
    print(f"spec={spec}: gpu {gt.tolist()} | oracle {ot.tolist()}", flush=True)
    assert gt.tolist() == ot.tolist()
    assert gst.accepted == ost.accepted
    # the prefill's MoE blocks: trunk KV of the last layer (after two MoE blocks)
    g.prefill(prompt)
    o = orc.OracleModel(sm)
    o.prefill(prompt)
    k, v = g.kv_export(2, 40)
    rk, rv = o.kv(2)
    assert rel_l2(k, rk) < 1e-4 and rel_l2(v, rv) < 1e-4
