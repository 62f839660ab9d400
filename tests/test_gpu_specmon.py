"""The decode loop's plain arm and the speculation monitor on the GPU.

- Plain steps replayed from a captured graph (decode_rounds(n > 1,
  spec=False)) give the oracle's plain-decode tokens, greedy and sampled.
- cmf_decode with spec = "auto" runs the reference's speculation monitor
  (SpecMon, pipeline.rs:661-694, with the trial of :2537, :2655-2760,
  :3181-3230): on a model whose MTP head is not accepted it times five
  speculative rounds and eight plain tokens, finds that a round does not
  pay (tokens_per_round * plain_ms <= round_ms * 1.03) and decodes the rest
  plain, and its tokens still equal the oracle's greedy tokens (greedy
  speculation emits the plain tokens, pipeline.rs:11543)."""
import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=4, n_kv=2, head_dim=128, inter=512, vocab=4096,
             max_seq=256, rope_theta=1e6, eps=1e-6)


@pytest.fixture(scope="module")
def small(gpu):
    from cmf_amd import synth
    from cmf_amd.model import Model
    sm = synth.synth_model(SMALL, seed=5, norm_noise=0.1, sigma=0.05)
    g = Model(sm)
    yield sm, g
    g.free()


@pytest.mark.parametrize("sampling", [False, True])
def test_captured_plain_steps_equal_oracle(small, sampling):
    """decode_rounds(n > 1, spec=False) replays one captured plain step;
    two calls in a row (the second replaying the kept graph)"""
    sm, g = small
    import cmf_amd
    from cmf_amd import synth
    prompt = synth.ids(29, 18, SMALL["vocab"])
    sg = cmf_amd.SamplerConfig(temperature=0.8, repetition_penalty=1.0) if sampling else None
    so = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0) if sampling else None
    g.prefill(prompt)
    g.decode_begin(sampler=sg, seed=91)
    g.decode_rounds(6, spec=False)
    g.decode_rounds(7, spec=False)
    got = g.tokens()
    ot, _ = orc.OracleModel(sm).generate(prompt, len(got) + 2, spec=False, sampler=so, seed=91)
    print("gpu", got.tolist(), flush=True)
    print("cpu", ot.tolist(), flush=True)
    assert len(got) == 13  # one token per plain step
    assert got.tolist() == ot[:len(got)].tolist()


def test_monitor_switches_unprofitable_speculation_off(small):
    sm, g = small
    from cmf_amd import synth
    prompt = synth.ids(31, 16, SMALL["vocab"])
    g.prefill(prompt)
    toks, st = g.decode(48, spec="auto", k=4)
    mon = g.monitor()
    print(f"tokens {len(toks)} accepted {st.accepted}/{st.drafted}; monitor {mon.phase_name}: "
          f"{mon.tokens:.2f} tok/round in {mon.round_ms:.3f} ms vs plain {mon.plain_ms:.3f} ms/tok; "
          f"{mon.spec_rounds} rounds, {mon.plain_steps} plain steps", flush=True)
    assert mon.spec_rounds == 5          # the trial's five rounds, then plain
    assert mon.plain_ms > 0.0 and mon.round_ms > 0.0
    assert mon.tokens * mon.plain_ms <= mon.round_ms * 1.03
    assert mon.phase_name == "plain" and mon.recheck_at > 48
    assert mon.plain_steps >= 48 - 5 * 5 - 1
    ot, _ = orc.OracleModel(sm).generate(prompt, 48, spec=False)
    assert toks[:48].tolist() == ot[:48].tolist()
