"""CPU pins of the oracle's MoE routing and expert FFN (moe_route,
pipeline.rs:10780-10841; moe_ffn_cpu, pipeline.rs:10997-11045) against the
tie rule, closed-form softmax / top-k in f64 and an f64 brute force over the
dequantized experts."""
import numpy as np
import pytest

from cmf_amd import synth
from oracle import oracle as orc

DT_Q8ROW, DT_Q4T, DT_Q4TP = 3, 11, 15


def _route_f64(lg, k, norm=True, scaling=1.0):
    lg = np.asarray(lg, np.float64)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    order = np.lexsort((np.arange(len(p)), -p))[:k]  # descending p, lower index first
    ws = p[order].sum() / scaling if norm else 1.0 / scaling
    return order, p[order] / ws


def test_route_ties_lower_index_first():
    idx, w = orc.moe_route([1.0, 3.0, 3.0, 0.0, 3.0, -1.0], 2)
    assert idx.tolist() == [1, 2]
    assert w.tolist() == [0.5, 0.5]
    idx, _ = orc.moe_route([0.0, 0.0, 0.0, 0.0], 4)
    assert idx.tolist() == [0, 1, 2, 3]


@pytest.mark.parametrize("norm,scaling", [(True, 1.0), (True, 2.5), (False, 1.0), (False, 16.0)])
def test_route_closed_form(norm, scaling):
    rng = np.random.default_rng(5)
    for _ in range(20):
        lg = rng.standard_normal(128).astype(np.float32) * 2
        idx, w = orc.moe_route(lg, 8, norm, scaling)
        ridx, rw = _route_f64(lg, 8, norm, scaling)
        assert idx.tolist() == ridx.tolist()
        np.testing.assert_allclose(w, rw, rtol=2e-6)
        if norm:
            assert abs(float(w.astype(np.float64).sum()) - scaling) < 1e-5 * scaling


def test_route_all_experts():
    lg = np.array([0.3, -1.0, 2.0, 0.3, 5.0], np.float32)
    idx, w = orc.moe_route(lg, 5)
    assert idx.tolist() == [4, 2, 0, 3, 1]
    assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6


def _experts(ne, hidden, inter, dt_gu, dt_down, seed):
    mk = {DT_Q4T: lambda s, r, c: synth.q4t_uniform(s, r, c), DT_Q8ROW: lambda s, r, c: synth.q8_uniform(s, r, c),
          DT_Q4TP: lambda s, r, c: synth.q4tp_uniform(s, r, c)}
    return [{"gate": mk[dt_gu](seed + 3 * e, inter, hidden), "up": mk[dt_gu](seed + 3 * e + 1, inter, hidden),
             "down": mk[dt_down](seed + 3 * e + 2, hidden, inter)} for e in range(ne)]


@pytest.mark.parametrize("dt_gu,dt_down", [(DT_Q4T, DT_Q4T), (DT_Q4TP, DT_Q4TP), (DT_Q8ROW, DT_Q4T)])
def test_moe_ffn_brute_force(dt_gu, dt_down):
    ne, H, I, k = 6, 64, 96, 3
    ex = _experts(ne, H, I, dt_gu, dt_down, 100 + dt_gu)
    rng = np.random.default_rng(dt_gu)
    x = rng.standard_normal(H).astype(np.float32)
    lg = rng.standard_normal(ne).astype(np.float32)
    got = orc.moe_ffn(ex, k, lg, x)
    idx, w = _route_f64(lg, k)
    ref = np.zeros(H)
    mag = np.zeros(H)
    for e, wi in zip(idx, w):
        G, U, D = (synth.dequant(ex[e][n]).astype(np.float64) for n in ("gate", "up", "down"))
        g, u = G @ x, U @ x
        h = g / (1 + np.exp(-g)) * u
        ref += wi * (D @ h)
        mag += abs(wi) * (np.abs(D) @ np.abs(h))
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-7)
