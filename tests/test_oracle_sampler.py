"""CPU pins of the oracle's sampler: SplitMix64 against Vigna's published
outputs, the argmax tie rule, the sparse top-k/top-p/min-p chain against a
dense brute force, and speculative acceptance against the theorem it
implements (the emitted token is distributed as the target p)."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as orc


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


Rng = orc.Rng


def test_splitmix64_published_outputs():
    L = orc.lib()
    r = Rng(0)
    assert [L.or_rng_next_u64(C.byref(r)) for _ in range(3)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    r = Rng(42)
    assert [L.or_rng_next_u64(C.byref(r)) for _ in range(3)] == [
        0xBDD732262FEB6E95, 0x28EFE333B266F103, 0x47526757130F9F52]
    r = Rng(0)
    f = [L.or_rng_next_f32(C.byref(r)) for _ in range(3)]
    assert np.allclose(f, [0.8833108, 0.43152797, 0.026433766], rtol=0, atol=1e-7)


def test_argmax_ties_to_highest_index():
    """sampler.rs:1130-1154"""
    L = orc.lib()
    v = np.array([1.0, 3.0, -2.0, 3.0, 0.5, 3.0, 2.9], dtype=np.float32)
    assert L.or_argmax(_p(v), len(v)) == 5
    v = np.array([-np.inf, -1.0, -1.0], dtype=np.float32)
    assert L.or_argmax(_p(v), len(v)) == 2


def _dense_chain(logits, t, top_k, top_p, min_p):
    """brute force in f64 over the whole vocabulary"""
    z = logits.astype(np.float64) / t
    p = np.exp(z - z.max())
    p /= p.sum()
    order = np.argsort(-logits.astype(np.float64), kind="stable")[:top_k]
    keep, cum = [], 0.0
    for i in order:
        if min_p > 0 and p[i] / p.max() < min_p:
            continue
        keep.append(i)
        cum += p[i]
        if 0 < top_p < 1 and cum >= top_p:
            break
    keep = np.array(sorted(keep))
    q = p[keep] / p[keep].sum()
    return keep, q


@pytest.mark.parametrize("seed,t,k,tp,mp", [(1, 0.8, 40, 0.9, 0.05), (2, 1.0, 5, 1.0, 0.0),
                                            (3, 0.5, 64, 0.7, 0.0), (4, 1.3, 20, 0.95, 0.1)])
def test_sparse_chain_matches_dense_bruteforce(seed, t, k, tp, mp):
    L = orc.lib()
    rng = np.random.default_rng(seed)
    n = 3000
    logits = (rng.standard_normal(n) * 2.0).astype(np.float32)
    cfg = orc.SamplerCfg(t, tp, k, 1.0, mp, 0.0)
    ids = np.empty(4 * 256 + 64, dtype=np.uint32)
    pr = np.empty(4 * 256 + 64, dtype=np.float32)
    m = L.or_sparse_distribution(_p(logits), n, C.byref(cfg), None, 0, _p(ids), _p(pr))
    want_ids, want_p = _dense_chain(logits, t, k, tp, mp)
    assert ids[:m].tolist() == want_ids.tolist()
    assert np.allclose(pr[:m], want_p, rtol=2e-5, atol=1e-7)


def _emp_accept(p_ids, p_pr, q_ids, q_pr, trials, seed):
    """tally of emitted tokens: d ~ q, then accept d or take the correction"""
    L = orc.lib()
    r = Rng(seed)
    pid, pp = np.asarray(p_ids, np.uint32), np.asarray(p_pr, np.float32)
    qid, qp = np.asarray(q_ids, np.uint32), np.asarray(q_pr, np.float32)
    counts = {}
    for _ in range(trials):
        d = L.or_draw_sparse(_p(qid), _p(qp), len(qid), C.byref(r))
        res = L.or_spec_accept_sparse(_p(pid), _p(pp), len(pid), _p(qid), _p(qp), len(qid), d, C.byref(r))
        tok = d if res < 0 else res
        counts[tok] = counts.get(tok, 0) + 1
    return counts


def test_spec_accept_emits_target_distribution():
    """sampler.rs:1285-1337: empirical L1 < 0.01 over 4e5 trials, and no
    token outside supp(p)"""
    p_ids, p_pr = [2, 5, 7, 11], [0.1, 0.4, 0.3, 0.2]
    q_ids, q_pr = [1, 2, 5, 11], [0.3, 0.3, 0.2, 0.2]
    trials = 400000
    counts = _emp_accept(p_ids, p_pr, q_ids, q_pr, trials, seed=99)
    assert set(counts) <= set(p_ids)
    emp = np.array([counts.get(i, 0) / trials for i in p_ids])
    assert np.abs(emp - np.array(p_pr)).sum() < 0.01


def test_spec_accept_identical_distributions_always_accept():
    """pipeline.rs:11567-11587 (constant logits): p == q accepts every draft"""
    L = orc.lib()
    ids = np.array([3, 4, 9], np.uint32)
    pr = np.array([0.2, 0.5, 0.3], np.float32)
    r = Rng(5)
    for _ in range(2000):
        d = L.or_draw_sparse(_p(ids), _p(pr), 3, C.byref(r))
        assert L.or_spec_accept_sparse(_p(ids), _p(pr), 3, _p(ids), _p(pr), 3, d, C.byref(r)) < 0


def test_spec_accept_dense_target_distribution():
    L = orc.lib()
    n = 6
    p = np.array([0.05, 0.25, 0.0, 0.3, 0.15, 0.25], np.float32)
    q = np.array([0.3, 0.1, 0.2, 0.1, 0.2, 0.1], np.float32)
    r = Rng(11)
    trials = 200000
    cnt = np.zeros(n)
    for _ in range(trials):
        d = L.or_categorical(_p(q), n, L.or_rng_next_f32(C.byref(r)))
        res = L.or_spec_accept_dense(_p(p), _p(q), n, d, C.byref(r))
        cnt[d if res < 0 else res] += 1
    assert cnt[2] == 0
    assert np.abs(cnt / trials - p).sum() < 0.012


def _ties_chain(logits, t, top_k, top_p, min_p):
    """brute force of par_topk's tie rule (sampler.rs:515-600): every entry
    >= the k-th largest value, the first 4 k + 64 of them in index order,
    then the chain of sparse_distribution_into (sampler.rs:440-514) in f64"""
    z = logits.astype(np.float64)
    kth = np.sort(z)[::-1][top_k - 1]
    cand = [i for i in range(len(z)) if z[i] >= kth][: 4 * top_k + 64]
    cand.sort(key=lambda i: (-z[i], i))
    e = np.exp((z - z.max()) / t)
    keep, cum = [], 0.0
    for i in cand:
        if min_p > 0 and e[i] < min_p:
            continue
        keep.append(i)
        cum += e[i] / e.sum()
        if 0 < top_p < 1 and cum >= top_p:
            break
    keep = np.array(sorted(keep))
    q = e[keep] / e[keep].sum()
    return keep, q


@pytest.mark.parametrize("levels,k,tp", [(8, 40, 1.0), (8, 40, 0.9), (64, 20, 1.0), (2, 10, 1.0), (2, 64, 0.5)])
def test_sparse_chain_keeps_ties_at_the_kth_value(levels, k, tp):
    """logits on a coarse grid: every entry tied with the k-th value stays a
    candidate (levels 8, 64: tens to hundreds of ties), at most 4 k + 64 of
    them in index order (levels 2: thousands tied at the top)"""
    L = orc.lib()
    rng = np.random.default_rng(100 + levels)
    n = 20000
    logits = np.floor(rng.standard_normal(n) * (levels / 8)).astype(np.float32)
    cfg = orc.SamplerCfg(1.0, tp, k, 1.0, 0.0, 0.0)
    ids = np.empty(4 * 256 + 64, dtype=np.uint32)
    pr = np.empty(4 * 256 + 64, dtype=np.float32)
    m = L.or_sparse_distribution(_p(logits), n, C.byref(cfg), None, 0, _p(ids), _p(pr))
    want_ids, want_p = _ties_chain(logits, 1.0, k, tp, 0.0)
    kth = np.sort(logits)[::-1][k - 1]
    assert (logits >= kth).sum() > k  # ties past the k-th place exist
    assert ids[:m].tolist() == want_ids.tolist()
    assert np.allclose(pr[:m], want_p, rtol=2e-5, atol=1e-7)
