"""Writes tests/golden/oracle_golden.npz: small seeded input/output vectors of
the CPU oracle (dequantization, exact-contract matmuls, the sparse sampling
chain, SplitMix64 streams and tiny-model greedy / sampled decodes).

The reference ships no golden vectors for this path and cannot be built here,
so these fixtures lock the oracle's own outputs after the oracle was pinned by
the known-answer and brute-force tests (tests/test_oracle_*.py): any later
change to the oracle that moves a result shows up as a fixture mismatch.

    python tests/golden/make_golden.py
"""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_golden.npz")

TINY = dict(n_layers=2, hidden=128, n_heads=4, n_kv=2, head_dim=32, inter=256, vocab=512, max_seq=64,
            rope_theta=1e6, eps=1e-6)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class Rng(C.Structure):
    _fields_ = [("state", C.c_uint64)]


def inputs():
    from cmf_amd import synth
    t = {"q8": synth.q8_uniform(21, 24, 192), "q4t": synth.q4t_uniform(22, 16, 256),
         "q4tp": synth.q4tp_uniform(23, 16, 320)}
    xs = {k: synth.normal(30 + i, 3 * v["cols"]).reshape(3, v["cols"]) for i, (k, v) in enumerate(t.items())}
    return t, xs


def compute():
    from cmf_amd import synth
    from oracle import oracle as orc
    L = orc.lib()
    t, xs = inputs()
    g = {}
    for k, v in t.items():
        if v["bytes"] is not None:
            g[f"{k}_payload"] = v["bytes"]
        else:
            g[f"{k}_q"], g[f"{k}_row_scale"] = v["q"], v["row_scale"]
        g[f"{k}_x"] = xs[k]
        g[f"{k}_y"] = orc.matmat(v, xs[k], threads=2)
        g[f"{k}_y_a8w8"] = orc.matmat(v, xs[k][:1], threads=2, a8w8=True)
    out = np.empty(16 * 320, np.float32)
    L.or_dequant_q4tp(_p(np.ascontiguousarray(t["q4tp"]["bytes"])), 16, 320, _p(out))
    g["q4tp_dequant"] = out.reshape(16, 320)
    r = Rng(1234)
    g["splitmix_1234"] = np.array([L.or_rng_next_u64(C.byref(r)) for _ in range(8)], np.uint64)
    logits = synth.normal(40, 2000, 2.0)
    cfg = orc.SamplerCfg(0.8, 0.9, 40, 1.0, 0.05, 0.0)
    ids = np.empty(4 * 256 + 64, np.uint32)
    pr = np.empty(4 * 256 + 64, np.float32)
    m = L.or_sparse_distribution(_p(logits), 2000, C.byref(cfg), None, 0, _p(ids), _p(pr))
    g["chain_logits"], g["chain_ids"], g["chain_p"] = logits, ids[:m].copy(), pr[:m].copy()
    sm = synth.synth_model(TINY, seed=3, norm_noise=0.1, sigma=0.05)
    prompt = synth.ids(5, 9, TINY["vocab"])
    g["tiny_prompt"] = prompt
    g["tiny_greedy"], _ = orc.OracleModel(sm, threads=2).generate(prompt, 16, spec=True, k=3)
    g["tiny_sampled"], _ = orc.OracleModel(sm, threads=2).generate(prompt, 16, spec=True, k=3, sampler=cfg, seed=7)
    return g


if __name__ == "__main__":
    np.savez_compressed(OUT, **compute())
    print(OUT, os.path.getsize(OUT), "bytes")
