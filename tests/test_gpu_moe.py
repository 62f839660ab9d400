"""GPU parity of the MoE FFN layer (BASELINE config 5 and smaller cases)
against the CPU oracle (moe_route + moe_ffn_cpu's serial expert loop).
Routing (expert ids) must be identical; outputs within relative L2 1e-3
(observed ~1e-7); weights within 1e-6 relative."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DT_Q8ROW, DT_Q4T, DT_Q4TP = 3, 11, 15
TOL = 1e-3


def _experts(ne, hidden, inter, dt_gu, dt_down, seed):
    from cmf_amd import synth
    mk = {DT_Q4T: synth.q4t_uniform, DT_Q8ROW: synth.q8_uniform, DT_Q4TP: synth.q4tp_uniform}
    return [{"gate": mk[dt_gu](seed + 3 * e, inter, hidden), "up": mk[dt_gu](seed + 3 * e + 1, inter, hidden),
             "down": mk[dt_down](seed + 3 * e + 2, hidden, inter)} for e in range(ne)]


def _run(gpu, ne, H, I, k, b, dt_gu=DT_Q4T, dt_down=DT_Q4T, seed=7, norm=True, scaling=1.0, bias=None):
    from cmf_amd import synth
    from cmf_amd.moe import MoE
    ex = _experts(ne, H, I, dt_gu, dt_down, seed)
    x = synth.normal(seed + 1000, b * H).reshape(b, H)
    lg = synth.normal(seed + 2000, b * ne).reshape(b, ne)
    if bias is not None:
        lg = (lg + np.asarray(bias, np.float32)).astype(np.float32)
    moe = MoE(ne, H, I, k, ex, norm_topk=norm, routed_scaling=scaling)
    out, idx, w = moe.ffn(x, lg)
    for t in range(b):
        ridx, rw = orc.moe_route(lg[t], k, norm, scaling)
        assert idx[t].tolist() == ridx.tolist(), f"token {t}: routing differs"
        np.testing.assert_allclose(w[t], rw, rtol=1e-6)
        ref = orc.moe_ffn(ex, k, lg[t], x[t], norm, scaling, threads=16)
        err = rel_l2(out[t], ref)
        print(f"ne={ne} H={H} I={I} k={k} b={b} token {t}: rel-L2 {err:.3e}", flush=True)
        assert err < TOL
    return moe, ex, x


@pytest.mark.parametrize("b", [1, 3, 5, 16])
def test_moe_small(gpu, b):
    _run(gpu, 8, 256, 128, 2, b)


@pytest.mark.parametrize("dt_gu,dt_down", [(DT_Q4TP, DT_Q4TP), (DT_Q8ROW, DT_Q4T), (DT_Q8ROW, DT_Q8ROW)])
def test_moe_codecs(gpu, dt_gu, dt_down):
    _run(gpu, 8, 256, 192, 3, 5, dt_gu, dt_down, seed=11)


def test_moe_scaling_no_norm(gpu):
    _run(gpu, 16, 128, 64, 4, 4, norm=False, scaling=2.5)


@pytest.mark.parametrize("ne", [64, 200, 300])
def test_moe_expert_counts(gpu, ne):
    """the routing's register layouts: 64 experts (one column per lane), up
    to 256 (four), more (sixteen), with ragged last columns"""
    _run(gpu, ne, 128, 64, 6, 3, seed=41)


@pytest.mark.parametrize("k", [1, 16])
def test_moe_top_k_extremes(gpu, k):
    """one rank per token, and 16 ranks (the per-token down launch's
    1024-thread workgroup)"""
    _run(gpu, 32, 128, 64, k, 3, seed=43)


@pytest.mark.parametrize("inter", [1024, 1152])
def test_moe_inter_sizes(gpu, inter):
    """FFN 1024: the largest per-token down instance (8 K steps); 1152: past
    it, the per-job down kernel and the combine"""
    _run(gpu, 16, 256, inter, 4, 3, seed=47)


def test_moe_all_experts_selected(gpu):
    """top_k = n_experts: every job runs, every token uses every expert."""
    _run(gpu, 4, 128, 64, 4, 5)


def test_moe_config5(gpu):
    """hidden 2048, 128 experts top-8, expert FFN 768,
    q4t experts, M=5 verify tokens."""
    _run(gpu, 128, 2048, 768, 8, 5, seed=5)


def test_moe_block_caller_routed(gpu):
    """moe_block (gpu.rs:2482): given experts and weights, including a
    repeated expert."""
    from cmf_amd import synth
    moe, ex, x = _run(gpu, 8, 256, 128, 4, 1, seed=21)
    experts = np.array([5, 1, 5, 0], np.int32)
    weights = np.array([0.5, -0.25, 0.125, 2.0], np.float32)
    got = moe.block(x[0], experts, weights)
    ref = np.zeros(256, np.float32)
    for e, wi in zip(experts, weights):
        one = np.full(8, -1e30, np.float32)
        one[e] = 0.0  # route to e alone with weight 1
        ref += wi * orc.moe_ffn(ex, 1, one, x[0])
    assert rel_l2(got, ref) < TOL


def test_moe_every_token_same_experts(gpu):
    """b = 8 tokens that all pick experts 3 and 5 (router bias): each job
    lists all eight tokens, the most the per-job-token kernels hold."""
    bias = np.zeros(8, np.float32)
    bias[[3, 5]] = 50.0
    _run(gpu, 8, 256, 128, 2, 8, seed=31, bias=bias)


_GROUPED_CHILD = r"""
import sys
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import cmf_amd as cmf
cmf.init(0)
import test_gpu_moe as t
t._run(None, 8, 256, 128, 2, 5)
t._run(None, 128, 2048, 768, 8, 5, seed=5)
print("ok")
"""


_PERJOB_CHILD = r"""
import sys
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import cmf_amd as cmf
cmf.init(0)
import test_gpu_moe as t
t._run(None, 8, 256, 128, 2, 5)
t._run(None, 128, 2048, 768, 8, 5, seed=5)
print("ok")
"""


def test_moe_per_job_down_path(gpu):
    """CMF_MOE_DOWN_TOK=0 (child process): routed batches through the
    per-job down kernel and the separate combine (the path of caller-routed
    jobs) instead of the per-token down + combine launch"""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, CMF_MOE_DOWN_TOK="0")
    r = subprocess.run([sys.executable, "-c", _PERJOB_CHILD, root], env=env, capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().splitlines()[-1] == "ok"


def test_moe_grouped_path(gpu):
    """CMF_MOE_GATHER=0 (child process): q4t experts at b <= 8 through the
    grouped GEMVs over all rows, the path of the other codecs and of larger
    batches, on the interleaved gate|up rows."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, CMF_MOE_GATHER="0")
    r = subprocess.run([sys.executable, "-c", _GROUPED_CHILD, root], env=env, capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and r.stdout.strip().splitlines()[-1] == "ok"
