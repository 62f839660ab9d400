"""GPU parity of the dequant GEMV / skinny GEMM family against the CPU oracle
(the reference's exact contract, qtensor.rs).  Tolerance: relative L2 1e-3
(BASELINE north star); observed errors are ~1e-6."""
import numpy as np
import pytest

from conftest import rel_l2
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _x(seed, b, cols):
    from cmf_amd import synth
    return synth.normal(seed, b * cols).reshape(b, cols)


def _check(gpu, t, xs, tol=TOL):
    w = gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
    got = gpu.matmul(w, xs)
    ref = orc.matmat(t, xs, threads=16)
    err = rel_l2(got, ref)
    print(f"dtype {t['dtype']} {t['rows']}x{t['cols']} b={xs.shape[0]}: rel-L2 {err:.3e}", flush=True)
    assert err < tol
    # every row and batch element individually
    for i in range(xs.shape[0]):
        assert rel_l2(got[i], ref[i]) < tol
    return got, ref


def test_q8_config1(gpu):
    from cmf_amd import synth
    t = synth.q8_uniform(11, 4096, 4096)
    _check(gpu, t, _x(12, 1, 4096))


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 16])
def test_q8_batches(gpu, m):
    from cmf_amd import synth
    t = synth.q8_normal(21 + m, 1024, 2048)
    _check(gpu, t, _x(22 + m, m, 2048))


@pytest.mark.parametrize("shape", [(12288, 4096), (4096, 12288)])
@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_q4t_config2(gpu, shape, m):
    from cmf_amd import synth
    t = synth.q4t_uniform(31 + shape[0], shape[0], shape[1])
    _check(gpu, t, _x(32 + m, m, shape[1]))


def test_q8_config5_projection(gpu):
    """BASELINE config 5's q8 4096x2048 attention projection at M=5"""
    from cmf_amd import synth
    t = synth.q8_uniform(5003, 4096, 2048)
    _check(gpu, t, _x(5004, 5, 2048))


@pytest.mark.parametrize("shape", [(12288, 4096), (4096, 12288)])
def test_q4tp_config3(gpu, shape):
    from cmf_amd import synth
    t = synth.q4tp_uniform(41 + shape[0], shape[0], shape[1])
    _check(gpu, t, _x(42, 5, shape[1]))


@pytest.mark.parametrize("m", [1, 3, 7, 13])
def test_q4tp_batches_small(gpu, m):
    from cmf_amd import synth
    t = synth.q4tp_uniform(51 + m, 512, 1024)
    _check(gpu, t, _x(52 + m, m, 1024))


def test_ragged_shapes(gpu):
    """rows not a multiple of 16, cols not a multiple of the K step"""
    from cmf_amd import synth
    _check(gpu, synth.q8_normal(61, 37, 80), _x(62, 3, 80))
    _check(gpu, synth.q4t_uniform(63, 45, 96), _x(64, 2, 96))
    _check(gpu, synth.q4tp_uniform(65, 19, 160), _x(66, 4, 160))
    _check(gpu, synth.q4t_uniform(67, 1, 32), _x(68, 1, 32))


@pytest.mark.parametrize("cols", [64, 448, 1024, 2048, 2112, 4096, 4160, 8192, 12288, 16384])
def test_m1_kernel_instances(gpu, cols):
    """M = 1 runs the per-wave operand-slice kernels (k_gemv_q8_m1 over a
    prepared operand; q4t through the seam: k_gemv_q4t_m1x staging its own
    operand up to 64 steps, k_gemv_q4t_m1 beyond); every instance size (q8: 1..192 K steps
    of 64 columns, q4t: 1..128 steps of 128 columns), ragged steps (4160 =
    65 q8 chunks, 32.5 q4t groups) and ragged rows"""
    from cmf_amd import synth
    _check(gpu, synth.q8_normal(81 + cols, 77, cols), _x(82 + cols, 1, cols))
    _check(gpu, synth.q4t_uniform(83 + cols, 93, cols), _x(84 + cols, 1, cols))


def _gemv_rows(gpu, w, x, rows, fused):
    """y = W x from the f32 row x on the device: fused=1 the kernel stages its
    operand itself, fused=0 the producer launch + the prepared-operand GEMV"""
    import ctypes as C
    dx, dy = gpu.DevBuf(x.nbytes), gpu.DevBuf(rows * 4)
    dx.upload(x)
    arr = (C.c_void_p * 1)(w.h)
    ms = C.c_float()
    gpu.check(gpu.lib().cmf_time_gemv_rows(arr, 1, dx.p, x.shape[-1], None, 1, dy.p, rows, fused, 0, 1,
                                            C.byref(ms)))
    y = dy.download((1, rows))
    dx.free()
    dy.free()
    return y


@pytest.mark.parametrize("cols", [64, 448, 1024, 2048, 4160, 8192])
def test_m1_staged_from_rows(gpu, cols):
    """q4t M = 1 from an f32 row: the kernel that stages its own operand
    slices (k_gemv_q4t_m1x, K <= 8192) writes the producer's planes and
    biases, so its result equals the prepared-operand kernel's bit for bit
    (both use the same waves x steps instance),
    and the oracle's within the bar; also with a row max in the last step
    (the workgroup-wide max must see every wave's columns)"""
    from cmf_amd import synth
    t = synth.q4t_uniform(91 + cols, 93, cols)
    w = gpu.Weight(t["dtype"], 93, cols, payload=t["bytes"])
    for seed in (0, 1):
        x = _x(92 + cols + seed, 1, cols)
        if seed:
            x[0, cols - 3] = 40.0  # the row max in the last columns
        fused = _gemv_rows(gpu, w, x, 93, 1)
        prep = _gemv_rows(gpu, w, x, 93, 0)
        ref = orc.matmat(t, x, threads=16)
        err = rel_l2(fused, ref)
        print(f"q4t 93x{cols} staged-from-rows: rel-L2 {err:.3e}", flush=True)
        assert err < TOL
        assert np.array_equal(fused.view(np.uint32), prep.view(np.uint32))
    w.free()


def test_large_batch_split(gpu):
    """q8 with b > 16: the int8 MFMA GEMM (37 rows: one ragged 64-row tile)"""
    from cmf_amd import synth
    _check(gpu, synth.q8_normal(71, 256, 512), _x(72, 37, 512))


@pytest.mark.parametrize("b", [17, 64, 130])
@pytest.mark.parametrize("fmt", ["q4t", "q4tp", "q8"])
def test_gemm_large_batch(gpu, fmt, b):
    """b > 16: the MFMA GEMM (ragged batch tiles and row blocks; q8 with an
    odd count of 64-column chunks: 640 columns = 10, 704 = 11)"""
    from cmf_amd import synth
    if fmt == "q8":
        _check(gpu, synth.q8_uniform(73 + b, 272, 704), _x(74 + b, b, 704))
        _check(gpu, synth.q8_uniform(75 + b, 4096, 1024), _x(76 + b, b, 1024))
        return
    mk = synth.q4t_uniform if fmt == "q4t" else synth.q4tp_uniform
    _check(gpu, mk(73 + b, 272, 640), _x(74 + b, b, 640))


@pytest.mark.parametrize("shape", [(12288, 4096), (4096, 12288)])
def test_gemm_config2_prefill(gpu, shape):
    """config 2 shapes at a prefill-sized batch (256 rows)"""
    from cmf_amd import synth
    _check(gpu, synth.q4t_uniform(75, *shape), _x(76, 256, shape[1]))


def test_q8_matvec_range(gpu):
    from cmf_amd import synth
    t = synth.q8_normal(81, 300, 256)
    w = gpu.Weight(t["dtype"], 300, 256, q=t["q"], row_scale=t["row_scale"])
    x = _x(82, 1, 256)
    out = np.zeros((1, 37), np.float32)
    assert gpu.q8_matvec_range(w, 5, x, 37, 256, out)
    ref = orc.matmat(t, x)[:, 5:42]
    assert rel_l2(out, ref) < TOL
    # the caller's row scales replace the stored ones (gpu.rs:1104 passes
    # row_scale[row0..] with every call)
    rs = (t["row_scale"][5:42] * np.linspace(0.5, 2.0, 37)).astype(np.float32)
    out2 = np.zeros((1, 37), np.float32)
    assert gpu.q8_matvec_range(w, 5, x, 37, 256, out2, row_scale=rs)
    t2 = dict(t, row_scale=t["row_scale"].copy())
    t2["row_scale"][5:42] = rs
    ref2 = orc.matmat(t2, x)[:, 5:42]
    print(f"caller scales: rel-L2 {rel_l2(out2, ref2):.2e}", flush=True)
    assert rel_l2(out2, ref2) < TOL and rel_l2(out2, ref) > 0.1
    # and the stored ones are untouched
    out3 = np.zeros((1, 37), np.float32)
    assert gpu.q8_matvec_range(w, 5, x, 37, 256, out3)
    assert rel_l2(out3, ref) < TOL
    out4 = np.zeros((2, 300), np.float32)
    rs_all = (t["row_scale"] * 1.5).astype(np.float32)
    x2 = _x(83, 2, 256)
    assert gpu.q8_matmat(w, x2, 2, 300, 256, out4, row_scale=rs_all)
    assert rel_l2(out4, orc.matmat(dict(t, row_scale=rs_all), x2)) < TOL


def _silu(x):
    x = x.astype(np.float32)
    with np.errstate(over="ignore"):  # exp(-x) = inf for very negative x: silu -> -0
        return (x / (np.float32(1) + np.exp(-x))).astype(np.float32)


@pytest.mark.parametrize("codec", ["q8", "q4t", "q4tp"])
def test_moe_block_jobs(gpu, codec):
    """moe_block (gpu.rs:2482) over MoeJob-shaped jobs with their own inputs
    and blend weights: out = sum_j w_j down_j(silu(gate_j xg_j) * up_j xu_j)"""
    from cmf_amd import synth
    H, I, nj = 256, 128, 3
    mk = {"q8": lambda s, r, c: synth.q8_normal(s, r, c, 0.05), "q4t": lambda s, r, c: synth.q4t_normal(s, r, c, 0.05),
          "q4tp": lambda s, r, c: synth.q4tp_uniform(s, r, c, 0.05)}[codec]
    W = lambda t: gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
    trios = [(mk(300 + 3 * j, I, H), mk(301 + 3 * j, I, H), mk(302 + 3 * j, H, I)) for j in range(nj)]
    ws = [W(t) for tr in trios for t in tr]
    jobs, ref = [], np.zeros(H, np.float32)
    for j, (g, u, d) in enumerate(trios):
        xg, xu = _x(400 + j, 1, H)[0], _x(500 + j, 1, H)[0]
        bw = np.float32(0.2 + 0.3 * j)
        job = {"gate": ws[3 * j], "up": ws[3 * j + 1], "down": ws[3 * j + 2], "xs_gate": xg, "xs_up": xu, "w": bw,
               "q4t": codec == "q4t", "q4tp": codec == "q4tp"}
        if codec == "q8" and j == 1:  # caller scales on one trio
            job["gate_row_scale"] = (g["row_scale"] * 0.7).astype(np.float32)
            g = dict(g, row_scale=job["gate_row_scale"])
        jobs.append(job)
        a = (_silu(orc.matmat(g, xg)[0]) * orc.matmat(u, xu)[0]).astype(np.float32)
        ref = (ref + bw * orc.matmat(d, a)[0]).astype(np.float32)
    got = gpu.moe_block_jobs(jobs, H)
    print(f"{codec}: rel-L2 {rel_l2(got, ref):.2e}", flush=True)
    assert rel_l2(got, ref) < TOL
    # the refusals of gpu.rs:814-841: the whole block is declined
    for bad in ({"swiglu_limit": 7.0}, {"q1": 1}, {"gu_q2": 1}, {"down_col": np.ones(I, np.float32)},
                {"q4t": codec != "q4t", "q4tp": codec == "q4t"}):
        jb = [dict(jobs[0]), dict(jobs[1], **bad)]
        assert gpu.moe_block_jobs(jb, H) is None, bad
    for w in ws:
        w.free()


def test_matvec_batch(gpu):
    """matvec_batch (gpu.rs:2494): independent matvecs of three codecs in one
    call; a Q1 job declines the whole batch"""
    from cmf_amd import synth
    ts = [synth.q8_normal(601, 96, 128, 0.05), synth.q4t_normal(602, 64, 256, 0.05), synth.q4tp_uniform(603, 32, 512)]
    ws = [gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
          for t in ts]
    xs = [_x(610 + i, 1, t["cols"])[0] for i, t in enumerate(ts)]
    rs0 = (ts[0]["row_scale"] * 2).astype(np.float32)
    outs = gpu.matvec_batch([(ws[0], xs[0], rs0, 3), (ws[1], xs[1], None, 11), (ws[2], xs[2], None, 15)])
    refs = [orc.matmat(dict(ts[0], row_scale=rs0), xs[0])[0], orc.matmat(ts[1], xs[1])[0], orc.matmat(ts[2], xs[2])[0]]
    for o, r in zip(outs, refs):
        assert rel_l2(o, r) < TOL
    assert gpu.matvec_batch([(ws[1], xs[1], None, 11), (ws[0], xs[0], None, 1)]) is None  # Q1 layout
    assert gpu.matvec_batch([(ws[1], xs[1], None, 15)]) is None  # layout != weight codec
    for w in ws:
        w.free()


def test_seam_declines_other_codec(gpu):
    from cmf_amd import synth
    t = synth.q4t_uniform(91, 64, 64)
    w = gpu.Weight(t["dtype"], 64, 64, payload=t["bytes"])
    out = np.zeros((1, 64), np.float32)
    assert gpu.q8_matmat(w, _x(92, 1, 64), 1, 64, 64, out) is False
    assert gpu.q4tp_matvec(w, _x(92, 1, 64), 64, 64, out) is False
    assert gpu.q4t_matvec(w, _x(92, 1, 64), 64, 64, out) is True


def test_q4tp_step0_equals_q4t(gpu):
    """A q4tp tensor whose ladder is flat (step 0) and a q4t tensor with the
    same nibbles and scale 2^lo give identical products."""
    from cmf_amd import synth
    rows, cols = 64, 256
    tp = synth.q4tp_uniform(101, rows, cols)
    gpr = cols // 32
    b = tp["bytes"].copy()
    params = b[rows * gpr * 16: rows * gpr * 16 + rows * 4].view(np.uint16).reshape(rows, 2)
    params[:, 1] = 0  # step = 0 -> every rung equals 2^lo
    q4t = np.empty(rows * gpr * 18, np.uint8).reshape(rows, gpr, 18)
    lo = params[:, 0].view(np.float16).astype(np.float32)
    s16 = np.exp2(lo).astype(np.float16)
    q4t[:, :, 0:2] = np.repeat(s16.view(np.uint8).reshape(rows, 1, 2), gpr, axis=1)
    q4t[:, :, 2:] = b[: rows * gpr * 16].reshape(rows, gpr, 16)
    ttp = dict(tp, bytes=b)
    tt = synth.tensor(synth.DT_Q4T, rows, cols, payload=q4t.reshape(-1))
    x = _x(102, 3, cols)
    if np.all(np.exp2(lo).astype(np.float16).astype(np.float32) == np.exp2(lo).astype(np.float32)):
        a = gpu.matmul(gpu.Weight(synth.DT_Q4TP, rows, cols, payload=b), x)
        c = gpu.matmul(gpu.Weight(synth.DT_Q4T, rows, cols, payload=tt["bytes"]), x)
        assert rel_l2(a, c) < 1e-6
    else:
        a = gpu.matmul(gpu.Weight(synth.DT_Q4TP, rows, cols, payload=b), x)
        assert rel_l2(a, orc.matmat(ttp, x)) < TOL


def test_ffn(gpu):
    """gpu.rs:1773 q4t_ffn: down(silu(gate x) * up x)"""
    from cmf_amd import synth
    H, I = 256, 512
    g, u, d = synth.q4t_normal(111, I, H), synth.q4t_normal(112, I, H), synth.q4t_normal(113, H, I)
    x = _x(114, 3, H)
    W = lambda t: gpu.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"])
    out = np.zeros((3, H), np.float32)
    assert gpu.ffn(W(g), W(u), W(d), x, 3, H, I, out)
    gg, uu = orc.matmat(g, x), orc.matmat(u, x)
    act = (gg / (1 + np.exp(-gg))) * uu
    ref = orc.matmat(d, act.astype(np.float32))
    assert rel_l2(out, ref) < TOL
