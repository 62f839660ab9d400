#!/usr/bin/env python3
"""Headline benchmark: spec-verify decode tok/s + q4t GEMV HBM GB/s, 1 MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A "step" is one speculative round (graph_spec_step of the reference,
pipeline.rs:3582-4213): K=4 MTP drafts, the 5-row verify over all 28 layers,
acceptance, the MTP re-warm and the commit, on the synthetic random-init
Qwen3-0.6B-arch model (attention q8, FFN q4t, lm_head/embedding q8) after a
2048-token prefill of seeded uniform ids.  `value` is emitted tokens per
second over exactly K timed rounds (inputs and weights resident in HBM).

`roofline` is the dominant GEMV of the metric, the q4t gate/up GEMV
12288x4096 at M=1, timed with HIP events on the library
stream over back-to-back launches rotating 10 weight copies (283 MB > the
256 MB last-level cache).  `cpu_baseline` is the C oracle (the reference's
CPU path restated) decoding from the GPU's prefilled state on the host cores.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8000.0  # GB/s, MI355X HBM3E
PEAK_F16 = 2500.0  # TFLOP/s, MI355X dense f16 MFMA
COPY_BYTES = 64 << 20  # counter-calibration copy (read + write of this many bytes)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4t_gemv_12288x4096_m1_traffic.txt")


ROOF_KERNEL = "k_gemv_q4t_m1<8, 4, false, 1>"  # the kernel the dispatch runs for the roofline GEMV


def measured_traffic():
    """HBM bytes per launch of the roofline GEMV from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), or
    None when no summary is present or it was measured on another kernel."""
    kern, val = None, None
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("kernel:"):
                    kern = line.split(":", 1)[1].strip()
                if line.startswith("traffic_bytes_per_launch:"):
                    val = int(float(line.split(":", 1)[1]))
    except OSError:
        return None
    return val if kern == ROOF_KERNEL else None
METRIC = "spec-verify decode tok/s + q4t GEMV HBM GB/s (% of peak), 1 MI355X"


def q4_bytes(rows, cols, m, dtype):
    gpr = cols // 32
    if dtype == "q4t":
        w = rows * gpr * 18
    else:  # q4tp: nibbles + row params + 5-bit codes
        w = rows * gpr * 16 + rows * 4 + rows * ((gpr * 5 + 7) // 8)
    return w + m * (rows + cols) * 4


def time_gemv(cmf, t, m, copies, iters=200, warmup=20, seed=7):
    """Average device ms per launch (HIP events, library stream) and GB/s."""
    import ctypes as C
    from cmf_amd import synth
    ws = [cmf.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
          for _ in range(copies)]
    x = synth.normal(seed, m * t["cols"]).reshape(m, t["cols"])
    dx = cmf.DevBuf(x.nbytes)
    dx.upload(x)
    pl = cmf.DevBuf(cmf.lib().cmf_prep_bytes(ws[0].h))
    xs = cmf.DevBuf(64 * 4)
    dy = cmf.DevBuf(m * t["rows"] * 4)
    cmf.check(cmf.lib().cmf_prep_dev(ws[0].h, dx.p, t["cols"], m, pl.p, xs.p))
    arr = (C.c_void_p * copies)(*[w.h for w in ws])
    ms = C.c_float()
    cmf.check(cmf.lib().cmf_time_gemv(arr, copies, pl.p, xs.p, m, dy.p, t["rows"], 0, warmup, iters, C.byref(ms)))
    for w in ws:
        w.free()
    return ms.value


def time_gemv_from_x(cmf, t, m, copies, fused, iters=200, warmup=20, seed=7):
    """Average ms per call of the GEMV from f32 rows x resident in HBM:
    fused=0 the operand producer launch + the GEMV, fused=1 one launch whose
    workgroups stage the operand themselves."""
    import ctypes as C
    from cmf_amd import synth
    ws = [cmf.Weight(t["dtype"], t["rows"], t["cols"], payload=t["bytes"], q=t["q"], row_scale=t["row_scale"])
          for _ in range(copies)]
    x = synth.normal(seed, m * t["cols"]).reshape(m, t["cols"])
    dx = cmf.DevBuf(x.nbytes)
    dx.upload(x)
    dy = cmf.DevBuf(m * t["rows"] * 4)
    arr = (C.c_void_p * copies)(*[w.h for w in ws])
    ms = C.c_float()
    cmf.check(cmf.lib().cmf_time_gemv_rows(arr, copies, dx.p, t["cols"], None, m, dy.p, t["rows"], fused, warmup,
                                           iters, C.byref(ms)))
    for w in ws:
        w.free()
    dx.free()
    dy.free()
    return ms.value


def gemm_sweep(cmf, synth):
    """Large-batch q4t GEMM (prefill / matmat b > 16) on the config-2 gate/up
    shape: MFMA rate counting both f16 halves of the operand (2 MFMAs per
    weight tile), against the 2.5 PFLOP/s dense f16 peak."""
    import ctypes as C
    t = synth.q4t_uniform(77, 12288, 4096)
    w = cmf.Weight(t["dtype"], 12288, 4096, payload=t["bytes"])
    res = []
    for m in (64, 256, 2048):
        x = synth.normal(78, m * 4096).reshape(m, 4096)
        dx, dy = cmf.DevBuf(x.nbytes), cmf.DevBuf(m * 12288 * 4)
        dx.upload(x)
        ms = C.c_float()
        cmf.check(cmf.lib().cmf_time_gemm(w.h, dx.p, m, dy.p, 3, 20, C.byref(ms)))
        mfma_flops = 2 * 2.0 * m * 12288 * 4096  # hi + lo halves
        res.append({"m": m, "us": round(ms.value * 1e3, 1),
                    "TFLOP/s": round(2.0 * m * 12288 * 4096 / ms.value / 1e9, 1),
                    "mfma_util": round(mfma_flops / ms.value / 1e9 / PEAK_F16, 4)})
        dx.free()
        dy.free()
    w.free()
    return res


def moe_layer(cmf, synth, b=5, ne=128, hidden=2048, inter=768, top_k=8):
    """the MoE FFN of an M=5 verify batch (router logits
    N(0,1), 128 q4t experts, top-8) and the 4096x2048 q8 attention projection
    at M=5, inputs resident in HBM.  Bytes: every distinct routed expert's
    gate/up/down weights once + activations; the projection's weights."""
    import ctypes as C
    from cmf_amd.moe import MoE
    ex = [{"gate": synth.q4t_uniform(900 + 3 * e, inter, hidden), "up": synth.q4t_uniform(901 + 3 * e, inter, hidden),
           "down": synth.q4t_uniform(902 + 3 * e, hidden, inter)} for e in range(ne)]
    moe = MoE(ne, hidden, inter, top_k, ex)
    x = synth.normal(5001, b * hidden).reshape(b, hidden)
    lg = synth.normal(5002, b * ne).reshape(b, ne)
    _, idx, _ = moe.ffn(x, lg)
    distinct = len(set(idx.ravel().tolist()))
    dx, dl, do = cmf.DevBuf(x.nbytes), cmf.DevBuf(lg.nbytes), cmf.DevBuf(x.nbytes)
    dx.upload(x)
    dl.upload(lg)
    ms = C.c_float()
    cmf.check(cmf.lib().cmf_time_moe(moe.h, dx.p, dl.p, b, do.p, 10, 200, C.byref(ms)))
    per_expert = 3 * inter * (hidden // 32) * 18
    moe_bytes = distinct * per_expert + b * (hidden + ne) * 4 + b * hidden * 4
    t8 = synth.q8_uniform(5003, 4096, 2048)
    pms = time_gemv(cmf, t8, b, copies=16)
    pbytes = 4096 * 2048 + 4096 * 4 + b * (2048 + 4096) * 4
    moe.free()
    for d in (dx, dl, do):
        d.free()
    return {"workload": f"M={b} verify tokens, {ne} q4t experts (hidden {hidden}, FFN {inter}), top-{top_k}, "
                        "router logits N(0,1); + q8 4096x2048 projection",
            "distinct_experts": distinct, "moe_us": round(ms.value * 1e3, 2),
            "moe_GB/s": round(moe_bytes / ms.value / 1e6, 1), "moe_bytes": moe_bytes,
            "proj_us": round(pms * 1e3, 2), "proj_GB/s": round(pbytes / pms / 1e6, 1),
            "layer_us": round((ms.value + pms) * 1e3, 2)}


def _cpu_rate(fn, min_s=0.5):
    """Seconds per call of fn on the host (repeated to at least min_s)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            return dt / n


def host_cpus():
    """(threads this process may use, physical cores behind them, logical
    CPUs of the host).  The pool is capped at OMP_NUM_THREADS when set (the
    GPU box sets it to the box's CPU share)."""
    aff = sorted(os.sched_getaffinity(0))
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    use = aff[:cap] if cap > 0 else aff
    cores = set()
    for cpu in use:
        try:
            base = f"/sys/devices/system/cpu/cpu{cpu}/topology/"
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                cores.add((pkg, f.read().strip()))
        except OSError:
            cores.add(("?", str(cpu)))
    return len(use), len(cores), os.cpu_count() or len(aff)


def cpu_baseline(sm, cpu_state, prompt, args):
    """The reference's CPU path restated (the C oracle) on the host cores:
    spec decode from the GPU's prefilled state with the verify rows batched
    (pipeline.rs:4275-4505) under both matvec contracts of the reference:
    a8w8 (split_act + integer dots) through the AVX-512 VNNI timing arm --
    the reference's default on an x86 host with VNNI, and `value` -- and the
    exact contract (CMF_SDOT=0), whose tokens the GPU's must equal.  Beside
    them the BASELINE configs' CPU kernels (configs 1-3, 5) under both."""
    from oracle import oracle as orc
    from cmf_amd import synth
    threads, phys, logical = host_cpus()
    fast = orc.fast_supported()
    legs = {}
    toks_exact = None
    for contract, n_cpu in (("a8w8", 24), ("exact", 6)):
        if contract == "a8w8" and not fast:
            continue
        o = orc.OracleModel(sm, threads=threads, a8w8=contract == "a8w8", fast=contract == "a8w8",
                            batch_verify=True)
        for li, (kk, vv) in enumerate(cpu_state["kv"]):
            o.import_kv(li, kk, vv)
        o.import_kv(-1, *cpu_state["mtp"])
        tc = time.perf_counter()
        ct, cst = o.decode(cpu_state["hidden"], cpu_state["next_pos"], prompt, n_cpu, spec=True, k=args.k)
        tcpu = time.perf_counter() - tc
        legs[contract] = {"tok/s": round(len(ct) / tcpu, 3), "tokens": len(ct), "rounds": cst.rounds,
                          "s": round(tcpu, 1)}
        if contract == "exact":
            toks_exact = ct
    # BASELINE configs 1-3 and 5 on the CPU path, exact and a8w8 (VNNI arm)
    kern = []

    def both(config, name, t, x, nbytes):
        for a8 in ((False, True) if fast else (False,)):
            sec = _cpu_rate(lambda: orc.matmat(t, x, threads=threads, fast=a8))
            e = {"config": config, "kernel": f"{name} ({'a8w8 VNNI' if a8 else 'exact'})", "us": round(sec * 1e6, 1)}
            if nbytes:
                e["GB/s"] = round(nbytes / sec / 1e9, 2)
            kern.append(e)

    t1 = synth.q8_uniform(11, 4096, 4096)
    both(1, "q8 4096x4096 M=1", t1, synth.normal(7, 4096).reshape(1, 4096), 4096 * 4096 + 4096 * 4)
    t2 = synth.q4t_uniform(31 + 12288, 12288, 4096)
    for m in (1, 8):
        both(2, f"q4t 12288x4096 M={m}", t2, synth.normal(7, m * 4096).reshape(m, 4096),
             q4_bytes(12288, 4096, m, "q4t"))
    t3 = synth.q4tp_uniform(41 + 12288, 12288, 4096)
    both(3, "q4tp 12288x4096 M=5", t3, synth.normal(7, 5 * 4096).reshape(5, 4096), q4_bytes(12288, 4096, 5, "q4tp"))
    ne, hidden, inter, top_k = 128, 2048, 768, 8
    ex = [{"gate": synth.q4t_uniform(900 + 3 * e, inter, hidden), "up": synth.q4t_uniform(901 + 3 * e, inter, hidden),
           "down": synth.q4t_uniform(902 + 3 * e, hidden, inter)} for e in range(ne)]
    xm = synth.normal(5001, 5 * hidden).reshape(5, hidden)
    lg = synth.normal(5002, 5 * ne).reshape(5, ne)
    sec = _cpu_rate(lambda: orc.moe_ffn_rows(ex, top_k, lg, xm, threads=threads))
    kern.append({"config": 5, "kernel": "MoE FFN M=5 (128 q4t experts, top-8; exact)", "us": round(sec * 1e6, 1)})
    both(5, "q8 4096x2048 M=5 projection", synth.q8_uniform(5003, 4096, 2048),
         synth.normal(7, 5 * 2048).reshape(5, 2048), 4096 * 2048)
    lead = "a8w8" if "a8w8" in legs else "exact"
    L = legs[lead]
    base = {"value": L["tok/s"], "unit": "tok/s", "cores": threads, "threads": threads,
            "host_physical_cores": phys, "host_logical_cpus": logical, "kind": "port",
            "sample": f"C oracle (the reference's CPU path restated; OpenMP over {threads} threads on {phys} "
                      f"physical cores of a {logical}-CPU host): {L['tokens']} tokens of spec decode (K={args.k}, "
                      f"{L['rounds']} rounds, verify rows batched, "
                      f"{'a8w8 contract on the AVX-512 VNNI kernels' if lead == 'a8w8' else 'exact contract'}) "
                      f"from the GPU's prefilled {args.ctx}-token state in {L['s']} s; the exact contract and "
                      f"the configs' kernels beside it",
            "contracts": legs, "kernels": kern}
    return base, toks_exact


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-gemv", action="store_true", help="skip the GEMV sweep")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE verify layer (config 5)")
    ap.add_argument("--moe-only", action="store_true", help="only the MoE verify layer (profiling runs)")
    ap.add_argument("--gemv-only", action="store_true", help="only the GEMV sweep (profiling runs)")
    ap.add_argument("--profile-gemv", action="store_true",
                    help="only the HBM-counter workload: 20 plain copies of 64 MiB (counter calibration), then "
                         "50 launches of the roofline GEMV (q4t 12288x4096 M=1)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the decode hot path has no "
                                   "multi-GPU leg (no collectives); run with --gpus 1"}))
        sys.exit(2)

    import cmf_amd as cmf
    from cmf_amd import synth
    cmf.init(0)
    if args.profile_gemv:
        import ctypes as C
        ms = C.c_float()
        cmf.check(cmf.lib().cmf_time_copy(COPY_BYTES, 4, 20, C.byref(ms)))
        t2 = synth.q4t_uniform(31 + 12288, 12288, 4096)
        g = time_gemv(cmf, t2, 1, copies=10, iters=50, warmup=10)
        print(json.dumps({"copy_bytes": COPY_BYTES, "copy_us": round(ms.value * 1e3, 2),
                          "gemv": "q4t 12288x4096 M=1", "gemv_us": round(g * 1e3, 3)}))
        return
    t_setup = time.perf_counter()
    out = {"metric": METRIC, "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded; random-init weights N(0,0.02) quantized)"}

    # ---------------- GEMV sweep ----------------
    kernels = []
    roof = None
    if not args.no_gemv:
        t1 = synth.q8_uniform(11, 4096, 4096)
        ms = time_gemv(cmf, t1, 1, copies=16)
        b = 4096 * 4096 + 3 * 4096 * 4
        kernels.append({"kernel": "q8 GEMV 4096x4096 M=1", "us": ms * 1e3, "GB/s": b / ms / 1e6,
                        "frac": b / ms / 1e6 / PEAK_HBM})
        for shape in [(12288, 4096), (4096, 12288)]:
            t2 = synth.q4t_uniform(31 + shape[0], shape[0], shape[1])
            for m in [1, 2, 4, 8, 16]:
                ms = time_gemv(cmf, t2, m, copies=10)
                b = q4_bytes(shape[0], shape[1], m, "q4t")
                e = {"kernel": f"q4t GEMV {shape[0]}x{shape[1]} M={m}", "us": ms * 1e3, "GB/s": b / ms / 1e6,
                     "frac": b / ms / 1e6 / PEAK_HBM}
                kernels.append(e)
                if shape == (12288, 4096) and m == 1:
                    import ctypes as C
                    # the same weight bytes read by a plain kernel of the GEMV's launch
                    # shape (the ceiling for one launch), and the call from f32 x
                    pr = C.c_float()
                    wbytes = 12288 * 4096 // 32 * 18
                    cmf.check(cmf.lib().cmf_time_read(wbytes, 10, 200, C.byref(pr)))
                    fx0 = time_gemv_from_x(cmf, t2, 1, 10, 0)
                    fx1 = time_gemv_from_x(cmf, t2, 1, 10, 1)
                    roof = {"bound": "hbm", "achieved": round(e["GB/s"], 1), "peak": PEAK_HBM, "unit": "GB/s",
                            "frac": round(e["frac"], 4), "traffic": measured_traffic(),
                            "kernel": f"{ROOF_KERNEL} (q4t gate/up 12288x4096, M=1, prepared operand)",
                            "bytes_per_launch": b, "avg_launch_us": round(ms * 1e3, 3),
                            "plain_read_us": round(pr.value * 1e3, 3),
                            "plain_read_GB/s": round(wbytes / pr.value / 1e6, 1),
                            "gemv_vs_plain_read": round(pr.value / ms, 4),
                            "from_f32_x_us": {"producer launch + GEMV": round(fx0 * 1e3, 3),
                                              "operand staged in the GEMV": round(fx1 * 1e3, 3)}}
            t3 = synth.q4tp_uniform(41 + shape[0], shape[0], shape[1])
            ms = time_gemv(cmf, t3, 5, copies=10)
            b = q4_bytes(shape[0], shape[1], 5, "q4tp")
            kernels.append({"kernel": f"q4tp GEMM {shape[0]}x{shape[1]} M=5", "us": ms * 1e3,
                            "GB/s": b / ms / 1e6, "frac": b / ms / 1e6 / PEAK_HBM})
        for e in kernels:
            for kk in ("us", "GB/s", "frac"):
                e[kk] = round(e[kk], 4 if kk == "frac" else 2)
        out["roofline"] = roof
        out["kernels"] = kernels
        import ctypes as C
        ms = C.c_float()
        cmf.check(cmf.lib().cmf_time_copy(COPY_BYTES, 4, 20, C.byref(ms)))
        out["device_copy_GB/s"] = round(2 * COPY_BYTES / ms.value / 1e6, 1)  # read + write, 64 MiB
        out["gemm"] = gemm_sweep(cmf, synth)
    if args.gemv_only:
        print(json.dumps(out))
        return

    # ---------------- MoE verify layer ----------------
    if not args.no_moe:
        out["moe"] = moe_layer(cmf, synth)
    if args.moe_only:
        print(json.dumps(out))
        return

    # ---------------- spec decode ----------------
    from cmf_amd.model import Model
    sm = synth.synth_model(synth.QWEN3_06B, seed=1)
    model = Model(sm)
    prompt = synth.ids(2024, args.ctx, sm["cfg"]["vocab"])
    model.prefill(prompt[:300])  # first call: buffers and kernels warmed
    tp = time.perf_counter()
    model.prefill(prompt)
    prefill_s = time.perf_counter() - tp
    next_pos, hidden = model.state()
    cpu_state = None
    if not args.no_cpu:
        c = sm["cfg"]
        cpu_state = {"kv": [model.kv_export(li, args.ctx) for li in range(c["n_layers"])],
                     "mtp": model.kv_export(-1, args.ctx - 1), "hidden": hidden, "next_pos": next_pos}
    model.decode_begin(seed=0)
    model.decode_rounds(args.warmup, spec=True, k=args.k)
    cmf.lib().cmf_sync()
    n0 = len(model.tokens())
    t0 = time.perf_counter()
    st = model.decode_rounds(args.steps, spec=True, k=args.k)
    cmf.lib().cmf_sync()
    dt = time.perf_counter() - t0
    toks = model.tokens()
    produced = len(toks) - n0
    out["value"] = round(produced / dt, 2)
    out["ms_per_step"] = round(dt * 1e3 / max(args.steps, 1), 4)
    out["spec"] = {"k": args.k, "rounds": args.steps, "tokens": produced, "accepted_total": st.accepted,
                   "drafted_total": st.drafted, "device_ms_per_round": round(st.device_ms / max(args.steps, 1), 4),
                   "acceptance": round(st.accepted / max(st.drafted, 1), 4)}
    # config 4 at T = 0.8 (sampler defaults otherwise, repetition penalty 1.0):
    # the device sparse chain + sampled acceptance, continuing from this state
    from cmf_amd import SamplerConfig
    n_s = max(8, args.steps // 4)
    model.decode_begin(SamplerConfig(temperature=0.8, repetition_penalty=1.0), seed=7)
    model.decode_rounds(2, spec=True, k=args.k)
    cmf.lib().cmf_sync()
    s0 = len(model.tokens())
    ts0 = time.perf_counter()
    sst = model.decode_rounds(n_s, spec=True, k=args.k)
    cmf.lib().cmf_sync()
    dts = time.perf_counter() - ts0
    out["sampled"] = {"temperature": 0.8, "top_k": 40, "top_p": 0.9, "min_p": 0.05, "rounds": n_s,
                      "tokens": len(model.tokens()) - s0, "tok/s": round((len(model.tokens()) - s0) / dts, 2),
                      "ms_per_round": round(dts * 1e3 / n_s, 4), "accepted": sst.accepted, "drafted": sst.drafted}
    # plain decode (spec=False, forward_token_graph's counterpart): greedy
    # tokens, each one trunk forward + lm_head + argmax, replayed from a
    # captured step
    model.decode_begin(seed=0)
    model.decode_rounds(4, spec=False)
    cmf.lib().cmf_sync()
    tp0 = time.perf_counter()
    model.decode_rounds(args.steps, spec=False)
    cmf.lib().cmf_sync()
    dtp = time.perf_counter() - tp0
    out["plain"] = {"tokens": args.steps, "ms_per_token": round(dtp * 1e3 / args.steps, 4),
                    "tok/s": round(args.steps / dtp, 2)}
    # the reference's decode loop with the speculation monitor (SpecMon,
    # pipeline.rs:661-694): five timed rounds, eight timed plain tokens, then
    # the faster arm (host-paced rounds, as the reference's)
    n_mon = 64
    tm0 = time.perf_counter()
    mt, mst = model.decode(n_mon, spec="auto", k=args.k)
    dtm = time.perf_counter() - tm0
    mon = model.monitor()
    out["spec_monitor"] = {"tokens": int(len(mt)), "s": round(dtm, 4), "decision": mon.phase_name,
                           "round_ms": round(mon.round_ms, 4), "tokens_per_round": round(mon.tokens, 3),
                           "plain_ms": round(mon.plain_ms, 4), "spec_rounds": mon.spec_rounds,
                           "plain_steps": mon.plain_steps, "accepted": mst.accepted, "drafted": mst.drafted}
    # HBM bytes a round must stream at ctx ~2048 (weights + KV), for context
    c = sm["cfg"]
    layer_w = sum(len(t["bytes"]) if t["bytes"] is not None else t["q"].nbytes + t["row_scale"].nbytes
                  for l in sm["layers"] for n, t in l.items() if isinstance(t, dict))
    mtp_w = sum(len(t["bytes"]) if t["bytes"] is not None else t["q"].nbytes + t["row_scale"].nbytes
                for n, t in sm["mtp"]["layer"].items() if isinstance(t, dict))
    lm_w = sm["lm_head"]["q"].nbytes + sm["lm_head"]["row_scale"].nbytes
    eh_w = sm["mtp"]["eh_proj"]["q"].nbytes
    kv = 2 * c["n_kv"] * c["head_dim"] * 4 * (next_pos + produced // 2)
    round_bytes = layer_w + lm_w + kv * c["n_layers"] + args.k * (mtp_w + eh_w + lm_w + kv)
    out["prefill"] = {"positions": args.ctx, "ms": round(prefill_s * 1e3, 1),
                      "tok/s": round(args.ctx / prefill_s, 1),
                      "path": "2048-position chunks on the q8 / q4t MFMA GEMMs, tiled causal attention"}
    out["spec"]["round_hbm_bytes"] = int(round_bytes)
    out["spec"]["round_hbm_GB/s"] = round(round_bytes / (dt / max(args.steps, 1)) / 1e9, 1)
    out["config"] = {"workload": f"spec-verify decode (MTP K={args.k}, greedy) on the synthetic Qwen3-0.6B-arch "
                                 f"model: 28 layers, hidden 1024, 16Q/8KV x 128, FFN 3072, vocab 151936, "
                                 f"attention q8 / FFN q4t / lm_head q8, context {args.ctx}",
                     "batch": 1, "context": args.ctx, "draft_k": args.k, "parallelism": "single GPU"}

    # ---------------- CPU baseline: the oracle from the same state ----------------
    if cpu_state is not None:
        out["cpu_baseline"], ct = cpu_baseline(sm, cpu_state, prompt, args)
        n = min(len(ct), len(toks))
        out["cpu_gpu_tokens_equal"] = bool(n > 0 and ct[:n].tolist() == toks[:n].tolist())
    out["setup_s"] = round(time.perf_counter() - t_setup, 1)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
