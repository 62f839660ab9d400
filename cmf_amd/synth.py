"""Seeded synthetic inputs of the benchmark configurations (host only).

All generators are SplitMix64 -> Box-Muller streams implemented in
csrc/synth.cpp; one stream per tensor row, so results do not depend on the
thread count.  Payloads use the reference's byte layouts (quant.rs).
"""
import numpy as np

from . import DT_Q4T, DT_Q4TP, DT_Q8ROW, _ptr, lib


def normal(seed, n, sigma=1.0):
    out = np.empty(int(n), dtype=np.float32)
    lib().cmf_synth_normal(seed, int(n), float(sigma), _ptr(out))
    return out


def ids(seed, n, vocab):
    out = np.empty(int(n), dtype=np.int32)
    lib().cmf_synth_ids(seed, int(n), int(vocab), _ptr(out))
    return out


def q4t_bytes(rows, cols):
    return rows * (cols // 32) * 18


def q4tp_bytes(rows, cols):
    gpr = cols // 32
    return rows * gpr * 16 + rows * 4 + rows * ((gpr * 5 + 7) // 8)


def tensor(dtype, rows, cols, q=None, row_scale=None, payload=None):
    return {"dtype": dtype, "rows": rows, "cols": cols, "q": q, "row_scale": row_scale, "bytes": payload}


def q8_uniform(seed, rows, cols):
    """Config 1: int8 uniform in [-127, 127], f32 row scale |N(0,1)|*0.01."""
    q = np.empty((rows, cols), dtype=np.int8)
    rs = np.empty(rows, dtype=np.float32)
    lib().cmf_synth_q8_uniform(seed, rows, cols, _ptr(q), _ptr(rs))
    return tensor(DT_Q8ROW, rows, cols, q=q, row_scale=rs)


def q4t_uniform(seed, rows, cols, sigma=0.02):
    """Config 2: nibbles uniform 0..15, f16 tile scale |N(0,1)|*sigma."""
    b = np.empty(q4t_bytes(rows, cols), dtype=np.uint8)
    lib().cmf_synth_q4t_uniform(seed, rows, cols, float(sigma), _ptr(b))
    return tensor(DT_Q4T, rows, cols, payload=b)


def q4tp_uniform(seed, rows, cols, sigma=0.02, ratio=1.1):
    """Config 3: per-row ladder lo=log2(|N|*sigma), step=log2(ratio); codes U{0..31}."""
    b = np.empty(q4tp_bytes(rows, cols), dtype=np.uint8)
    lib().cmf_synth_q4tp_uniform(seed, rows, cols, float(sigma), float(ratio), _ptr(b))
    return tensor(DT_Q4TP, rows, cols, payload=b)


def q8_normal(seed, rows, cols, sigma=0.02):
    """Weights ~N(0, sigma^2) quantized to q8_row (absmax/127, f16-rounded)."""
    q = np.empty((rows, cols), dtype=np.int8)
    rs = np.empty(rows, dtype=np.float32)
    lib().cmf_synth_q8_normal(seed, rows, cols, float(sigma), _ptr(q), _ptr(rs))
    return tensor(DT_Q8ROW, rows, cols, q=q, row_scale=rs)


def q4t_normal(seed, rows, cols, sigma=0.02):
    """Weights ~N(0, sigma^2) quantized to q4_tiled (absmax/7 per 32-group)."""
    b = np.empty(q4t_bytes(rows, cols), dtype=np.uint8)
    lib().cmf_synth_q4t_normal(seed, rows, cols, float(sigma), _ptr(b))
    return tensor(DT_Q4T, rows, cols, payload=b)


def dequant(t):
    """f32 [rows, cols] of a synthetic tensor (numpy restatement of the
    quant.rs dequantizers, for small reference checks)."""
    rows, cols = t["rows"], t["cols"]
    if t["dtype"] == DT_Q8ROW:
        return t["q"].astype(np.float32) * t["row_scale"][:, None]
    gpr = cols // 32
    b = t["bytes"]
    if t["dtype"] == DT_Q4T:
        tiles = b[: rows * gpr * 18].reshape(rows, gpr, 18)
        s = tiles[:, :, :2].copy().view(np.float16).astype(np.float32)[:, :, 0]
        nib = tiles[:, :, 2:]
    else:
        nib = b[: rows * gpr * 16].reshape(rows, gpr, 16)
        params = b[rows * gpr * 16: rows * gpr * 16 + rows * 4].copy().view(np.float16).astype(np.float32)
        params = params.reshape(rows, 2)
        stride = (gpr * 5 + 7) // 8
        codes = b[rows * gpr * 16 + rows * 4:].reshape(rows, stride)
        ratio = np.exp2(params[:, 1]).astype(np.float32)
        lad = np.empty((rows, 32), dtype=np.float32)
        lad[:, 0] = np.exp2(params[:, 0]).astype(np.float32)
        for c in range(1, 32):
            lad[:, c] = (lad[:, c - 1] * ratio).astype(np.float32)
        g = np.arange(gpr)
        bit = g * 5
        lo = codes[:, bit // 8].astype(np.uint16)
        nxt = np.minimum(bit // 8 + 1, stride - 1)
        hi = np.where((bit % 8) > 3, codes[:, nxt], 0).astype(np.uint16)
        code = ((lo | (hi << 8)) >> (bit % 8).astype(np.uint16)) & 0x1F
        s = np.take_along_axis(lad, code.astype(np.int64), axis=1)
    w = np.empty((rows, gpr, 32), dtype=np.float32)
    w[:, :, 0::2] = (nib & 0x0F).astype(np.float32) - 8.0
    w[:, :, 1::2] = (nib >> 4).astype(np.float32) - 8.0
    return (w * s[:, :, None]).reshape(rows, cols)


# --------------------------------------------------------------------------
# synthetic Qwen3-arch model
# --------------------------------------------------------------------------
QWEN3_06B = dict(n_layers=28, hidden=1024, n_heads=16, n_kv=8, head_dim=128, inter=3072,
                 vocab=151936, max_seq=4096, rope_theta=1e6, eps=1e-6)


def _w(dtype, seed, rows, cols, sigma):
    if dtype == DT_Q8ROW:
        return q8_normal(seed, rows, cols, sigma)
    if dtype == DT_Q4T:
        return q4t_normal(seed, rows, cols, sigma)
    raise ValueError("synthetic model weights: q8 or q4t")


def _norm(seed, n, noise):
    if noise == 0.0:
        return np.ones(n, dtype=np.float32)
    return (1.0 + normal(seed, n, noise)).astype(np.float32)


def _layer(cfg, seed, attn_dt, ffn_dt, sigma, noise):
    H, hd, nh, nkv, I = cfg["hidden"], cfg["head_dim"], cfg["n_heads"], cfg["n_kv"], cfg["inter"]
    s = lambda i: (seed * 1000003 + i) & 0xFFFFFFFFFFFFFFFF
    return {
        "input_norm": _norm(s(1), H, noise), "post_norm": _norm(s(2), H, noise),
        "q_norm": _norm(s(3), hd, noise), "k_norm": _norm(s(4), hd, noise),
        "wq": _w(attn_dt, s(5), nh * hd, H, sigma), "wk": _w(attn_dt, s(6), nkv * hd, H, sigma),
        "wv": _w(attn_dt, s(7), nkv * hd, H, sigma), "wo": _w(attn_dt, s(8), H, nh * hd, sigma),
        "gate": _w(ffn_dt, s(9), I, H, sigma), "up": _w(ffn_dt, s(10), I, H, sigma),
        "down": _w(ffn_dt, s(11), H, I, sigma),
    }


def _moe(cfg, seed, moe, ffn_dtype, sigma):
    """A routed-expert FFN (Qwen3-MoE: softmax router, no shared expert):
    router [n_experts x hidden] q8, experts gate/up [inter x hidden] and down
    [hidden x inter] in ffn_dtype."""
    H, ne, I = cfg["hidden"], moe["n_experts"], moe["inter"]
    s = lambda i: (seed * 1000033 + i) & 0xFFFFFFFFFFFFFFFF
    if moe.get("router_dtype", "q8") == "f16":  # the reference converter keeps routers at f16
        rv = normal(s(1), ne * H, moe.get("router_sigma", 0.1)).astype(np.float16)
        router = {"dtype": 1, "rows": ne, "cols": H, "q": None, "row_scale": None, "bytes": rv.view(np.uint8)}
    else:
        router = q8_normal(s(1), ne, H, moe.get("router_sigma", 0.1))
    return {"router": router, "top_k": moe["top_k"],
            "norm_topk": moe.get("norm_topk", True), "routed_scaling": moe.get("routed_scaling", 1.0),
            "experts": [{"gate": _w(ffn_dtype, s(10 + 3 * e), I, H, sigma), "up": _w(ffn_dtype, s(11 + 3 * e), I, H, sigma),
                         "down": _w(ffn_dtype, s(12 + 3 * e), H, I, sigma)} for e in range(ne)]}


def synth_model(cfg=None, seed=1, attn_dtype=DT_Q8ROW, ffn_dtype=DT_Q4T, mtp=True, sigma=0.02,
                norm_noise=0.0, moe=None):
    """Random-init Qwen3-arch weights: N(0, sigma^2) then quantized (attention
    q8, FFN q4t; lm_head, tied embedding and eh_proj q8).  moe = {"n_experts",
    "top_k", "inter", "layers": [indices], optional "router_dtype": "q8" |
    "f16"} makes those layers' FFNs routed experts (Qwen3-MoE); the MTP
    block stays dense."""
    cfg = dict(QWEN3_06B if cfg is None else cfg)
    m = {"cfg": cfg}
    m["layers"] = [_layer(cfg, seed * 131 + li, attn_dtype, ffn_dtype, sigma, norm_noise)
                   for li in range(cfg["n_layers"])]
    if moe:
        for li in moe["layers"]:
            L = m["layers"][li]
            for n in ("gate", "up", "down"):
                del L[n]
            L["moe"] = _moe(cfg, seed * 131 + li, moe, ffn_dtype, sigma)
    m["lm_head"] = q8_normal(seed * 7 + 3, cfg["vocab"], cfg["hidden"], sigma)
    m["final_norm"] = _norm(seed * 7 + 4, cfg["hidden"], norm_noise)
    if mtp:
        H = cfg["hidden"]
        m["mtp"] = {
            "enorm": _norm(seed * 7 + 5, H, norm_noise), "hnorm": _norm(seed * 7 + 6, H, norm_noise),
            "eh_proj": q8_normal(seed * 7 + 8, H, 2 * H, sigma),
            "layer": _layer(cfg, seed * 131 + 99991, attn_dtype, ffn_dtype, sigma, norm_noise),
            "norm": _norm(seed * 7 + 9, H, norm_noise),
        }
    return m


def accept_model(cfg, seed=5, sigma=0.05, norm_noise=0.1, eh_noise=10.0, logit_scale=8.0):
    """A synthetic model whose MTP head drafts tokens the trunk accepts.

    Random-init trunks with a tied embedding fall into runs of one token
    (the tied lm_head favours the input's own row); this head repeats its
    input token: eh_proj = [I | noise] acts as the identity on the
    normalised embedding half, plus int8 noise of std `eh_noise` (/127) on
    every entry, which lets the hidden half and the MTP block move the
    draft (at eh_noise 30 no draft survives).  logit_scale multiplies the
    final and MTP norms, so temperature-0.8 distributions are peaked
    enough to accept draws.  Used to put the speculative accept, commit
    and re-warm paths under test (rounds with 0 < a < K)."""
    sm = synth_model(cfg, seed=seed, sigma=sigma, norm_noise=norm_noise)
    H = sm["cfg"]["hidden"]
    noise = normal(seed * 7 + 11, H * 2 * H, eh_noise).reshape(H, 2 * H)
    q = np.clip(np.round(noise), -127, 127).astype(np.int8)
    q[np.arange(H), np.arange(H)] = 127
    sm["mtp"]["eh_proj"] = tensor(DT_Q8ROW, H, 2 * H, q=q, row_scale=np.full(H, 1.0 / 127.0, np.float32))
    sm["final_norm"] = (sm["final_norm"] * logit_scale).astype(np.float32)
    sm["mtp"]["norm"] = (sm["mtp"]["norm"] * logit_scale).astype(np.float32)
    return sm


def constant_head_model(cfg, seed=5, sigma=0.05):
    """The reference's speculative_accepts_constant_oracle model
    (pipeline.rs:11567-11587): every lm_head row equal, so every logit ties
    and both the trunk and the draft head pick the highest id."""
    sm = synth_model(cfg, seed=seed, sigma=sigma)
    V, H = sm["cfg"]["vocab"], sm["cfg"]["hidden"]
    sm["lm_head"] = tensor(DT_Q8ROW, V, H, q=np.full((V, H), 1, np.int8), row_scale=np.full(V, 0.01, np.float32))
    return sm
