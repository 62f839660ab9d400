"""Test-side .cmf v2 writer and hash64 (test infrastructure, not product code).

An independent restatement of the reference writer `CmfModel::write_ref`
(crates/cortiq-core/src/format.rs:1165-1332) and `encode_directory`
(:1334-1360), and of hash64 (crates/cortiq-core/src/hash.rs:18-35), used to
build the files the native reader (csrc/container.cpp) is checked on.
`hash64_py` is pinned by the reference's cross-implementation vectors
(crates/cortiq-core/tests/roundtrip.rs:227-233).
"""
import json
import struct

import numpy as np

MASK64 = (1 << 64) - 1
MAGIC = b"CMF\x01"
VERSION = 2
ENVELOPE_LEN, RECORD_LEN = 128, 56
DATA_ALIGN, TENSOR_ALIGN, LARGE_MIN, LARGE_ALIGN = 4096, 64, 16 * 1024, 4096
F_TENSOR_DIR, F_BINARY_MASKS, F_QUANT_2F = 1, 2, 4


def _fmix64(x):
    x ^= x >> 33
    x = (x * 0xFF51AFD7ED558CCD) & MASK64
    x ^= x >> 33
    x = (x * 0xC4CEB9FE1A85EC53) & MASK64
    x ^= x >> 33
    return x


def hash64_py(b):
    """hash.rs:18-35 in plain Python (vectorised over the full words)."""
    b = bytes(b)
    n = len(b)
    full = n // 8
    acc = 0
    if full:
        w = np.frombuffer(b[: full * 8], dtype="<u8").astype(np.uint64)
        with np.errstate(over="ignore"):
            x = w.copy()
            x ^= x >> np.uint64(33)
            x *= np.uint64(0xFF51AFD7ED558CCD)
            x ^= x >> np.uint64(33)
            x *= np.uint64(0xC4CEB9FE1A85EC53)
            x ^= x >> np.uint64(33)
            x ^= np.arange(full, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
        acc = int(np.bitwise_xor.reduce(x))
    rem = n % 8
    if rem:
        w8 = b[full * 8:] + bytes(8 - rem)
        acc ^= _fmix64(struct.unpack("<Q", w8)[0]) ^ ((full * 0x9E3779B97F4A7C15) & MASK64)
    acc ^= n
    return _fmix64(acc & MASK64)


def _align(x, a):
    return (x + a - 1) // a * a


def encode_directory(entries):
    """entries: (name, dtype, shape, off, nbytes, hash) -> directory bytes."""
    pool = b""
    recs = []
    pool_off = 16 + len(entries) * RECORD_LEN
    for name, dtype, shape, off, nbytes, h in entries:
        nb = name.encode("utf-8")
        dims = list(shape) + [0] * (6 - len(shape))
        recs.append(struct.pack("<IHBB6IQQQ", len(pool), len(nb), dtype, len(shape), *dims, off, nbytes, h))
        pool += nb
    return struct.pack("<QQ", len(entries), pool_off) + b"".join(recs) + pool


def write(path, header, tensors, masks=None, vocab=None, index=None, features=None):
    """header: dict (CmfHeader JSON); tensors: [(name, dtype, shape, bytes)].
    masks / index are opaque section bytes here.  Returns the entries."""
    entries = []
    cur = 0
    for name, dtype, shape, data in tensors:
        data = bytes(data)
        cur = _align(cur, LARGE_ALIGN if len(data) >= LARGE_MIN else TENSOR_ALIGN)
        entries.append((name, dtype, tuple(shape), cur, len(data), hash64_py(data)))
        cur += len(data)
    data_len = cur
    dir_bytes = encode_directory(entries)
    header = dict(header)
    if masks is not None or vocab is not None or index is not None:
        sh = {}
        for k, v in (("masks", masks), ("vocab", vocab), ("index", index)):
            if v is not None:
                sh[k] = f"{hash64_py(v):016x}"
        header["section_hashes"] = sh
    hj = json.dumps(header, separators=(",", ":")).encode("utf-8")
    req = F_TENSOR_DIR
    if masks is not None:
        req |= F_BINARY_MASKS
    if any(t[1] in (8, 9) for t in tensors):
        req |= F_QUANT_2F
    if features is not None:
        req = features
    header_off = ENVELOPE_LEN
    dir_off = header_off + len(hj)
    data_off = _align(dir_off + len(dir_bytes), DATA_ALIGN)
    secs = [(header_off, len(hj)), (dir_off, len(dir_bytes)), (data_off, data_len)]
    pos = data_off + data_len
    for blob in (masks, vocab, index):
        n = 0 if blob is None else len(blob)
        secs.append((pos if n else 0, n))
        pos += n
    env = MAGIC + struct.pack("<III", VERSION, 0, req)
    for off, ln in secs:
        env += struct.pack("<QQ", off, ln)
    env += struct.pack("<QQ", hash64_py(hj), hash64_py(dir_bytes))
    env += bytes(ENVELOPE_LEN - len(env))
    with open(path, "wb") as f:
        f.write(env)
        f.write(hj)
        f.write(dir_bytes)
        f.write(bytes(data_off - (dir_off + len(dir_bytes))))
        p = 0
        for (name, dtype, shape, data), e in zip(tensors, entries):
            f.write(bytes(e[3] - p))
            f.write(bytes(data))
            p = e[3] + len(bytes(data))
        for blob in (masks, vocab, index):
            if blob is not None:
                f.write(bytes(blob))
    return entries


# --------------------------------------------------------------------------
# reference encoders (crates/cortiq-core/tests/roundtrip.rs:84-121)
# --------------------------------------------------------------------------
def encode_q8_row(vals, rows, cols):
    """int8 quants, then f16 row scales (absmax/127, 1e-10 for a zero row;
    round half away from zero, clamp to [-128, 127])."""
    v = np.asarray(vals, dtype=np.float32).reshape(rows, cols)
    am = np.abs(v).max(axis=1)
    sc = np.where(am == 0, np.float32(1e-10), am / np.float32(127.0)).astype(np.float32)
    r = v / sc[:, None]
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + 0.5), -128, 127).astype(np.int8)
    return q.tobytes() + sc.astype(np.float16).tobytes()


def f16_bytes(vals):
    return np.asarray(vals, dtype=np.float32).astype(np.float16).tobytes()


def bf16_bytes(vals):
    """round-to-nearest-even f32 -> bf16 (finite inputs)."""
    u = np.asarray(vals, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r.tobytes()


# --------------------------------------------------------------------------
# a synthetic model dict (cmf_amd.synth.synth_model) as a .cmf file
# --------------------------------------------------------------------------
def arch_of(cfg, mtp=True, tie=True, **extra):
    a = {"arch_name": "qwen3", "hidden_size": cfg["hidden"], "intermediate_size": cfg["inter"],
         "num_layers": cfg["n_layers"], "num_attention_heads": cfg["n_heads"], "num_kv_heads": cfg["n_kv"],
         "head_dim": cfg["head_dim"], "vocab_size": cfg["vocab"],
         "layer_types": ["FullAttention"] * cfg["n_layers"], "rms_norm_eps": cfg["eps"],
         "norm_style": "qwen", "rope_theta": cfg["rope_theta"], "tie_word_embeddings": tie,
         "partial_rotary_factor": 1.0, "max_position_embeddings": cfg["max_seq"],
         "linear_conv_kernel_dim": None, "linear_num_key_heads": None, "linear_num_value_heads": None}
    if mtp:
        a["mtp"] = {"num_layers": 1, "share_lm_head": True, "share_embed": True}
    a.update(extra)
    return a


def header_of(arch):
    return {"format": "cmf", "version": VERSION, "arch": arch, "quant_type": "Q8_ROW"}


def round_q8_scales(t):
    """The tensor with its q8 row scales rounded to f16 (the file's form)."""
    if t["dtype"] == 3:
        t = dict(t, row_scale=np.asarray(t["row_scale"], np.float32).astype(np.float16).astype(np.float32))
    return t


def f16_model(sm):
    """The synthetic model with every q8 row scale rounded to f16."""
    def layer(l):
        out = {k: round_q8_scales(v) if isinstance(v, dict) and k != "moe" else v for k, v in l.items()}
        if "moe" in l:
            mo = l["moe"]
            out["moe"] = dict(mo, router=round_q8_scales(mo["router"]),
                              experts=[{k: round_q8_scales(v) for k, v in ex.items()} for ex in mo["experts"]])
        return out
    out = dict(sm, layers=[layer(l) for l in sm["layers"]], lm_head=round_q8_scales(sm["lm_head"]))
    if "embed" in sm:
        out["embed"] = round_q8_scales(sm["embed"])
    if "mtp" in sm:
        mt = sm["mtp"]
        out["mtp"] = dict(mt, eh_proj=round_q8_scales(mt["eh_proj"]), layer=layer(mt["layer"]))
    return out


def _mat(t):
    if t["dtype"] == 3:
        q = np.ascontiguousarray(t["q"], dtype=np.int8)
        return t["dtype"], q.tobytes() + np.asarray(t["row_scale"], np.float32).astype(np.float16).tobytes()
    return t["dtype"], bytes(np.asarray(t["bytes"], np.uint8))


def model_tensors(sm, norm_dtype=0):
    """[(name, dtype, shape, bytes)] of a model dict under the reference's
    Qwen3 names (loader.rs); norms as f32 (0), f16 (1) or bf16 (2)."""
    enc = {0: lambda v: np.asarray(v, np.float32).tobytes(), 1: f16_bytes, 2: bf16_bytes}[norm_dtype]
    out = []

    def vec(name, v):
        out.append((name, norm_dtype, (len(v),), enc(v)))

    def mat(name, t):
        dt, b = _mat(t)
        out.append((name, dt, (t["rows"], t["cols"]), b))

    def layer(p, l):
        vec(p + "input_layernorm.weight", l["input_norm"])
        vec(p + "post_attention_layernorm.weight", l["post_norm"])
        vec(p + "self_attn.q_norm.weight", l["q_norm"])
        vec(p + "self_attn.k_norm.weight", l["k_norm"])
        for k, n in (("wq", "q_proj"), ("wk", "k_proj"), ("wv", "v_proj"), ("wo", "o_proj")):
            mat(p + f"self_attn.{n}.weight", l[k])
        if "moe" in l:  # router (as stored: q8 or f16) + experts by index
            mo = l["moe"]
            mat(p + "mlp.gate.weight", mo["router"])
            for e, ex in enumerate(mo["experts"]):
                for k in ("gate", "up", "down"):
                    mat(p + f"mlp.experts.{e}.{k}_proj.weight", ex[k])
            return
        for k in ("gate", "up", "down"):
            mat(p + f"mlp.{k}_proj.weight", l[k])

    if "embed" in sm:
        mat("model.embed_tokens.weight", sm["embed"])
        mat("lm_head.weight", sm["lm_head"])
    else:
        mat("model.embed_tokens.weight", sm["lm_head"])
    for i, l in enumerate(sm["layers"]):
        layer(f"model.layers.{i}.", l)
    vec("model.norm.weight", sm["final_norm"])
    if "mtp" in sm:
        mt = sm["mtp"]
        vec("model.mtp.enorm.weight", mt["enorm"])
        vec("model.mtp.hnorm.weight", mt["hnorm"])
        mat("model.mtp.eh_proj.weight", mt["eh_proj"])
        layer("model.mtp.layers.0.", mt["layer"])
        vec("model.mtp.norm.weight", mt["norm"])
    return out


def write_model(path, sm, norm_dtype=0, **arch_extra):
    moe = next((l["moe"] for l in sm["layers"] if "moe" in l), None)
    if moe is not None and "moe" not in arch_extra:
        arch_extra["moe"] = {"num_experts": len(moe["experts"]), "top_k": moe["top_k"],
                             "moe_intermediate_size": moe["experts"][0]["gate"]["rows"],
                             "norm_topk_prob": bool(moe.get("norm_topk", True))}
    arch = arch_of(sm["cfg"], mtp="mtp" in sm, tie="embed" not in sm, **arch_extra)
    return write(path, header_of(arch), model_tensors(sm, norm_dtype))
