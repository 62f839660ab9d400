"""Qwen3-arch weights from a .cmf file into the device model.

Follows the dense full-attention arm of the reference loader
(crates/cortiq-engine/src/loader.rs: top-level weights :714-724, attention
`load_full_attn` :819-, FFN `build_ffn_at`, the MTP block :1140-1211) and
`QTensor::from_model` (crates/cortiq-engine/src/qtensor.rs:182-349) for the
matrix formats the MI355X kernels serve:
  q8_row      -> int8 rows + row scales (f16 in the file, f32 after load)
  q4_tiled    -> the payload as stored
  q4_tiled_p  -> the payload as stored
Norm vectors may be f32, f16 or bf16 (converted to f32 as dequant_tensor
does).  A file this engine cannot run (other architectures or layer kinds,
other matrix formats, an MTP stack of more than one block) is refused with a
CmfError that names what is missing; nothing is converted silently.
"""
import numpy as np

from . import DT_Q4T, DT_Q4TP, DT_Q8ROW, CmfError
from .container import CmfFile, MissingTensor, dequant_vector

# arch fields whose non-default values this engine does not implement
# (ModelArch, cortiq-core/src/types.rs:346-520): name -> the default
_DEFAULTS = {
    "norm_style": "qwen", "partial_rotary_factor": 1.0, "yarn": None, "attention_heads_per_layer": None,
    "hidden_act": "silu", "embed_multiplier": 1.0, "query_pre_attn_scalar": None, "sliding_window": None,
    "sliding_window_pattern": None, "rope_local_base_freq": None, "local_partial_rotary_factor": None,
    "global_head_dim": None, "num_global_kv_heads": None, "global_partial_rotary_factor": None,
    "final_logit_softcapping": None, "mla": None, "activation_situ_beta": None,
    "activation_situ_linear_beta": None, "attn_logit_softcapping": None, "attn_v_norm": False,
    "linear_core": None, "head_clusters": None, "rope_freq_factors": None, "logit_multiplier": None,
    "g3n": None, "kda_gate_lower_bound": None, "num_loops": 1, "loop_final_norm": False,
}
_REQUIRED = ("hidden_size", "intermediate_size", "num_layers", "num_attention_heads", "num_kv_heads", "head_dim",
             "vocab_size", "layer_types", "rms_norm_eps", "max_position_embeddings")


def check_arch(arch):
    """The model config of a supported arch, else CmfError."""
    for k in _REQUIRED:
        if k not in arch:
            raise CmfError(f"header arch: missing field `{k}`")
    bad = [k for k, d in _DEFAULTS.items() if arch.get(k, d) != d]
    if bad:
        raise CmfError("this engine runs dense full-attention Qwen3-style models; unsupported arch fields: " +
                       ", ".join(f"{k}={arch[k]!r}" for k in bad))
    lt = arch["layer_types"]
    if len(lt) != arch["num_layers"] or any(t != "FullAttention" for t in lt):
        raise CmfError("this engine runs full-attention layers only (layer_types)")
    moe = arch.get("moe")
    if moe is not None:
        # MoeConfig (cortiq-core/src/types.rs:251-281): the Qwen3-MoE subset
        bad = [k for k, d in (("shared_expert_intermediate_size", None), ("router_sigmoid", False),
                              ("router_resonance", False)) if moe.get(k, d) != d]
        if bad:
            raise CmfError("this engine runs softmax-routed experts without a shared expert; unsupported "
                           "arch.moe fields: " + ", ".join(f"{k}={moe[k]!r}" for k in bad))
        for k in ("num_experts", "top_k", "moe_intermediate_size"):
            if k not in moe:
                raise CmfError(f"header arch.moe: missing field `{k}`")
    return {"n_layers": int(arch["num_layers"]), "hidden": int(arch["hidden_size"]),
            "n_heads": int(arch["num_attention_heads"]), "n_kv": int(arch["num_kv_heads"]),
            "head_dim": int(arch["head_dim"]), "inter": int(arch["intermediate_size"]),
            "vocab": int(arch["vocab_size"]), "max_seq": int(arch["max_position_embeddings"]),
            "rope_theta": float(arch.get("rope_theta", 10000.0)), "eps": float(arch["rms_norm_eps"])}


def matrix(f, name, shape=None, dense_ok=False):
    """One weight matrix in the model-dict form (QTensor::from_model);
    dense_ok: an f32 / f16 / bf16 tensor is kept as stored (MoE routers,
    which the reference converter writes at f16)."""
    e = f.tensor(name)
    if e is None:
        raise MissingTensor(f"tensor '{name}' not found in CMF directory")
    if len(e.shape) != 2:
        raise CmfError(f"QTensor::from_model needs 2-D, got '{name}'")
    rows, cols = e.shape
    if shape is not None and (rows, cols) != tuple(shape):
        raise CmfError(f"tensor '{name}': shape {[rows, cols]}, expected {list(shape)}")
    raw = f.entry_bytes(e)
    if dense_ok and e.dtype in (0, 1, 2):  # f32 / f16 / bf16 kept as stored (widened to f32 on upload)
        return {"dtype": e.dtype, "rows": rows, "cols": cols, "q": None, "row_scale": None, "bytes": raw}
    if e.dtype == DT_Q8ROW:
        n = rows * cols
        q = raw[:n].view(np.int8).reshape(rows, cols)
        rs = raw[n: n + 2 * rows].view("<u2").view(np.float16).astype(np.float32)
        return {"dtype": DT_Q8ROW, "rows": rows, "cols": cols, "q": q, "row_scale": rs, "bytes": None}
    if e.dtype in (DT_Q4T, DT_Q4TP) and cols % 32 == 0:
        return {"dtype": e.dtype, "rows": rows, "cols": cols, "q": None, "row_scale": None, "bytes": raw}
    raise CmfError(f"tensor '{name}': dtype {e.dtype_name} is not served by the MI355X kernels "
                   "(q8_row, q4_tiled, q4_tiled_p)")


def vector(f, name, n):
    e = f.tensor(name)
    if e is None:
        raise MissingTensor(f"tensor '{name}' not found in CMF directory")
    if e.n_elems != n:
        raise CmfError(f"tensor '{name}': {e.n_elems} values, expected {n}")
    return dequant_vector(e, f.entry_bytes(e))


def _layer(f, p, c, arch=None):
    H, hd, nh, nkv, I = c["hidden"], c["head_dim"], c["n_heads"], c["n_kv"], c["inter"]
    return {
        "input_norm": vector(f, p + "input_layernorm.weight", H),
        "post_norm": vector(f, p + "post_attention_layernorm.weight", H),
        "q_norm": vector(f, p + "self_attn.q_norm.weight", hd),
        "k_norm": vector(f, p + "self_attn.k_norm.weight", hd),
        "wq": matrix(f, p + "self_attn.q_proj.weight", (nh * hd, H)),
        "wk": matrix(f, p + "self_attn.k_proj.weight", (nkv * hd, H)),
        "wv": matrix(f, p + "self_attn.v_proj.weight", (nkv * hd, H)),
        "wo": matrix(f, p + "self_attn.o_proj.weight", (H, nh * hd)),
        **_ffn(f, p, c, arch),
    }


def _ffn(f, p, c, arch):
    """The block's FFN (build_ffn_at, loader.rs:~200-400): routed experts
    when `mlp.gate.weight` (the router) is present, else dense SwiGLU."""
    H, I = c["hidden"], c["inter"]
    if arch is None or f.tensor(p + "mlp.gate.weight") is None:
        return {"gate": matrix(f, p + "mlp.gate_proj.weight", (I, H)),
                "up": matrix(f, p + "mlp.up_proj.weight", (I, H)),
                "down": matrix(f, p + "mlp.down_proj.weight", (H, I))}
    mc = arch.get("moe")
    if mc is None:
        raise CmfError(f"{p}mlp.gate.weight present but header has no arch.moe block")
    for extra in ("mlp.shared_expert.gate_proj.weight", "mlp.expert_bias"):
        if f.tensor(p + extra) is not None:
            raise CmfError(f"{p}{extra}: shared experts and selection biases are not run by this engine")
    Ie = int(mc["moe_intermediate_size"])
    experts = []
    for e in range(int(mc["num_experts"])):  # by tensor presence up to the header count (loader.rs)
        q = f"{p}mlp.experts.{e}."
        if f.tensor(q + "gate_proj.weight") is None:
            break
        experts.append({"gate": matrix(f, q + "gate_proj.weight", (Ie, H)),
                        "up": matrix(f, q + "up_proj.weight", (Ie, H)),
                        "down": matrix(f, q + "down_proj.weight", (H, Ie))})
    if not experts:
        raise CmfError(f"{p}: router present but no expert tensors")
    router = matrix(f, p + "mlp.gate.weight", (len(experts), H), dense_ok=True)
    return {"moe": {"router": router, "experts": experts, "top_k": int(mc["top_k"]),
                    "norm_topk": bool(mc.get("norm_topk_prob", False)),
                    "routed_scaling": float(mc.get("routed_scaling_factor") or 1.0)}}


def load(f, max_seq=None):
    """The model dict `cmf_amd.model.Model` takes, read from a CmfFile (or a
    path, opened with open_sharded).  Tensor payloads stay views of the file
    mapping until the model uploads them.  max_seq caps the KV capacity
    (default: the arch's max_position_embeddings)."""
    if not isinstance(f, CmfFile):
        f = CmfFile.open_sharded(f)
    c = check_arch(f.arch)
    if max_seq is not None:
        c["max_seq"] = min(c["max_seq"], int(max_seq))
    H, V = c["hidden"], c["vocab"]
    m = {"cfg": c, "file": f}
    m["layers"] = [_layer(f, f"model.layers.{i}.", c, f.arch) for i in range(c["n_layers"])]
    m["final_norm"] = vector(f, "model.norm.weight", H)
    embed = matrix(f, "model.embed_tokens.weight", (V, H))
    if f.tensor("lm_head.weight") is not None:
        m["lm_head"] = matrix(f, "lm_head.weight", (V, H))
        m["embed"] = embed
    elif f.arch.get("tie_word_embeddings", False):
        m["lm_head"] = embed
    else:
        raise MissingTensor("tensor 'lm_head.weight (and tie_word_embeddings is false)' not found")
    mtp_cfg = f.arch.get("mtp")
    present = f.tensor("model.mtp.layers.0.self_attn.q_proj.weight") is not None or \
        f.tensor("model.mtp.eh_proj.weight") is not None
    if mtp_cfg is not None and present:
        if int(mtp_cfg.get("num_layers", 0)) != 1:
            raise CmfError(f"MTP with {mtp_cfg.get('num_layers')} blocks not supported yet (only 1)")
        if not mtp_cfg.get("share_lm_head", True) or not mtp_cfg.get("share_embed", True):
            raise CmfError("this engine runs an MTP head that shares the embedding and lm_head")
        p = "model.mtp."
        m["mtp"] = {"enorm": vector(f, p + "enorm.weight", H), "hnorm": vector(f, p + "hnorm.weight", H),
                    "eh_proj": matrix(f, p + "eh_proj.weight", (H, 2 * H)),
                    "layer": _layer(f, p + "layers.0.", c), "norm": vector(f, p + "norm.weight", H)}
    return m
