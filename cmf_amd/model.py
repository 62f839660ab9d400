"""The device-resident decode engine (libcmfhip cmf_model_*).

Mirrors the reference pipeline's decode entry points (pipeline.rs):
prefill (prompt positions + MTP warm), the speculative decode loop
(graph_spec_step rounds) or plain decode, and the batched verify forward
(forward_batch_graph)."""
import ctypes as C

import numpy as np

from . import (CmfError, GenStats, LayerDesc, ModelConfig, SamplerConfig, SpecState, Tensor, _ptr, check, lib)

SPARSE_CAP = 4 * 64 + 64  # CMF_SPARSE_CAP: entries of a sparse distribution list


def _tensor(t, keep):
    q = rs = b = None
    if t["q"] is not None:
        q = np.ascontiguousarray(t["q"], dtype=np.int8)
        rs = np.ascontiguousarray(t["row_scale"], dtype=np.float32)
        keep += [q, rs]
    if t["bytes"] is not None:
        b = np.ascontiguousarray(t["bytes"], dtype=np.uint8)
        keep.append(b)
    return Tensor(t["dtype"], t["rows"], t["cols"], _ptr(q), _ptr(rs), _ptr(b))


def _f32(a, keep):
    a = np.ascontiguousarray(a, dtype=np.float32)
    keep.append(a)
    return _ptr(a)


def _layer(l, keep):
    dense = "moe" not in l
    empty = Tensor(0, 0, 0, None, None, None)
    t = lambda n: _tensor(l[n], keep) if dense else empty
    return LayerDesc(_f32(l["input_norm"], keep), _f32(l["post_norm"], keep), _f32(l["q_norm"], keep),
                     _f32(l["k_norm"], keep), _tensor(l["wq"], keep), _tensor(l["wk"], keep),
                     _tensor(l["wv"], keep), _tensor(l["wo"], keep), t("gate"), t("up"), t("down"))


class Model:
    def __init__(self, sm):
        c = sm["cfg"]
        self.cfg = c
        mc = ModelConfig(c["n_layers"], c["hidden"], c["n_heads"], c["n_kv"], c["head_dim"], c["inter"],
                         c["vocab"], c["max_seq"], c["rope_theta"], c["eps"])
        h = C.c_void_p()
        check(lib().cmf_model_create(C.byref(mc), C.byref(h)))
        self.h = h
        self.moes = []  # the MoE layers the model borrows (freed after it)
        for li, l in enumerate(sm["layers"]):
            keep = []
            if "moe" in l:
                from .moe import MoE
                mo = l["moe"]
                ex = mo["experts"]
                moe = MoE(len(ex), c["hidden"], ex[0]["gate"]["rows"], mo["top_k"], ex,
                          norm_topk=mo.get("norm_topk", True), routed_scaling=mo.get("routed_scaling", 1.0))
                self.moes.append(moe)
                check(lib().cmf_model_set_layer_moe(self.h, li, C.byref(_layer(l, keep)),
                                                    C.byref(_tensor(mo["router"], keep)), moe.h))
                continue
            check(lib().cmf_model_set_layer(self.h, li, C.byref(_layer(l, keep))))
        keep = []
        check(lib().cmf_model_set_head(self.h, C.byref(_tensor(sm["lm_head"], keep)),
                                       _f32(sm["final_norm"], keep)))
        if "embed" in sm:  # untied embedding table
            keep = []
            check(lib().cmf_model_set_embed(self.h, C.byref(_tensor(sm["embed"], keep))))
        self.has_mtp = "mtp" in sm
        if self.has_mtp:
            mt, keep = sm["mtp"], []
            check(lib().cmf_model_set_mtp(self.h, _f32(mt["enorm"], keep), _f32(mt["hnorm"], keep),
                                          C.byref(_tensor(mt["eh_proj"], keep)),
                                          C.byref(_layer(mt["layer"], keep)), _f32(mt["norm"], keep)))

    @classmethod
    def from_cmf(cls, path, max_seq=None):
        """A model loaded from a .cmf file (or shard 1 of a sharded one)."""
        from .loader import load
        return cls(load(path, max_seq=max_seq))

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().cmf_prefill(self.h, _ptr(ids), len(ids)))

    def decode(self, max_tokens, sampler=None, seed=0, spec=True, k=4):
        """Returns (tokens, stats).  sampler=None is greedy.  spec: False
        (plain steps), True (speculative rounds throughout) or "auto" (the
        reference's speculation monitor decides, pipeline.rs:661-694;
        `monitor()` then reports its state)."""
        sc = sampler if sampler is not None else SamplerConfig(temperature=0.0, repetition_penalty=1.0)
        out = np.zeros(max_tokens + k + 2, dtype=np.int32)
        st = GenStats()
        mode = 2 if spec == "auto" else (1 if spec else 0)
        ok = check(lib().cmf_decode(self.h, max_tokens, C.byref(sc), seed, mode, k, _ptr(out), C.byref(st)))
        if not ok:
            raise CmfError("decode declined (penalised sampler config or top_k beyond the device sampler)")
        return out[: st.generated].copy(), st

    def monitor(self):
        """The speculation monitor of the last decode (cmf_spec_state)."""
        ms = SpecState()
        check(lib().cmf_spec_monitor(self.h, C.byref(ms)))
        return ms

    def decode_begin(self, sampler=None, seed=0):
        sc = sampler if sampler is not None else SamplerConfig(temperature=0.0, repetition_penalty=1.0)
        if not check(lib().cmf_decode_begin(self.h, C.byref(sc), seed)):
            raise CmfError("decode declined (penalised sampler config or top_k beyond the device sampler)")

    def decode_rounds(self, n, spec=True, k=4):
        st = GenStats()
        check(lib().cmf_decode_rounds(self.h, n, 1 if spec else 0, k, C.byref(st)))
        return st

    def tokens(self):
        out = np.zeros(self.cfg["max_seq"] + 32, dtype=np.int32)
        n = lib().cmf_decode_tokens(self.h, _ptr(out), len(out))
        if n < 0:
            check(n)
        return out[:n].copy()

    def forward_batch(self, tokens, pos0, want_logits=True):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        b = len(tokens)
        hid = np.empty((b, self.cfg["hidden"]), dtype=np.float32)
        lg = np.empty((b, self.cfg["vocab"]), dtype=np.float32) if want_logits else None
        check(lib().cmf_forward_batch(self.h, _ptr(tokens), b, pos0, _ptr(hid), _ptr(lg)))
        return hid, lg

    def verify_step(self, tokens, pos0, sampler=None, q=None, uniforms=None, want_logits=False):
        """cmf_verify_step: returns (accepted, next_token, argmax [b], logits
        [b][vocab] or None).  q = (ids [b-1][64], probs [b-1][64], n [b-1])
        and uniforms [b] for a sampled verify."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        b = len(tokens)
        keep = []
        qi = qp = qn = u = None
        if q is not None:
            # rows of CMF_SPARSE_CAP entries (narrower rows are padded)
            qi = np.zeros((b - 1, SPARSE_CAP), np.int32)
            qp = np.zeros((b - 1, SPARSE_CAP), np.float32)
            w = np.asarray(q[0]).shape[1]
            assert w <= SPARSE_CAP and np.asarray(q[1]).shape == (b - 1, w)
            qi[:, :w] = q[0]
            qp[:, :w] = q[1]
            qn = np.ascontiguousarray(q[2], dtype=np.int32)
        if uniforms is not None:
            u = np.zeros(b, np.float32)
            u[: len(uniforms)] = uniforms
        am = np.empty(b, np.int32)
        lg = np.empty((b, self.cfg["vocab"]), np.float32) if want_logits else None
        a, nxt = C.c_int(), C.c_int()
        rc = check(lib().cmf_verify_step(self.h, _ptr(tokens), b, pos0, C.byref(sampler) if sampler else None,
                                         _ptr(qi), _ptr(qp), _ptr(qn), _ptr(u), _ptr(am), _ptr(lg),
                                         C.byref(a), C.byref(nxt)))
        if not rc:
            raise CmfError("verify declined (sampler config beyond the device sampler)")
        return a.value, nxt.value, am, lg

    def sparse_distribution(self, logits, sampler):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        ids = np.empty(SPARSE_CAP, np.int32)
        pr = np.empty(SPARSE_CAP, np.float32)
        n = lib().cmf_sparse_distribution(self.h, _ptr(logits), C.byref(sampler), _ptr(ids), _ptr(pr))
        if n <= 0:
            check(n)
            raise CmfError("sparse_distribution declined")
        return ids[:n].copy(), pr[:n].copy()

    def kv_truncate(self, n):
        check(lib().cmf_kv_truncate(self.h, n))

    def state(self):
        np_ = C.c_int()
        hid = np.empty(self.cfg["hidden"], dtype=np.float32)
        check(lib().cmf_state_get(self.h, C.byref(np_), _ptr(hid)))
        return np_.value, hid

    def kv_export(self, li, n):
        c = self.cfg
        k = np.empty((c["n_kv"], n, c["head_dim"]), dtype=np.float32)
        v = np.empty_like(k)
        check(lib().cmf_kv_export(self.h, li, n, _ptr(k), _ptr(v)))
        return k, v

    def free(self):
        if getattr(self, "h", None):
            lib().cmf_model_free(self.h)
            self.h = None
        for moe in getattr(self, "moes", []):
            moe.free()
        self.moes = []

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
