"""ctypes bindings of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker / CPU baseline, never by the
product package cmf_amd.  The C sources restate the reference CPU path of
infosave2007/cmf and cite it file:line (see oracle.h).
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
DT_Q8ROW, DT_Q4T, DT_Q4TP = 3, 11, 15


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class QT(C.Structure):
    _fields_ = [("dtype", C.c_int), ("rows", C.c_int), ("cols", C.c_int), ("q", C.c_void_p),
                ("row_scale", C.c_void_p), ("bytes", C.c_void_p)]


class Cfg(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("hidden", C.c_int), ("n_heads", C.c_int), ("n_kv", C.c_int),
                ("head_dim", C.c_int), ("inter", C.c_int), ("vocab", C.c_int), ("max_seq", C.c_int),
                ("rope_theta", C.c_float), ("eps", C.c_double)]


class Layer(C.Structure):
    _fields_ = [("input_norm", C.c_void_p), ("post_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("wq", QT), ("wk", QT), ("wv", QT), ("wo", QT), ("gate", QT),
                ("up", QT), ("down", QT), ("n_experts", C.c_int), ("top_k", C.c_int), ("norm_topk", C.c_int),
                ("routed_scaling", C.c_float), ("router", QT), ("experts", C.c_void_p)]


class Model(C.Structure):
    _fields_ = [("cfg", Cfg), ("layers", C.c_void_p), ("lm_head", QT), ("final_norm", C.c_void_p),
                ("has_mtp", C.c_int), ("enorm", C.c_void_p), ("hnorm", C.c_void_p), ("mtp_norm", C.c_void_p),
                ("eh_proj", QT), ("mtp", Layer), ("threads", C.c_int), ("embed", QT), ("a8w8", C.c_int),
                ("fast", C.c_int), ("batch_verify", C.c_int)]


class KV(C.Structure):
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("len", C.c_int)]


class State(C.Structure):
    _fields_ = [("trunk", C.c_void_p), ("mtp", KV), ("inv_freq", C.c_void_p)]


class SamplerCfg(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("repetition_penalty", C.c_float), ("min_p", C.c_float), ("presence_penalty", C.c_float)]


class GenCfg(C.Structure):
    _fields_ = [("spec", C.c_int), ("k", C.c_int), ("sc", SamplerCfg), ("seed", C.c_uint64)]


class Rng(C.Structure):
    """or_rng: SplitMix64 state; seq/nseq replace its uniforms in order."""
    _fields_ = [("state", C.c_uint64), ("seq", C.c_void_p), ("nseq", C.c_int), ("used", C.c_int)]


class GenStats(C.Structure):
    _fields_ = [("drafted", C.c_int), ("accepted", C.c_int), ("rounds", C.c_int), ("hist", C.c_int * 17)]


_lib = None
P = C.c_void_p


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        sig = {
            "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_f32_to_f16": (C.c_uint16, [C.c_float]),
            "or_dequant_q8_row": (None, [P, C.c_int, C.c_int, P]),
            "or_dequant_q4t": (None, [P, C.c_size_t, P]),
            "or_q4tp_code": (C.c_int, [P, C.c_size_t, C.c_size_t]),
            "or_q4tp_put_code": (None, [P, C.c_size_t, C.c_int]),
            "or_q4tp_ladder": (None, [P, C.c_size_t, P]),
            "or_dequant_q4tp": (None, [P, C.c_int, C.c_int, P]),
            "or_matvec": (None, [C.POINTER(QT), P, P, C.c_int]),
            "or_matmat": (None, [C.POINTER(QT), P, C.c_int, P, C.c_int]),
            "or_matvec_a8w8": (None, [C.POINTER(QT), P, P, C.c_int]),
            "or_matmat_a8w8": (None, [C.POINTER(QT), P, C.c_int, P, C.c_int]),
            "or_fast_supported": (C.c_int, []),
            "or_fast_matmat_a8w8": (C.c_int, [C.POINTER(QT), P, C.c_int, P, C.c_int]),
            "or_split_act": (C.c_int, [P, C.c_int, P, P, P, P, P]),
            "or_rng_next_u64": (C.c_uint64, [P]),
            "or_rng_next_f32": (C.c_float, [P]),
            "or_argmax": (C.c_uint32, [P, C.c_int]),
            "or_sparse_distribution": (C.c_int, [P, C.c_int, C.POINTER(SamplerCfg), P, C.c_int, P, P]),
            "or_draw_sparse": (C.c_uint32, [P, P, C.c_int, P]),
            "or_spec_accept_sparse": (C.c_int64, [P, P, C.c_int, P, P, C.c_int, C.c_uint32, P]),
            "or_spec_accept_dense": (C.c_int64, [P, P, C.c_int, C.c_uint32, P]),
            "or_categorical": (C.c_uint32, [P, C.c_int, C.c_float]),
            "or_sample": (C.c_uint32, [P, C.c_int, C.POINTER(SamplerCfg), P, C.c_int, P]),
            "or_rms_norm": (None, [P, P, C.c_int, C.c_double, P]),
            "or_rope_inv_freq": (None, [C.c_int, C.c_float, P]),
            "or_embed": (None, [C.POINTER(Model), C.c_uint32, P]),
            "or_forward": (None, [C.POINTER(Model), C.POINTER(State), P, C.c_int]),
            "or_logits": (None, [C.POINTER(Model), P, P]),
            "or_mtp_step": (None, [C.POINTER(Model), C.POINTER(State), P, C.c_uint32, C.c_int, P, P]),
            "or_generate": (C.c_int, [C.POINTER(Model), C.POINTER(State), P, C.c_int, C.c_int,
                                      C.POINTER(GenCfg), P, C.POINTER(GenStats)]),
            "or_decode": (C.c_int, [C.POINTER(Model), C.POINTER(State), P, C.c_int, P, C.c_int, C.c_int,
                                    C.POINTER(GenCfg), P, P, C.POINTER(GenStats)]),
            "or_verify_step": (C.c_int, [C.POINTER(Model), C.POINTER(State), P, C.c_int, P, C.c_int,
                                         C.POINTER(SamplerCfg), P, P, P, C.c_int, C.POINTER(Rng), P, C.c_int,
                                         C.c_int, P, P, P]),
            "or_moe_route": (C.c_int, [P, C.c_int, C.c_int, C.c_int, C.c_float, P, P]),
            "or_moe_ffn": (None, [P, C.c_int, C.c_int, C.c_int, C.c_float, P, P, C.c_int, P, C.c_int]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def qt(t, keep):
    q = rs = b = None
    if t.get("q") is not None:
        q = np.ascontiguousarray(t["q"], dtype=np.int8)
        rs = np.ascontiguousarray(t["row_scale"], dtype=np.float32)
        keep += [q, rs]
    if t.get("bytes") is not None:
        b = np.ascontiguousarray(t["bytes"], dtype=np.uint8)
        keep.append(b)
    return QT(t["dtype"], t["rows"], t["cols"], _p(q), _p(rs), _p(b))


def fast_supported():
    """True when the host has AVX-512 VNNI (the timing arm can run)."""
    return bool(lib().or_fast_supported())


def matmat(t, xs, threads=8, a8w8=False, fast=False):
    """Reference matmul [b][rows]: the exact contract, or a8w8 (the batch
    order of the reference's x86 VNNI arms); fast=True runs a8w8 through the
    AVX-512 VNNI timing arm, which must give the same values."""
    keep = []
    w = qt(t, keep)
    xs = np.ascontiguousarray(np.atleast_2d(xs), dtype=np.float32)
    b = xs.shape[0]
    out = np.empty((b, t["rows"]), dtype=np.float32)
    if fast:
        if lib().or_fast_matmat_a8w8(C.byref(w), _p(xs), b, _p(out), threads) != 0:
            raise RuntimeError("the VNNI timing arm needs AVX-512 VNNI and a quantized tensor")
    elif a8w8:
        lib().or_matmat_a8w8(C.byref(w), _p(xs), b, _p(out), threads)
    else:
        lib().or_matmat(C.byref(w), _p(xs), b, _p(out), threads)
    return out


def _f32(a, keep):
    a = np.ascontiguousarray(a, dtype=np.float32)
    keep.append(a)
    return _p(a)


def _layer(l, keep):
    dense = "moe" not in l
    empty = QT(0, 0, 0, None, None, None)
    L = Layer(_f32(l["input_norm"], keep), _f32(l["post_norm"], keep), _f32(l["q_norm"], keep),
              _f32(l["k_norm"], keep), qt(l["wq"], keep), qt(l["wk"], keep), qt(l["wv"], keep),
              qt(l["wo"], keep), qt(l["gate"], keep) if dense else empty, qt(l["up"], keep) if dense else empty,
              qt(l["down"], keep) if dense else empty)
    if not dense:
        mo = l["moe"]
        ex = (QT * (3 * len(mo["experts"])))(*[qt(e[n], keep) for e in mo["experts"] for n in ("gate", "up", "down")])
        keep.append(ex)
        L.n_experts = len(mo["experts"])
        L.top_k = mo["top_k"]
        L.norm_topk = 1 if mo.get("norm_topk", True) else 0
        L.routed_scaling = mo.get("routed_scaling", 1.0)
        r = mo["router"]
        if r["dtype"] in (1, 2):  # f16 / bf16 file tensor: widened to f32 at load (load_matrix)
            raw = np.ascontiguousarray(r["bytes"], dtype=np.uint8).view(np.uint16)
            f = raw.view(np.float16).astype(np.float32) if r["dtype"] == 1 else \
                (raw.astype(np.uint32) << 16).view(np.float32)
            r = {"dtype": 0, "rows": r["rows"], "cols": r["cols"], "q": None, "row_scale": None,
                 "bytes": np.ascontiguousarray(f).view(np.uint8)}
        L.router = qt(r, keep)
        L.experts = C.cast(ex, C.c_void_p)
    return L


class OracleModel:
    """The CPU reference model over the same synthetic arrays the GPU uses."""

    def __init__(self, sm, threads=8, a8w8=False, fast=False, batch_verify=False):
        c = sm["cfg"]
        self.c = c
        self.sm = sm
        self.keep = []
        layers = (Layer * c["n_layers"])(*[_layer(l, self.keep) for l in sm["layers"]])
        self.keep.append(layers)
        m = Model()
        m.cfg = Cfg(c["n_layers"], c["hidden"], c["n_heads"], c["n_kv"], c["head_dim"], c["inter"], c["vocab"],
                    c["max_seq"], c["rope_theta"], c["eps"])
        m.layers = C.cast(layers, C.c_void_p)
        m.lm_head = qt(sm["lm_head"], self.keep)
        if "embed" in sm:  # untied embedding table
            m.embed = qt(sm["embed"], self.keep)
        m.final_norm = _f32(sm["final_norm"], self.keep)
        m.threads = threads
        m.a8w8 = 1 if a8w8 else 0
        m.fast = 1 if fast else 0
        m.batch_verify = 1 if batch_verify else 0
        if "mtp" in sm:
            mt = sm["mtp"]
            m.has_mtp = 1
            m.enorm = _f32(mt["enorm"], self.keep)
            m.hnorm = _f32(mt["hnorm"], self.keep)
            m.mtp_norm = _f32(mt["norm"], self.keep)
            m.eh_proj = qt(mt["eh_proj"], self.keep)
            m.mtp = _layer(mt["layer"], self.keep)
        self.m = m
        self.reset()

    def reset(self, kv_len=0, mtp_len=0):
        c = self.c
        shape = (c["n_kv"], c["max_seq"], c["head_dim"])
        self.kk = [np.zeros(shape, np.float32) for _ in range(c["n_layers"] + 1)]
        self.vv = [np.zeros(shape, np.float32) for _ in range(c["n_layers"] + 1)]
        self.kvs = (KV * c["n_layers"])(*[KV(_p(self.kk[i]), _p(self.vv[i]), kv_len) for i in range(c["n_layers"])])
        self.inv = np.empty(c["head_dim"] // 2, np.float32)
        lib().or_rope_inv_freq(c["head_dim"], c["rope_theta"], _p(self.inv))
        self.st = State(C.cast(self.kvs, C.c_void_p), KV(_p(self.kk[-1]), _p(self.vv[-1]), mtp_len), _p(self.inv))

    def import_kv(self, li, k, v):
        """Load rows [0, n) of layer li (-1: MTP) from [n_kv][n][hd] arrays."""
        i = li if li >= 0 else self.c["n_layers"]
        n = k.shape[1]
        self.kk[i][:, :n] = k
        self.vv[i][:, :n] = v
        if li >= 0:
            self.kvs[li].len = n
        else:
            self.st.mtp.len = n

    def generate(self, prompt, max_tokens, spec=True, k=4, sampler=None, seed=0):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        sc = sampler or SamplerCfg(0.0, 0.9, 40, 1.0, 0.05, 0.0)
        g = GenCfg(1 if spec else 0, k, sc, seed)
        out = np.zeros(max_tokens + k + 2, np.uint32)
        st = GenStats()
        n = lib().or_generate(C.byref(self.m), C.byref(self.st), _p(prompt), len(prompt), max_tokens, C.byref(g),
                              _p(out), C.byref(st))
        return out[:n].astype(np.int32), st

    def decode(self, hidden, next_pos, ids, max_tokens, spec=True, k=4, sampler=None, seed=0):
        hidden = np.ascontiguousarray(hidden, dtype=np.float32).copy()
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        sc = sampler or SamplerCfg(0.0, 0.9, 40, 1.0, 0.05, 0.0)
        g = GenCfg(1 if spec else 0, k, sc, seed)
        out = np.zeros(max_tokens + k + 2, np.uint32)
        st = GenStats()
        rs = C.c_uint64(seed)
        n = lib().or_decode(C.byref(self.m), C.byref(self.st), _p(hidden), next_pos, _p(ids), len(ids), max_tokens,
                            C.byref(g), C.byref(rs), _p(out), C.byref(st))
        return out[:n].astype(np.int32), st

    def verify_step(self, hidden, pos0, tokens, sampler=None, q=None, uniforms=None, seed=0, past=None,
                    warm_tip=True):
        """or_verify_step: returns (a, next, hidden row a, argmax [b], logits
        [b][vocab]).  q = (ids [b-1][S], probs [b-1][S], n [b-1]) for
        sampling; uniforms replace the seeded stream's draws in order."""
        V = self.c["vocab"]
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        b = len(tokens)
        hidden = np.ascontiguousarray(hidden, dtype=np.float32).copy()
        sc = sampler or SamplerCfg(0.0, 0.9, 40, 1.0, 0.05, 0.0)
        keep = []
        qi = qp = qn = None
        stride = 0
        if q is not None:
            qi = np.ascontiguousarray(q[0], dtype=np.uint32)
            qp = np.ascontiguousarray(q[1], dtype=np.float32)
            qn = np.ascontiguousarray(q[2], dtype=np.int32)
            stride = qi.shape[1]
        u = None if uniforms is None else np.ascontiguousarray(uniforms, dtype=np.float32)
        rng = Rng(seed, _p(u), 0 if u is None else len(u), 0)
        past = np.ascontiguousarray(tokens[:1] if past is None else past, dtype=np.uint32)
        am = np.empty(b, np.uint32)
        lg = np.empty((b, V), np.float32)
        nxt = C.c_uint32(0)
        a = lib().or_verify_step(C.byref(self.m), C.byref(self.st), _p(hidden), pos0, _p(tokens), b, C.byref(sc),
                                 _p(qi), _p(qp), _p(qn), stride, C.byref(rng), _p(past), len(past),
                                 1 if warm_tip else 0, _p(lg), _p(am), C.byref(nxt))
        self.rng_used = rng.used
        return a, int(nxt.value), hidden, am.astype(np.int32), lg

    def kv(self, li):
        """(k, v) rows [0, len) of layer li (-1: the MTP block), [n_kv][len][hd]."""
        i = li if li >= 0 else self.c["n_layers"]
        n = self.kvs[li].len if li >= 0 else self.st.mtp.len
        return self.kk[i][:, :n].copy(), self.vv[i][:, :n].copy()

    def prefill(self, prompt):
        """prompt positions through the trunk + MTP warm pairs; returns the tip hidden"""
        h = None
        for p, t in enumerate(prompt):
            h = self.forward(int(t), p)
            if "mtp" in self.sm and p + 1 < len(prompt):
                lib().or_mtp_step(C.byref(self.m), C.byref(self.st), _p(h), int(prompt[p + 1]), p, None, None)
        return h

    def forward(self, tok, pos):
        h = np.empty(self.c["hidden"], np.float32)
        lib().or_embed(C.byref(self.m), tok, _p(h))
        lib().or_forward(C.byref(self.m), C.byref(self.st), _p(h), pos)
        return h

    def logits(self, h):
        out = np.empty(self.c["vocab"], np.float32)
        lib().or_logits(C.byref(self.m), _p(np.ascontiguousarray(h, np.float32)), _p(out))
        return out


def moe_route(logits, top_k, norm_topk=True, routed_scaling=1.0):
    """moe_route (pipeline.rs:10780-10841): (idx [k], w [k]) for one token."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.empty(max(top_k, 1), np.int32)
    w = np.empty(max(top_k, 1), np.float32)
    k = lib().or_moe_route(_p(lg), len(lg), top_k, 1 if norm_topk else 0, routed_scaling, _p(idx), _p(w))
    return idx[:k], w[:k]


def moe_ffn_rows(experts, top_k, router_logits, xs, norm_topk=True, routed_scaling=1.0, threads=8):
    """moe_ffn_cpu for each row of a batch (the experts marshalled once)."""
    keep = []
    arr = (QT * (3 * len(experts)))(*[qt(ex[n], keep) for ex in experts for n in ("gate", "up", "down")])
    lg = np.ascontiguousarray(router_logits, dtype=np.float32)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    out = np.empty((xs.shape[0], experts[0]["down"]["rows"]), np.float32)
    for i in range(xs.shape[0]):
        lib().or_moe_ffn(C.cast(arr, C.c_void_p), len(experts), top_k, 1 if norm_topk else 0, routed_scaling,
                         _p(lg[i]), _p(xs[i]), xs.shape[1], _p(out[i]), threads)
    return out


def moe_ffn(experts, top_k, router_logits, x, norm_topk=True, routed_scaling=1.0, threads=8):
    """moe_ffn_cpu for one token: experts = [{"gate", "up", "down"}, ...]."""
    keep = []
    arr = (QT * (3 * len(experts)))(*[qt(ex[n], keep) for ex in experts for n in ("gate", "up", "down")])
    lg = np.ascontiguousarray(router_logits, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(experts[0]["down"]["rows"], np.float32)
    lib().or_moe_ffn(C.cast(arr, C.c_void_p), len(experts), top_k, 1 if norm_topk else 0, routed_scaling, _p(lg), _p(x), len(x),
                     _p(out), threads)
    return out
