"""cmf_amd — MI355X (gfx950) backend for the cortiq decode hot path.

Python mirror of the engine's GPU backend seam (crates/cortiq-engine/src/gpu.rs
of infosave2007/cmf) over the C ABI of libcmfhip.so (include/cmf_hip.h).
The seam functions keep the reference's names and meaning: they return True
when the GPU did the work and False when it declined (the caller then runs its
CPU path); genuine failures raise CmfError.  There is no CPU fallback inside
this package: if libcmfhip.so is missing, importing the library raises.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# CMF_LIB: another build of the library (A/B timing of two builds on one box)
LIB_PATH = os.environ.get("CMF_LIB") or os.path.join(_HERE, "libcmfhip.so")

DT_Q8ROW, DT_Q4T, DT_Q4TP = 3, 11, 15


class CmfError(RuntimeError):
    pass


_lib = None


def lib():
    """The loaded libcmfhip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise CmfError(f"{LIB_PATH} is missing: run `python -m cmf_amd.build` (hipcc, gfx950)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class ModelConfig(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("hidden", C.c_int), ("n_heads", C.c_int), ("n_kv", C.c_int),
                ("head_dim", C.c_int), ("inter", C.c_int), ("vocab", C.c_int), ("max_seq", C.c_int),
                ("rope_theta", C.c_float), ("eps", C.c_double)]


class Tensor(C.Structure):
    _fields_ = [("dtype", C.c_int), ("rows", C.c_int), ("cols", C.c_int),
                ("q", C.c_void_p), ("row_scale", C.c_void_p), ("bytes", C.c_void_p)]


class LayerDesc(C.Structure):
    _fields_ = [("input_norm", C.c_void_p), ("post_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("wq", Tensor), ("wk", Tensor), ("wv", Tensor), ("wo", Tensor),
                ("gate", Tensor), ("up", Tensor), ("down", Tensor)]


class SamplerConfig(C.Structure):
    """SamplerConfig (sampler.rs:88-121); defaults as Default::default()."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_uint32),
                ("repetition_penalty", C.c_float), ("min_p", C.c_float), ("presence_penalty", C.c_float)]

    def __init__(self, temperature=0.7, top_p=0.9, top_k=40, repetition_penalty=1.1, min_p=0.05,
                 presence_penalty=0.0):
        super().__init__(temperature, top_p, top_k, repetition_penalty, min_p, presence_penalty)


class MoeJob(C.Structure):
    """cmf_moe_job: one caller-routed expert trio (MoeJob, gpu.rs:814-841)."""
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
                ("gate_row_scale", C.c_void_p), ("up_row_scale", C.c_void_p), ("down_row_scale", C.c_void_p),
                ("xs_gate", C.c_void_p), ("xs_up", C.c_void_p), ("down_col", C.c_void_p), ("w", C.c_float),
                ("q1", C.c_int), ("q4t", C.c_int), ("q4tp", C.c_int), ("gu_q2", C.c_int),
                ("swiglu_limit", C.c_float)]


class BatchJob(C.Structure):
    """cmf_batch_job: one independent matvec (BatchJob, gpu.rs:843-864)."""
    _fields_ = [("w", C.c_void_p), ("rows", C.c_int), ("cols", C.c_int), ("row_scale", C.c_void_p),
                ("xs", C.c_void_p), ("layout", C.c_int)]


class GenStats(C.Structure):
    _fields_ = [("generated", C.c_int), ("drafted", C.c_int), ("accepted", C.c_int), ("rounds", C.c_int),
                ("device_ms", C.c_double)]


class SpecState(C.Structure):
    """cmf_spec_state: the speculation monitor of a model's last decode
    (SpecMon and its trial, pipeline.rs:642-694)."""
    _fields_ = [("round_ms", C.c_double), ("tokens", C.c_double), ("plain_ms", C.c_double), ("n", C.c_int),
                ("fails", C.c_int), ("phase", C.c_int), ("trial_rounds", C.c_int), ("gen0", C.c_int),
                ("recheck_at", C.c_int), ("t0_ms", C.c_double), ("spec_rounds", C.c_int), ("plain_steps", C.c_int)]

    PHASES = ("trial", "plain trial", "speculating", "plain")

    @property
    def phase_name(self):
        return self.PHASES[self.phase]


class FileSections(C.Structure):
    """cmf_file_sections: the envelope of an open .cmf file."""
    _fields_ = [("required_features", C.c_uint32), ("off", C.c_uint64 * 6), ("len", C.c_uint64 * 6),
                ("header_hash", C.c_uint64), ("dir_hash", C.c_uint64), ("base", C.c_void_p),
                ("file_len", C.c_uint64)]


class FileTensor(C.Structure):
    """cmf_file_tensor: one tensor directory record."""
    _fields_ = [("name", C.c_void_p), ("name_len", C.c_int), ("dtype", C.c_int), ("ndim", C.c_int),
                ("shape", C.c_uint64 * 6), ("off", C.c_uint64), ("nbytes", C.c_uint64), ("hash", C.c_uint64),
                ("shard", C.c_int), ("data", C.c_void_p)]


# every symbol include/cmf_hip.h declares, with its ctypes signature
_P, _I, _F, _S, _U64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint64
SIGNATURES = {
    "cmf_last_error": (C.c_char_p, []),
    "cmf_init": (_I, [_I]),
    "cmf_device_count": (_I, []),
    "cmf_sync": (_I, []),
    "cmf_weight_upload": (_I, [_P, _S, _I, _I, _I, C.POINTER(_P)]),
    "cmf_weight_upload_q8": (_I, [_P, _P, _I, _I, C.POINTER(_P)]),
    "cmf_weight_free": (_I, [_P]),
    "cmf_weight_device_bytes": (_S, [_P]),
    "cmf_q8_matvec_range": (_I, [_P, _I, _P, _P, _I, _I, _P]),
    "cmf_q8_matmat": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "cmf_moe_block_jobs": (_I, [C.POINTER(MoeJob), _I, _P]),
    "cmf_matvec_batch": (_I, [C.POINTER(BatchJob), _I, C.POINTER(_P)]),
    "cmf_matmat_a8w8": (_I, [_P, _P, _I, _P]),
    "cmf_q4t_matvec": (_I, [_P, _P, _I, _I, _P]),
    "cmf_q4t_matmat": (_I, [_P, _P, _I, _I, _I, _P]),
    "cmf_q4tp_matvec": (_I, [_P, _P, _I, _I, _P]),
    "cmf_q4tp_matmat": (_I, [_P, _P, _I, _I, _I, _P]),
    "cmf_ffn": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "cmf_dev_alloc": (_P, [_S]),
    "cmf_dev_free": (_I, [_P]),
    "cmf_h2d": (_I, [_P, _P, _S]),
    "cmf_d2h": (_I, [_P, _P, _S]),
    "cmf_prep_bytes": (_S, [_P]),
    "cmf_prep_dev": (_I, [_P, _P, _I, _I, _P, _P]),
    "cmf_gemv_prepared": (_I, [_P, _P, _P, _I, _P, _I, _I]),
    "cmf_gemv_dev_noalloc": (_I, [_P, _P, _I, _I, _P, _I]),
    "cmf_time_gemv": (_I, [C.POINTER(_P), _I, _P, _P, _I, _P, _I, _I, _I, _I, C.POINTER(_F)]),
    "cmf_time_copy": (_I, [_S, _I, _I, C.POINTER(_F)]),
    "cmf_time_read": (_I, [_S, _I, _I, C.POINTER(_F)]),
    "cmf_time_attention": (_I, [_P, _I, _I, _I, _I, C.POINTER(_F)]),
    "cmf_time_gemv_rows": (_I, [C.POINTER(_P), _I, _P, _I, _P, _I, _P, _I, _I, _I, _I, C.POINTER(_F)]),
    "cmf_time_gemm": (_I, [_P, _P, _I, _P, _I, _I, C.POINTER(_F)]),
    "cmf_moe_create": (_I, [_I, _I, _I, _I, _I, _F, C.POINTER(_P)]),
    "cmf_moe_free": (_I, [_P]),
    "cmf_moe_set_expert": (_I, [_P, _I, C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor)]),
    "cmf_moe_ffn": (_I, [_P, _P, _P, _I, _P, _P, _P]),
    "cmf_moe_ffn_dev": (_I, [_P, _P, _P, _I, _P]),
    "cmf_moe_block": (_I, [_P, _P, _P, _P, _I, _P]),
    "cmf_time_moe": (_I, [_P, _P, _P, _I, _P, _I, _I, C.POINTER(_F)]),
    "cmf_model_create": (_I, [C.POINTER(ModelConfig), C.POINTER(_P)]),
    "cmf_model_free": (_I, [_P]),
    "cmf_model_set_layer": (_I, [_P, _I, C.POINTER(LayerDesc)]),
    "cmf_model_set_head": (_I, [_P, C.POINTER(Tensor), _P]),
    "cmf_model_set_layer_moe": (_I, [_P, _I, C.POINTER(LayerDesc), C.POINTER(Tensor), _P]),
    "cmf_model_set_mtp": (_I, [_P, _P, _P, C.POINTER(Tensor), C.POINTER(LayerDesc), _P]),
    "cmf_model_fused_blocks": (_I, [_P]),
    "cmf_model_prefill_xcd": (_I, [_P]),
    "cmf_model_xl_fallbacks": (_I, [_P]),
    "cmf_prefill": (_I, [_P, _P, _I]),
    "cmf_decode": (_I, [_P, _I, C.POINTER(SamplerConfig), _U64, _I, _I, _P, C.POINTER(GenStats)]),
    "cmf_decode_begin": (_I, [_P, C.POINTER(SamplerConfig), _U64]),
    "cmf_spec_monitor": (_I, [_P, C.POINTER(SpecState)]),
    "cmf_decode_rounds": (_I, [_P, _I, _I, _I, C.POINTER(GenStats)]),
    "cmf_decode_tokens": (_I, [_P, _P, _I]),
    "cmf_forward_batch": (_I, [_P, _P, _I, _I, _P, _P]),
    "cmf_kv_truncate": (_I, [_P, _I]),
    "cmf_verify_step": (_I, [_P, _P, _I, _I, C.POINTER(SamplerConfig), _P, _P, _P, _P, _P, _P, C.POINTER(_I),
                             C.POINTER(_I)]),
    "cmf_sparse_distribution": (_I, [_P, _P, C.POINTER(SamplerConfig), _P, _P]),
    "cmf_state_get": (_I, [_P, C.POINTER(_I), _P]),
    "cmf_kv_export": (_I, [_P, _I, _I, _P, _P]),
    "cmf_model_set_embed": (_I, [_P, C.POINTER(Tensor)]),
    # .cmf container (csrc/container.cpp)
    "cmf_hash64": (_U64, [_P, _S]),
    "cmf_file_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "cmf_file_close": (_I, [_P]),
    "cmf_file_info": (_I, [_P, C.POINTER(FileSections)]),
    "cmf_file_count": (_I, [_P]),
    "cmf_file_entry": (_I, [_P, _I, C.POINTER(FileTensor)]),
    "cmf_file_find": (_I, [_P, C.c_char_p, _S]),
    "cmf_file_attach_shard": (_I, [_P, _P]),
    "cmf_file_verify": (_I, [_P, _P, C.c_char_p, _S, C.POINTER(_I)]),
    # host-only synthetic data generators (csrc/synth.cpp)
    "cmf_synth_normal": (None, [_U64, C.c_int64, _F, _P]),
    "cmf_synth_q8_uniform": (None, [_U64, _I, _I, _P, _P]),
    "cmf_synth_q4t_uniform": (None, [_U64, _I, _I, _F, _P]),
    "cmf_synth_q4tp_uniform": (None, [_U64, _I, _I, _F, _F, _P]),
    "cmf_synth_q8_normal": (None, [_U64, _I, _I, _F, _P, _P]),
    "cmf_synth_q4t_normal": (None, [_U64, _I, _I, _F, _P]),
    "cmf_synth_ids": (None, [_U64, _I, _I, _P]),
}


def _declare(L):
    for name, (res, args) in SIGNATURES.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def check(rc):
    """0 -> True (done), >0 -> False (declined), <0 -> CmfError."""
    if rc < 0:
        raise CmfError(lib().cmf_last_error().decode())
    return rc == 0


def init(device=0):
    check(lib().cmf_init(device))


def device_count():
    return lib().cmf_device_count()


# --------------------------------------------------------------------------
# weights
# --------------------------------------------------------------------------
class Weight:
    """A device-resident quantized tensor (the reference's resident weight,
    keyed here by handle instead of (model, idx))."""

    def __init__(self, dtype, rows, cols, payload=None, q=None, row_scale=None):
        self.dtype, self.rows, self.cols = dtype, rows, cols
        h = C.c_void_p()
        if dtype == DT_Q8ROW and q is not None:
            q = np.ascontiguousarray(q, dtype=np.int8)
            rs = np.ascontiguousarray(row_scale, dtype=np.float32)
            check(lib().cmf_weight_upload_q8(_ptr(q), _ptr(rs), rows, cols, C.byref(h)))
        else:
            payload = np.ascontiguousarray(payload, dtype=np.uint8)
            check(lib().cmf_weight_upload(_ptr(payload), payload.nbytes, dtype, rows, cols, C.byref(h)))
        self.h = h

    @property
    def device_bytes(self):
        return lib().cmf_weight_device_bytes(self.h)

    def free(self):
        if self.h:
            lib().cmf_weight_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _seam_out(rows, b=1):
    return np.empty((b, rows), dtype=np.float32)


def _f32_or_none(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def q8_matvec_range(w, row0, xs, rows, cols, out, row_scale=None):
    """gpu.rs:1104 — rows [row0, row0+rows) of q8 w times xs into out, with
    the caller's row scales [rows] (None: the upload-time ones)."""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    rs = _f32_or_none(row_scale)
    return check(lib().cmf_q8_matvec_range(w.h, row0, _ptr(rs), _ptr(xs), rows, cols, _ptr(out)))


def q8_matmat(w, xs, b, rows, cols, out, row_scale=None):
    """gpu.rs:1155 — out[b*rows + r]."""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    rs = _f32_or_none(row_scale)
    return check(lib().cmf_q8_matmat(w.h, _ptr(rs), _ptr(xs), b, rows, cols, _ptr(out)))


def moe_block_jobs(jobs, hidden):
    """moe_block (gpu.rs:2482) over caller-routed jobs: each a dict with
    gate/up/down (Weight), xs_gate, xs_up, w and optionally *_row_scale,
    q1, q4t, q4tp, gu_q2, swiglu_limit, down_col.  Returns the [hidden]
    output, or None when declined."""
    keep = []

    def arr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=np.float32)
        keep.append(a)
        return _ptr(a)
    cj = (MoeJob * len(jobs))()
    for i, j in enumerate(jobs):
        cj[i] = MoeJob(j["gate"].h, j["up"].h, j["down"].h, arr(j.get("gate_row_scale")),
                       arr(j.get("up_row_scale")), arr(j.get("down_row_scale")), arr(j["xs_gate"]),
                       arr(j["xs_up"]), arr(j.get("down_col")), j["w"], int(j.get("q1", 0)), int(j.get("q4t", 0)),
                       int(j.get("q4tp", 0)), int(j.get("gu_q2", 0)), j.get("swiglu_limit", 0.0))
    out = np.zeros(hidden, np.float32)
    return out if check(lib().cmf_moe_block_jobs(cj, len(jobs), _ptr(out))) else None


def matvec_batch(jobs):
    """matvec_batch (gpu.rs:2494): jobs = [(Weight, xs, row_scale or None,
    layout)], returns the outputs, or None when declined."""
    keep = []
    cj = (BatchJob * len(jobs))()
    outs = [np.zeros(w.rows, np.float32) for w, _, _, _ in jobs]
    for i, (w, xs, rs, layout) in enumerate(jobs):
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        rs = _f32_or_none(rs)
        keep += [xs, rs]
        cj[i] = BatchJob(w.h, w.rows, w.cols, _ptr(rs), _ptr(xs), layout)
    po = (C.c_void_p * len(jobs))(*[_ptr(o) for o in outs])
    return outs if check(lib().cmf_matvec_batch(cj, len(jobs), po)) else None


def q4t_matvec(w, xs, rows, cols, out):
    """gpu.rs:2423"""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    return check(lib().cmf_q4t_matvec(w.h, _ptr(xs), rows, cols, _ptr(out)))


def q4t_matmat(w, xs, b, rows, cols, out):
    """gpu.rs:2439"""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    return check(lib().cmf_q4t_matmat(w.h, _ptr(xs), b, rows, cols, _ptr(out)))


def q4tp_matvec(w, xs, rows, cols, out):
    """gpu.rs:2400"""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    return check(lib().cmf_q4tp_matvec(w.h, _ptr(xs), rows, cols, _ptr(out)))


def q4tp_matmat(w, xs, b, rows, cols, out):
    """gpu.rs:2358"""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    return check(lib().cmf_q4tp_matmat(w.h, _ptr(xs), b, rows, cols, _ptr(out)))


def ffn(w1, w3, w2, xs, b, hidden, inter, out):
    """gpu.rs:1773/1794 q4t_ffn / q4tp_ffn: out = w2 (silu(w1 x) * w3 x)."""
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    return check(lib().cmf_ffn(w1.h, w3.h, w2.h, _ptr(xs), b, hidden, inter, _ptr(out)))


def matmul(w, xs):
    """Convenience: w * xs for xs [b][cols] (any b), returns [b][rows]."""
    xs = np.ascontiguousarray(np.atleast_2d(xs), dtype=np.float32)
    b = xs.shape[0]
    out = np.empty((b, w.rows), dtype=np.float32)
    fn = {DT_Q8ROW: q8_matmat, DT_Q4T: q4t_matmat, DT_Q4TP: q4tp_matmat}[w.dtype]
    if not fn(w, xs, b, w.rows, w.cols, out):
        raise CmfError("declined")
    return out


def matmul_a8w8(w, xs):
    """w * xs under the a8w8 contract (split_act operand, integer tile dots,
    exact outliers): xs [b][cols] (any b), returns [b][rows]."""
    xs = np.ascontiguousarray(np.atleast_2d(xs), dtype=np.float32)
    b = xs.shape[0]
    out = np.empty((b, w.rows), dtype=np.float32)
    check(lib().cmf_matmat_a8w8(w.h, _ptr(xs), b, _ptr(out)))
    return out


# --------------------------------------------------------------------------
# device buffers (plumbing for device-resident benchmarks; no torch needed)
# --------------------------------------------------------------------------
class DevBuf:
    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.p = lib().cmf_dev_alloc(self.nbytes)
        if not self.p:
            raise CmfError(lib().cmf_last_error().decode())

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(lib().cmf_h2d(self.p, _ptr(arr), arr.nbytes))

    def download(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype=dtype)
        check(lib().cmf_d2h(_ptr(out), self.p, out.nbytes))
        return out

    def free(self):
        if self.p:
            lib().cmf_dev_free(self.p)
            self.p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
