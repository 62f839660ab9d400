"""Device MoE FFN (libcmfhip cmf_moe_*): the reference's MoeFfn layer
(pipeline.rs:10868-11045) with device routing (moe_route,
pipeline.rs:10780-10841) for a verify batch, and moe_block (gpu.rs:2482) for
caller-routed jobs of one token."""
import ctypes as C

import numpy as np

from . import CmfError, _ptr, check, lib
from .model import _tensor


class MoE:
    def __init__(self, n_experts, hidden, inter, top_k, experts, norm_topk=True, routed_scaling=1.0):
        """experts: per expert a dict with "gate", "up", "down" tensors (synth
        tensor dicts in quant.rs layouts)."""
        self.ne, self.hidden, self.inter, self.top_k = n_experts, hidden, inter, top_k
        h = C.c_void_p()
        check(lib().cmf_moe_create(n_experts, hidden, inter, top_k, 1 if norm_topk else 0, routed_scaling,
                                   C.byref(h)))
        self.h = h
        for e, ex in enumerate(experts):
            keep = []
            g, u, d = _tensor(ex["gate"], keep), _tensor(ex["up"], keep), _tensor(ex["down"], keep)
            if not check(lib().cmf_moe_set_expert(self.h, e, C.byref(g), C.byref(u), C.byref(d))):
                raise CmfError(f"expert {e}: codec declined by the device")

    def ffn(self, x, router_logits):
        """moe_ffn for b tokens: returns (out [b][hidden], idx [b][top_k], w [b][top_k])."""
        x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
        lg = np.ascontiguousarray(np.atleast_2d(router_logits), dtype=np.float32)
        b = x.shape[0]
        out = np.empty((b, self.hidden), np.float32)
        idx = np.empty((b, self.top_k), np.int32)
        w = np.empty((b, self.top_k), np.float32)
        check(lib().cmf_moe_ffn(self.h, _ptr(x), _ptr(lg), b, _ptr(out), _ptr(idx), _ptr(w)))
        return out, idx, w

    def block(self, x, experts, weights):
        """moe_block: one token, caller-routed (experts, weights)."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        ex = np.ascontiguousarray(experts, dtype=np.int32)
        ws = np.ascontiguousarray(weights, dtype=np.float32)
        out = np.empty(self.hidden, np.float32)
        check(lib().cmf_moe_block(self.h, _ptr(x), _ptr(ex), _ptr(ws), len(ex), _ptr(out)))
        return out

    def free(self):
        if self.h:
            lib().cmf_moe_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
