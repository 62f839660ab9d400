"""The C ABI boundary on the CPU: libcmfhip.so loads, exports every entry
point include/cmf_hip.h declares (and the Python mirror binds exactly those),
and the library reports errors instead of crashing when no GPU is present."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cmf_hip.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    return sorted(set(re.findall(r"\b(cmf_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_seam():
    names = _declared()
    for n in ("cmf_q8_matvec_range", "cmf_q8_matmat", "cmf_q4t_matvec", "cmf_q4t_matmat", "cmf_q4tp_matvec",
              "cmf_q4tp_matmat", "cmf_ffn", "cmf_prefill", "cmf_decode", "cmf_forward_batch", "cmf_kv_truncate",
              "cmf_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import cmf_amd
    L = cmf_amd.lib()
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert not missing, missing


def test_python_mirror_binds_exactly_the_header():
    import cmf_amd
    assert sorted(n for n in cmf_amd.SIGNATURES if n.startswith("cmf_") and not n.startswith("cmf_synth_")) \
        == _declared()


def test_no_gpu_is_an_error_not_a_crash():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import cmf_amd
    L = cmf_amd.lib()
    assert L.cmf_init(0) < 0
    assert len(L.cmf_last_error()) > 0
