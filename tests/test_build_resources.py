"""Every gfx950 kernel of libcmfhip must run without scratch (private
memory) spills: a spilling kernel is slow, and a large per-lane scratch size
can exceed the scratch aperture at full occupancy."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "cmf_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def _resources(name):
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--offload-device-only", "-x", "hip", "-c", os.path.join(SRC, name), "-o",
           os.devnull, "-Rpass-analysis=kernel-resource-usage"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out, cur = {}, None
    for line in r.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and cur:
            out[cur] = int(m.group(1))
    return out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("name", sorted(f for f in os.listdir(SRC) if f.endswith(".hip")))
def test_no_scratch(name):
    res = _resources(name)
    bad = {k: v for k, v in res.items() if v > 0}
    assert not bad, f"kernels with scratch spills in {name}: {bad}"
