"""Build libcmfhip.so (gfx950) in-tree with hipcc.

    python -m cmf_amd.build            # compile every source, link the library

Objects go to cmf_amd/_build/, the library to cmf_amd/libcmfhip.so.  Every
HIP source is compiled with packed FP32 disabled (no v_pk_*_f32).
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcmfhip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-function", "-Wno-unused-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources():
    return sorted(f for f in os.listdir(SRC) if f.endswith((".hip", ".cpp")))


def _compile(name):
    src = os.path.join(SRC, name)
    obj = os.path.join(OUT, name + ".o")
    lang = ["-x", "hip"] if name.endswith(".hip") else []
    cmd = [HIPCC] + FLAGS + lang + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 target feature: harmless
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32" not in l)
    return name, r.returncode, err, obj


def build(verbose=True):
    os.makedirs(OUT, exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        for name, rc, err, obj in ex.map(_compile, sources()):
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {name}:\n{err}")
            if err.strip() and verbose:
                print(err, file=sys.stderr)
            objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
