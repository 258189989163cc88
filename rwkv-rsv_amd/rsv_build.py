"""Builds librsv_hip.so (HIP backend, C-ABI) and librsv_host.so (C++ model
driver) in-tree for gfx950 with hipcc.  Object files are rebuilt only when a
source or header is newer than the object, unless force=True."""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "_build")
ROOT = os.path.dirname(HERE)
INC = os.path.join(ROOT, "include")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", INC, "-I", CSRC,
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result", "-Wno-unused-value"]
COMMON += os.environ.get("RSV_EXTRA_FLAGS", "").split()

BACKEND_SRCS = ["backend.cpp", "k_gemv.hip", "k_wkv.hip", "k_misc.hip", "k_sample.hip", "k_gemm.hip",
                "k_skinny.hip", "k_sparse.hip"]
HOST_SRCS = ["host.cpp"]


def _headers():
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs += [os.path.join(INC, f) for f in os.listdir(INC) if f.endswith(".h")]
    return hs


def _compile(src, force):
    s = os.path.join(CSRC, src)
    o = os.path.join(OUT, src + ".o")
    newest = max([os.path.getmtime(s)] + [os.path.getmtime(h) for h in _headers()])
    if not force and os.path.exists(o) and os.path.getmtime(o) >= newest:
        return o
    lang = ["-x", "hip"] if src.endswith((".hip", ".cpp")) else []
    cmd = [HIPCC] + COMMON + lang + ["-c", s, "-o", o]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return o


def build(force=False, jobs=8):
    os.makedirs(OUT, exist_ok=True)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), BACKEND_SRCS + HOST_SRCS))
    back = objs[: len(BACKEND_SRCS)]
    host = objs[len(BACKEND_SRCS):]
    out = os.environ.get("RSV_BUILD_OUT")  # another directory for the libraries (experiments)
    lib = os.path.join(out or OUT, "librsv_hip.so")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib] + back
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    hlib = os.path.join(out or OUT, "librsv_host.so")
    cmd = [HIPCC, "-shared", "-fPIC", "-o", hlib] + host + ["-L", OUT, "-lrsv_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    return lib, hlib


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
