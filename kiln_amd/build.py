"""Build recipe of libkiln_attn.so (gfx950 only), in-tree next to this file.

    python -m kiln_amd.build        # or: python kiln_amd/build.py

hipcc compiles every HIP source for gfx950 with packed-FP32 instruction selection disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops), then links one shared library.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkiln_attn.so")
HOST = os.path.join(HERE, "host")
DIT_LIB = os.path.join(HERE, "libkiln_dit.so")
DIT_SOURCES = ["dit.cpp", "sampler.cpp", "capi_dit.cpp"]
ENGINE = os.path.join(HERE, "kiln_engine")
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-honor-nans", "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


def _compile(src, where=CSRC):
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"]
    cmd = [HIPCC, *lang, *FLAGS, "-c", os.path.join(where, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass does not know the packed-fp32 target feature and says so: harmless
    return out


def build(verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    # the step driver (host C++ over the C ABI above), linked against libkiln_attn.so
    with ThreadPoolExecutor(max_workers=len(DIT_SOURCES)) as ex:
        dobjs = list(ex.map(lambda f: _compile(f, HOST), DIT_SOURCES))
    tmp = DIT_LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *dobjs, "-L" + HERE, "-lkiln_attn",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, DIT_LIB)
    if verbose:
        print("built", DIT_LIB)
    # the engine process (JSON-lines protocol) over the driver
    eobj = _compile("engine_main.cpp", HOST)
    tmp = ENGINE + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", eobj, "-L" + HERE, "-lkiln_dit", "-lkiln_attn", "-lpthread",
           "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, ENGINE)
    if verbose:
        print("built", ENGINE)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
