"""Build libgdn_hip.so (the C-ABI library in include/gdn.h) for gfx950 with hipcc.

    python -m linear_attention_op_amd.build        # or __graft_entry__.build()

Objects go to linear_attention_op_amd/_build/, the library to linear_attention_op_amd/libgdn_hip.so.  The HBM
stream probe (csrc/hbm_stream.hip), a measurement yardstick that only bench.py loads, becomes libgdn_stream.so.
The C host driver of the ABI (csrc/gdn_driver.c, plain C against include/gdn.h and the HIP runtime) becomes
linear_attention_op_amd/gdn_driver, linked to libgdn_hip.so beside it.
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgdn_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["gdn_linear.hip", "gdn_mixer.hip", "gdn_delta.hip", "gdn_chunk.hip", "gdn_api.cpp"]
STREAM_SOURCES = ["hbm_stream.hip"]
STREAM_LIB = os.path.join(HERE, "libgdn_stream.so")
DRIVER_SRC = os.path.join(CSRC, "gdn_driver.c")
DRIVER = os.path.join(HERE, "gdn_driver")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-result",
    # no packed fp32 VALU ops (v_pk_fma_f32 and friends): compile plain float code to scalar VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the gfx950 target feature above; that warning is expected noise
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _link(objs, lib, verbose):
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}", file=sys.stderr)


def _driver(verbose):
    tmp = DRIVER + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", DRIVER_SRC,
           "-o", tmp, f"-L{HERE}", "-lgdn_hip", f"-L{ROCM}/lib", "-lamdhip64", "-lm", "-Wl,-rpath,$ORIGIN",
           f"-Wl,-rpath,{ROCM}/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gcc failed for gdn_driver.c:\n{r.stderr}")
    if r.stderr.strip():
        print(r.stderr, file=sys.stderr)
    os.replace(tmp, DRIVER)
    if verbose:
        print(f"built {DRIVER}", file=sys.stderr)


def build(verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = SOURCES + STREAM_SOURCES
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(objs[:len(SOURCES)], LIB, verbose)
    _link(objs[len(SOURCES):], STREAM_LIB, verbose)
    _driver(verbose)
    return LIB


if __name__ == "__main__":
    build()
