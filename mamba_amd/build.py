"""Builds libmamba_ss.so, the HIP selective-scan library, for gfx950.

``python -m mamba_amd.build`` (or ``build()``) compiles every source under
``mamba_amd/csrc`` with hipcc into ``mamba_amd/_lib/libmamba_ss.so``.  The
library is built in-tree so that it travels with the source tree.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libmamba_ss.so")
ARCH = os.environ.get("MAMBA_AMD_ARCH", "gfx950")
SOURCES = ["ss_api.hip", "ss_fwd.hip", "ss_bwd.hip", "conv1d.hip", "rms_norm.hip", "decode.hip", "decode_linear.hip"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build_command(out=LIB_PATH):
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # packed fp32 VALU ops are disabled on purpose: the scan is written in
        # scalar fp32 and must not be vectorised into v_pk_* forms
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
        "-I", os.path.join(HERE, "..", "include"),
        "-o", out,
    ] + [os.path.join(CSRC, s) for s in SOURCES]


def build(verbose=False):
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = build_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
