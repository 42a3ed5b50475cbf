"""Builds libmamba_ss.so, the HIP selective-scan library, for gfx950.

``python -m mamba_amd.build`` (or ``build()``) compiles every source under
``mamba_amd/csrc`` with hipcc (one object per source, in parallel) and links
them into ``mamba_amd/_lib/libmamba_ss.so``.  The library is built in-tree
so that it travels with the source tree.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "_lib")
OBJ_DIR = os.path.join(LIB_DIR, "obj")
LIB_PATH = os.path.join(LIB_DIR, "libmamba_ss.so")
ARCH = os.environ.get("MAMBA_AMD_ARCH", "gfx950")
SOURCES = ["ss_api.hip", "ss_fwd.hip", "ss_bwd.hip", "conv1d.hip", "rms_norm.hip", "decode.hip", "decode_linear.hip"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def compile_flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        # packed fp32 VALU ops are disabled on purpose: the scan is written in
        # scalar fp32 and must not be vectorised into v_pk_* forms
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
        "-I", os.path.join(HERE, "..", "include"),
    ]


def build_command(out=LIB_PATH):
    """One hipcc command that compiles and links everything (for reference)."""
    return [hipcc()] + compile_flags() + ["-shared", "-o", out] + [os.path.join(CSRC, s) for s in SOURCES]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{res.stderr[-8000:]}")


def build(verbose=False, jobs=None):
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    objs = [os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[cc] + compile_flags() + ["-c", "-o", o, os.path.join(CSRC, s)] for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
