"""CPU checks of the C ABI (libmamba_ss.so) and of the host side, no GPU.

* the library loads, reports its ABI version and exports every function
  that include/mamba_ss.h declares;
* the ctypes structs of mamba_amd/_native.py have the sizes and field offsets
  that a C compiler gives the header's structs (a small C program built here)
  and that the library reports (ss_struct_sizes);
* ss_fwd_check / ss_bwd_check (argument checks only, no device work) accept a
  valid argument block and reject each kind of bad one with a message;
* the Python boundary refuses CPU tensors (there is no CPU path) and fails
  loudly when the library is missing;
* nothing in the product package imports the oracle;
* the benchmark's byte model gives the figures its docstring states and it
  refuses more than one GPU.
"""
import ctypes
import json
import os
import re
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mamba_ss.h")


@pytest.fixture(scope="module")
def nat():
    from mamba_amd import _native
    if not os.path.exists(_native.LIB_PATH):
        from mamba_amd import build
        build.build()
    return _native


@pytest.fixture(scope="module")
def lib(nat):
    return nat.load()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(ss_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_exported_list(nat):
    assert header_functions() == sorted(nat.EXPORTED)


def test_library_exports_every_declared_function(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib._name], capture_output=True, text=True, check=True).stdout
    defined = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for name in header_functions():
        assert name in defined, f"{name} is declared in mamba_ss.h but not exported"
        assert getattr(lib, name) is not None


def test_version_and_constants(lib, nat):
    assert lib.ss_abi_version() == nat.ABI_VERSION == 16
    assert lib.ss_chunk_size() == 16
    assert lib.ss_max_dstate() == 256
    assert lib.ss_last_error() == b""


C_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "mamba_ss.h"
#define F(T, m) printf(#T " " #m " %zu\n", offsetof(T, m));
int main(void) {
    printf("sizeof ss_fwd_args %zu\nsizeof ss_bwd_args %zu\n", sizeof(ss_fwd_args), sizeof(ss_bwd_args));
    FIELDS
    return 0;
}
"""


def test_struct_layout_matches_c_compiler(nat, lib, tmp_path):
    structs = ((nat.FwdArgs, "ss_fwd_args"), (nat.BwdArgs, "ss_bwd_args"),
               (nat.Conv1dArgs, "ss_conv1d_args"), (nat.Conv1dBwdArgs, "ss_conv1d_bwd_args"),
               (nat.RmsNormArgs, "ss_rmsnorm_args"), (nat.RmsNormBwdArgs, "ss_rmsnorm_bwd_args"),
               (nat.StateUpdateArgs, "ss_state_update_args"), (nat.Conv1dUpdateArgs, "ss_conv1d_update_args"),
               (nat.DecodeLinearArgs, "ss_decode_linear_args"))
    fields = [f"F({name}, {n})" for T, name in structs for n, _ in T._fields_]
    fields += [f'printf("sizeof {name} %zu\\n", sizeof({name}));' for _, name in structs]
    src = tmp_path / "probe.c"
    src.write_text(C_PROBE.replace("FIELDS", "\n    ".join(fields)))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines()
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in lines}
    assert got[("sizeof", "ss_fwd_args")] == ctypes.sizeof(nat.FwdArgs)
    assert got[("sizeof", "ss_bwd_args")] == ctypes.sizeof(nat.BwdArgs)
    for T, name in structs:
        assert got[("sizeof", name)] == ctypes.sizeof(T), name
        for n, _ in T._fields_:
            assert got[(name, n)] == getattr(T, n).offset, f"{name}.{n}"
    fs, bs = ctypes.c_int64(), ctypes.c_int64()
    lib.ss_struct_sizes(ctypes.byref(fs), ctypes.byref(bs))
    assert (fs.value, bs.value) == (ctypes.sizeof(nat.FwdArgs), ctypes.sizeof(nat.BwdArgs))
    lib.ss_struct_sizes(None, None)   # either pointer may be NULL


# ------------------------------------------------------------ argument checks --
FAKE = 1 << 20   # a 16-byte aligned, never dereferenced address


def valid_fwd(nat, batch=2, dim=32, seqlen=100, dstate=16, itype=None, has_z=True):
    itype = nat.SS_F32 if itype is None else itype
    a = nat.FwdArgs()
    a.batch, a.dim, a.seqlen, a.dstate, a.n_groups = batch, dim, seqlen, dstate, 1
    a.itype, a.is_var_B, a.is_var_C = itype, 1, 1
    a.has_D, a.has_delta_bias, a.has_z, a.delta_softplus = 1, 1, int(has_z), 1
    a.n_chunks = (seqlen + 15) // 16
    for t in ("u", "delta", "z", "out", "y"):
        setattr(a, f"{t}_batch_stride", dim * seqlen)
        setattr(a, f"{t}_dim_stride", seqlen)
    a.A_dim_stride, a.A_dstate_stride = dstate, 1
    for t in ("B", "C"):
        setattr(a, f"{t}_batch_stride", dstate * seqlen)
        setattr(a, f"{t}_group_stride", dstate * seqlen)
        setattr(a, f"{t}_dstate_stride", seqlen)
    for i, p in enumerate(("u", "delta", "A", "B", "C", "D", "delta_bias", "z", "out", "x", "y")):
        setattr(a, p, FAKE + 4096 * i)
    return a


def valid_bwd(nat, **kw):
    b = nat.BwdArgs()
    b.f = valid_fwd(nat, **kw)
    dim, seqlen = b.f.dim, b.f.seqlen
    for t in ("dout", "du", "ddelta", "dz"):
        setattr(b, f"{t}_batch_stride", dim * seqlen)
        setattr(b, f"{t}_dim_stride", seqlen)
    for i, p in enumerate(("dout", "du", "ddelta", "dz", "dA", "dB", "dC", "dD", "ddelta_bias")):
        setattr(b, p, FAKE + 65536 + 4096 * i)
    return b


def fwd_rc(lib, a):
    return lib.ss_fwd_check(ctypes.byref(a)), lib.ss_last_error().decode()


def bwd_rc(lib, b):
    return lib.ss_bwd_check(ctypes.byref(b)), lib.ss_last_error().decode()


def test_valid_blocks_pass(nat, lib):
    for itype in (nat.SS_F32, nat.SS_BF16, nat.SS_F16):
        assert fwd_rc(lib, valid_fwd(nat, itype=itype))[0] == nat.SS_OK
        assert bwd_rc(lib, valid_bwd(nat, itype=itype))[0] == nat.SS_OK
    assert fwd_rc(lib, valid_fwd(nat, dstate=256))[0] == nat.SS_OK
    assert fwd_rc(lib, valid_fwd(nat, dstate=1))[0] == nat.SS_OK
    # checkpoint windows: 0 (the default span) up to 2^31 bytes
    for window in (1, 64 << 10, 1 << 31):
        a = valid_fwd(nat)
        a.x_window_bytes = window
        assert fwd_rc(lib, a)[0] == nat.SS_OK


def test_empty_problem_needs_no_pointers(nat, lib):
    for dims in ((0, 32, 100), (2, 0, 100), (2, 32, 0)):
        a = valid_fwd(nat, *dims)
        for p in ("u", "delta", "A", "B", "C", "x", "out"):
            setattr(a, p, None)
        assert fwd_rc(lib, a)[0] == nat.SS_OK


FWD_BREAKS = [
    ("negative size", lambda a: setattr(a, "seqlen", -1), "INVALID", "negative size"),
    ("dstate 0", lambda a: setattr(a, "dstate", 0), "UNSUPPORTED", "dstate"),
    ("dstate 257", lambda a: setattr(a, "dstate", 257), "UNSUPPORTED", "dstate"),
    ("unknown itype", lambda a: setattr(a, "itype", 7), "INVALID", "itype"),
    ("groups not dividing dim", lambda a: setattr(a, "n_groups", 3), "INVALID", "n_groups"),
    ("zero groups", lambda a: setattr(a, "n_groups", 0), "INVALID", "n_groups"),
    ("wrong n_chunks", lambda a: setattr(a, "n_chunks", 6), "INVALID", "n_chunks"),
    ("u NULL", lambda a: setattr(a, "u", None), "INVALID", "u is NULL"),
    ("last_state misaligned", lambda a: setattr(a, "last_state", FAKE + 2), "INVALID", "last_state is misaligned"),
    ("out NULL", lambda a: setattr(a, "out", None), "INVALID", "out is NULL"),
    ("D NULL with has_D", lambda a: setattr(a, "D", None), "INVALID", "D is NULL"),
    ("z NULL with has_z", lambda a: setattr(a, "z", None), "INVALID", "z is NULL"),
    ("misaligned delta", lambda a: setattr(a, "delta", FAKE + 2), "INVALID", "delta is misaligned"),
    ("misaligned A", lambda a: setattr(a, "A", FAKE + 1), "INVALID", "A is misaligned"),
    ("negative stride", lambda a: setattr(a, "B_dstate_stride", -1), "INVALID", "negative stride"),
    ("negative checkpoint window", lambda a: setattr(a, "x_window_bytes", -1), "INVALID", "x_window_bytes"),
    ("checkpoint window past 2^31", lambda a: setattr(a, "x_window_bytes", (1 << 31) + 1), "INVALID",
     "x_window_bytes"),
    ("huge grid", lambda a: (setattr(a, "batch", 1 << 40), setattr(a, "n_chunks", a.n_chunks)), "UNSUPPORTED",
     "too large"),
]


@pytest.mark.parametrize("case", [c[0] for c in FWD_BREAKS])
def test_fwd_check_rejects(nat, lib, case):
    _, brk, code, msg = next(c for c in FWD_BREAKS if c[0] == case)
    a = valid_fwd(nat)
    brk(a)
    rc, err = fwd_rc(lib, a)
    assert rc == getattr(nat, f"SS_ERR_{code}"), (rc, err)
    assert msg in err
    # the same block inside a backward call is rejected the same way (out is not needed there)
    if case != "out NULL":
        b = valid_bwd(nat)
        brk(b.f)
        assert bwd_rc(lib, b)[0] == getattr(nat, f"SS_ERR_{code}")


BWD_BREAKS = [
    ("x NULL", lambda b: setattr(b.f, "x", None), "x is NULL"),
    ("dout NULL", lambda b: setattr(b, "dout", None), "dout is NULL"),
    ("du NULL", lambda b: setattr(b, "du", None), "du is NULL"),
    ("dz NULL with has_z", lambda b: setattr(b, "dz", None), "dz is NULL"),
    ("dB NULL", lambda b: setattr(b, "dB", None), "dB is NULL"),
    ("dD NULL with has_D", lambda b: setattr(b, "dD", None), "dD is NULL"),
    ("saved y NULL with has_z", lambda b: setattr(b.f, "y", None), "y (saved pre-gate output) is NULL"),
    ("misaligned dA", lambda b: setattr(b, "dA", FAKE + 65536 + 2), "dA is misaligned"),
    ("negative dout stride", lambda b: setattr(b, "dout_dim_stride", -5), "negative stride"),
]


def test_forward_without_checkpoints_is_valid(nat, lib):
    # a forward that no backward follows passes no x (and no y); last_state is optional
    a = valid_fwd(nat)
    a.x, a.y = None, None
    assert lib.ss_fwd_check(ctypes.byref(a)) == nat.SS_OK, lib.ss_last_error()
    a.last_state = FAKE + 8 * 4096
    assert lib.ss_fwd_check(ctypes.byref(a)) == nat.SS_OK, lib.ss_last_error()


@pytest.mark.parametrize("case", [c[0] for c in BWD_BREAKS])
def test_bwd_check_rejects(nat, lib, case):
    _, brk, msg = next(c for c in BWD_BREAKS if c[0] == case)
    b = valid_bwd(nat)
    brk(b)
    rc, err = bwd_rc(lib, b)
    assert rc == nat.SS_ERR_INVALID and msg in err, (rc, err)


def test_optional_pointers_may_be_null_when_absent(nat, lib):
    b = valid_bwd(nat, has_z=False)
    b.f.has_D = b.f.has_delta_bias = 0
    b.f.D = b.f.delta_bias = b.f.z = b.f.y = None
    b.dz = b.dD = b.ddelta_bias = None
    assert bwd_rc(lib, b)[0] == nat.SS_OK
    a = valid_fwd(nat)
    a.y = None   # has_z without y: the forward then just does not save the pre-gate output
    assert fwd_rc(lib, a)[0] == nat.SS_OK


def test_null_argument_block(nat, lib):
    assert lib.ss_fwd_check(None) == nat.SS_ERR_INVALID
    assert lib.ss_bwd_check(None) == nat.SS_ERR_INVALID
    assert "null argument block" in lib.ss_last_error().decode()


def test_error_message_is_per_thread(nat, lib):
    import threading
    a = valid_fwd(nat)
    a.dstate = 0
    assert fwd_rc(lib, a)[0] != nat.SS_OK
    seen = {}

    def other():
        seen["msg"] = lib.ss_last_error().decode()
    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "dstate" in lib.ss_last_error().decode()


def test_check_status_maps_to_exceptions(nat, lib):
    a = valid_fwd(nat)
    a.itype = 9
    rc = lib.ss_fwd_check(ctypes.byref(a))
    with pytest.raises(ValueError, match="itype"):
        nat.check(rc, "ss_fwd")
    nat.check(nat.SS_OK, "ss_fwd")


# ------------------------------------------------------------------ host side --
def test_python_boundary_refuses_cpu_tensors():
    from mamba_amd import selective_scan as ss
    from mamba_amd.ops.selective_scan_interface import SelectiveScanFn, selective_scan_fn
    u = torch.randn(1, 4, 8)
    A = -torch.ones(4, 2)
    B = torch.randn(1, 1, 2, 8)
    with pytest.raises(ValueError, match="no CPU path"):
        ss.forward(u, u.clone(), A, B, B.clone(), None, None, True)
    with pytest.raises(ValueError, match="no CPU path"):
        selective_scan_fn(u, u.clone(), A, B, B.clone())
    with pytest.raises(ValueError, match="no CPU path"):
        SelectiveScanFn.apply(u, u.clone(), A, B, B.clone(), None)


def test_missing_library_fails_loudly(monkeypatch):
    from mamba_amd import _native
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", os.path.join(ROOT, "no_such_dir", "libmamba_ss.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _native.load()


def test_product_package_does_not_import_the_oracle():
    pkg = os.path.join(ROOT, "mamba_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.M), f
                assert "ss_oracle" not in text and "selective_scan_ref" not in text.replace(
                    "reference's pure-PyTorch selective_scan_ref", ""), f


def test_bench_byte_model():
    sys.path.insert(0, ROOT)
    import bench
    fwd, bwd = bench.algorithmic_bytes(8, 1536, 16, 2048, 4)
    assert (fwd, bwd) == (404_860_928, 709_058_560)
    assert sum(bench.algorithmic_bytes(4, 5120, 16, 8192, 2)) == 3_700_482_048


def test_bench_inputs_and_provenance(tmp_path, monkeypatch):
    """The bench draws its own inputs (its GPU leg imports nothing from
    oracle/), with the oracle's distributions and draw order; a stored
    traffic figure is reported only for the kernel sources it was taken with."""
    sys.path.insert(0, ROOT)
    import bench
    import torch
    from oracle.selective_scan_ref import make_inputs
    got = bench.synthetic_inputs(2, 32, 16, 64, seed=7, dtype=torch.bfloat16)
    want = make_inputs(2, 32, 16, 64, seed=7, dtype=torch.bfloat16)
    for k in ("u", "delta", "z", "B", "C", "dout", "delta_bias", "A", "D"):
        assert torch.equal(got[k], want[k]), k
    # the scan leg of main() and the helpers it calls do not name the oracle
    import inspect
    src = inspect.getsource(bench.main)
    assert "import" not in src.split("cpu_baseline(")[0] or "oracle" not in "".join(
        l for l in src.split("cpu_baseline(")[0].splitlines() if "import" in l)
    rec = {"sources_sha256": bench.kernel_sources_digest(), "k": 123}
    (tmp_path / "profiles").mkdir()
    (tmp_path / "profiles" / "traffic_w.json").write_text(json.dumps(rec))
    (tmp_path / "mamba_amd").symlink_to(os.path.join(ROOT, "mamba_amd"))
    monkeypatch.setattr(bench, "_HERE", str(tmp_path))
    assert bench.stored_traffic("w", "k")[0] == 123
    rec["sources_sha256"] = "0" * 64
    (tmp_path / "profiles" / "traffic_w.json").write_text(json.dumps(rec))
    val, why = bench.stored_traffic("w", "k")
    assert val is None and "stale" in why
    assert bench.cpu_threads() >= 1 and bench.cpu_model()


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_kernel_name_query(nat, lib):
    def fname(a):
        r = lib.ss_fwd_kernel_name(ctypes.byref(a))
        return None if r is None else r.decode()

    def bname(b):
        r = lib.ss_bwd_kernel_name(ctypes.byref(b))
        return None if r is None else r.decode()
    # dstate 16, variable B / C, 16-channel groups: cooperative fast paths, at
    # any seqlen (a ragged one ends in a partial tile of identity steps)
    assert fname(valid_fwd(nat, seqlen=128)) == "ss_fwd_fast"
    assert bname(valid_bwd(nat, seqlen=128)) == "ss_bwd_fast"
    assert fname(valid_fwd(nat, seqlen=100)) == "ss_fwd_fast"
    assert fname(valid_fwd(nat, seqlen=7)) == "ss_fwd_fast"
    assert bname(valid_bwd(nat, seqlen=100)) == "ss_bwd_fast"
    assert bname(valid_bwd(nat, seqlen=1)) == "ss_bwd_fast"
    # dstate 16 S (32, 64, ..., 256): the fast kernels once per 16-state slice
    # (with the workspace ss_*_workspace_bytes asks for); other dstates, or
    # constant B / C, take the general kernels
    for n in (32, 48, 64, 256):
        assert fname(valid_fwd(nat, seqlen=128, dstate=n)) == "ss_fwd_fast"
        assert bname(valid_bwd(nat, seqlen=128, dstate=n)) == "ss_bwd_fast"
    for n in (8, 24, 200):
        assert fname(valid_fwd(nat, seqlen=128, dstate=n)) == "ss_fwd_kernel"
        assert bname(valid_bwd(nat, seqlen=128, dstate=n)) == "ss_bwd_kernel"
    a = valid_fwd(nat, seqlen=128, dstate=32)
    a.is_var_B = 0
    a.B_batch_stride, a.B_group_stride, a.B_dstate_stride = 0, 32, 1
    assert fname(a) == "ss_fwd_kernel"
    # dstate 16 with B and C, or one of them, constant ((dim, dstate) fp32):
    # the fast kernels
    def const_bc(x, both=True):
        x.is_var_B = 0
        x.B_batch_stride, x.B_group_stride, x.B_dstate_stride = 0, 16, 1
        if both:
            x.is_var_C = 0
            x.C_batch_stride, x.C_group_stride, x.C_dstate_stride = 0, 16, 1
        return x
    assert fname(const_bc(valid_fwd(nat, seqlen=100))) == "ss_fwd_fast"
    assert fname(const_bc(valid_fwd(nat, seqlen=100), both=False)) == "ss_fwd_fast"
    b = valid_bwd(nat, seqlen=100)
    const_bc(b.f)
    assert bname(b) == "ss_bwd_fast"
    b = valid_bwd(nat, seqlen=100)
    const_bc(b.f, both=False)
    assert bname(b) == "ss_bwd_fast"
    # no work, and invalid arguments
    assert fname(valid_fwd(nat, batch=0)) == ""
    bad = valid_fwd(nat)
    bad.dstate = 0
    assert fname(bad) is None and "dstate" in lib.ss_last_error().decode()


def test_workspace_query(nat, lib):
    # 2 channel blocks per group: one slice, no workspace
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(valid_bwd(nat, seqlen=128))) == 0
    # at most 96 channel blocks per slice: 1536 channels in one group (96
    # blocks) accumulate directly; 3072 (192 blocks) use 2 slices of dB and dC
    # (batch * dstate * seqlen floats each)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(valid_bwd(nat, batch=2, dim=1536, seqlen=128))) == 0
    b = valid_bwd(nat, batch=2, dim=3072, seqlen=128)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 2 * 2 * (2 * 16 * 128) * 4
    # dstate 32: two passes of the fast kernel, each with the one padded dB / dC
    # slice of a ragged seqlen (2 x (2 x 16 x 128) floats), then the two fp32
    # accumulators of the sums over states (2 x batch x dim x seqlen floats)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(valid_bwd(nat, dim=1536, seqlen=100, dstate=32))) == (
        2 * (2 * 16 * 128) * 4 + 2 * 2 * 1536 * 100 * 4)
    # the forward's accumulator is one such array
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(valid_fwd(nat, dim=1536, seqlen=100, dstate=32))) == (
        2 * 1536 * 100 * 4)
    # the general kernel (dstate 24) uses none; invalid arguments give -1
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(valid_bwd(nat, dim=1536, seqlen=100, dstate=24))) == 0
    bad = valid_bwd(nat)
    bad.dout = None
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(bad)) == -1
    assert "dout is NULL" in lib.ss_last_error().decode()
    # 5120 channels: 320 blocks, 4 slices; 26112 channels: 1632 blocks, capped at 16 slices
    b = valid_bwd(nat, batch=1, dim=5120, seqlen=64)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 2 * 4 * (16 * 64) * 4
    b = valid_bwd(nat, batch=1, dim=26112, seqlen=64)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 2 * 16 * (16 * 64) * 4
    # one long sequence: no dB / dC slices (96 blocks), 8 sequence segments (-> 768 workgroups)
    b = valid_bwd(nat, batch=1, dim=1536, seqlen=32768)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 1 * 8 * 1536 * 17 * 4
    # 3072 channels: 2 slices, then 4 segments (192 blocks -> 768 workgroups)
    b = valid_bwd(nat, batch=1, dim=3072, seqlen=32768)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 2 * 2 * (16 * 32768) * 4 + 1 * 4 * 3072 * 17 * 4
    # a seqlen that is not a multiple of 32: one slice whose rows are padded
    # to a multiple of 32 steps (1001 -> 1024, 2064 -> 2080), even with few
    # channel blocks (768 workgroups: no sequence segments)
    b = valid_bwd(nat, batch=8, dim=1536, seqlen=1001)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 2 * 1 * (8 * 16 * 1024) * 4
    b = valid_bwd(nat, batch=8, dim=1536, seqlen=2064)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 2 * 1 * (8 * 16 * 2080) * 4
    # ... and with several slices (2 for 192 channel blocks)
    b = valid_bwd(nat, batch=4, dim=3072, seqlen=2064)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == 2 * 2 * (4 * 16 * 2080) * 4


# --------------------------------------------------------------------- RMSNorm --
def valid_norm(nat, rows=4, dim=768, dtype=None):
    a = nat.RmsNormArgs()
    a.rows, a.dim = rows, dim
    a.dtype = nat.SS_BF16 if dtype is None else dtype
    a.w_dtype, a.eps = a.dtype, 1e-6
    a.x_row_stride = a.residual_row_stride = a.out_row_stride = a.residual_out_row_stride = dim
    a.x, a.residual, a.weight, a.out, a.residual_out, a.rstd = (FAKE + 65536 * i for i in range(6))
    return a


def valid_norm_bwd(nat, rows=4, dim=768, dtype=None):
    g = nat.RmsNormBwdArgs()
    g.rows, g.dim = rows, dim
    g.dtype = nat.SS_BF16 if dtype is None else dtype
    g.w_dtype = g.dtype
    g.s_row_stride = g.dout_row_stride = g.dresidual_out_row_stride = g.dx_row_stride = dim
    g.s, g.weight, g.rstd, g.dout, g.dresidual_out, g.dx, g.dweight, g.workspace = (
        FAKE + 65536 * i for i in range(8))
    g.workspace_bytes = 1 << 30
    return g


@pytest.mark.parametrize("case", ["neg_rows", "dtype", "w_dtype", "null_x", "null_weight", "misaligned_out",
                                  "neg_stride", "neg_eps"])
def test_rmsnorm_fwd_rejects(nat, lib, case):
    a = valid_norm(nat)
    if case == "neg_rows":
        a.rows = -1
    elif case == "dtype":
        a.dtype = 7
    elif case == "w_dtype":
        a.w_dtype = nat.SS_F16              # neither the row dtype (bf16) nor fp32
    elif case == "null_x":
        a.x = None
    elif case == "null_weight":
        a.weight = None
    elif case == "misaligned_out":
        a.out = FAKE + 1
    elif case == "neg_stride":
        a.residual_row_stride = -768
    elif case == "neg_eps":
        a.eps = -1.0
    rc = lib.ss_rmsnorm_fwd(ctypes.byref(a), None)
    assert rc in (nat.SS_ERR_INVALID, nat.SS_ERR_UNSUPPORTED)
    assert lib.ss_last_error().decode()


def test_rmsnorm_empty_and_bwd_rejects(nat, lib):
    # no rows or no columns: nothing to launch
    assert lib.ss_rmsnorm_fwd(ctypes.byref(valid_norm(nat, rows=0)), None) == nat.SS_OK
    assert lib.ss_rmsnorm_fwd(ctypes.byref(valid_norm(nat, dim=0)), None) == nat.SS_OK
    assert lib.ss_rmsnorm_bwd(ctypes.byref(valid_norm_bwd(nat, dim=0)), None) == nat.SS_OK
    g = valid_norm_bwd(nat)
    g.workspace = None
    assert lib.ss_rmsnorm_bwd(ctypes.byref(g), None) == nat.SS_ERR_INVALID
    assert "workspace" in lib.ss_last_error().decode()
    g = valid_norm_bwd(nat)
    g.workspace_bytes = 16
    assert lib.ss_rmsnorm_bwd(ctypes.byref(g), None) == nat.SS_ERR_INVALID
    g = valid_norm_bwd(nat, dim=20000)
    assert lib.ss_rmsnorm_bwd(ctypes.byref(g), None) == nat.SS_ERR_UNSUPPORTED
    g = valid_norm_bwd(nat)
    g.rstd = None
    assert lib.ss_rmsnorm_bwd(ctypes.byref(g), None) == nat.SS_ERR_INVALID
    g = valid_norm_bwd(nat)
    g.dweight = None
    assert lib.ss_rmsnorm_bwd(ctypes.byref(g), None) == nat.SS_ERR_INVALID


def valid_conv_bwd(nat, batch=2, dim=64, seqlen=5000):
    g = nat.Conv1dBwdArgs()
    g.f.batch, g.f.dim, g.f.seqlen, g.f.width = batch, dim, seqlen, 4
    g.f.itype, g.f.has_bias, g.f.silu = nat.SS_BF16, 1, 1
    g.f.x_batch_stride, g.f.x_dim_stride = dim * seqlen, seqlen
    g.f.out_batch_stride, g.f.out_dim_stride = dim * seqlen, seqlen
    g.f.w_dim_stride, g.f.w_width_stride = 4, 1
    g.f.x, g.f.weight, g.f.bias, g.f.out = (FAKE + 65536 * i for i in range(4))
    g.dout_batch_stride, g.dout_dim_stride = dim * seqlen, seqlen
    g.dx_batch_stride, g.dx_dim_stride = dim * seqlen, seqlen
    g.dout, g.dx, g.dweight, g.dbias = (FAKE + 65536 * (4 + i) for i in range(4))
    return g


def test_conv1d_bwd_workspace_query_and_rejects(nat, lib):
    # 5 fp32 partials (4 right-aligned taps + bias) per (batch row, channel,
    # sequence tile of 1024 steps: the fewest steps a workgroup takes)
    assert lib.ss_conv1d_bwd_workspace_bytes(ctypes.byref(valid_conv_bwd(nat))) == 2 * 64 * 5 * 5 * 4
    assert lib.ss_conv1d_bwd_workspace_bytes(ctypes.byref(valid_conv_bwd(nat, seqlen=1024))) == 2 * 64 * 5 * 4
    assert lib.ss_conv1d_bwd_workspace_bytes(ctypes.byref(valid_conv_bwd(nat, seqlen=0))) == 0
    assert lib.ss_conv1d_bwd_workspace_bytes(ctypes.byref(valid_conv_bwd(nat, batch=-1))) == -1
    g = valid_conv_bwd(nat)
    g.workspace, g.workspace_bytes = FAKE + 2, 1 << 20
    assert lib.ss_conv1d_bwd(ctypes.byref(g), None) == nat.SS_ERR_INVALID
    assert "misaligned" in lib.ss_last_error().decode()
    g = valid_conv_bwd(nat)
    g.workspace, g.workspace_bytes = FAKE, 2 * 64 * 5 * 5 * 4 - 4
    assert lib.ss_conv1d_bwd(ctypes.byref(g), None) == nat.SS_ERR_INVALID
    assert "workspace_bytes" in lib.ss_last_error().decode()


def test_rmsnorm_workspace_query(lib):
    # one fp32 row of dim column sums per backward workgroup (8 rows each, at most 512 workgroups)
    assert lib.ss_rmsnorm_bwd_workspace_bytes(32768, 768) == 512 * 768 * 4
    assert lib.ss_rmsnorm_bwd_workspace_bytes(20, 768) == 3 * 768 * 4
    assert lib.ss_rmsnorm_bwd_workspace_bytes(0, 768) == 0
    assert lib.ss_rmsnorm_bwd_workspace_bytes(-1, 768) == -1


def test_decode_linear_workspace_query(nat, lib):
    # K is split over workgroups only for shapes with fewer than 64 16 x 16
    # output tiles, into at most 4 slices of at least 2 K units (32 elements,
    # or 16 when k_in is not a multiple of 32); the workspace is a fixed 256
    # bytes of tile counters (one per tile of the largest split shape, so every
    # shape finds its counters at zero) plus one fp32 16 x 16 partial tile per
    # (tile, slice)
    def q(batch, n_out, k_in):
        a = nat.DecodeLinearArgs()
        a.batch, a.n_out, a.k_in = batch, n_out, k_in
        return lib.ss_decode_linear_workspace_bytes(ctypes.byref(a))
    assert q(16, 80, 1536) == 256 + 5 * 4 * 1024             # x-projection: 5 tiles, 4 slices of 384
    assert q(16, 768, 1536) == 256 + 48 * 4 * 1024           # output projection: 48 tiles
    assert q(16, 37, 80) == 256 + 3 * 2 * 1024               # 3 tiles, 5 units of 16: slices of 3 and 2
    assert q(16, 16, 128) == 256 + 1 * 2 * 1024              # 1 tile, 4 units: 2 slices
    assert q(33, 64, 256) == 256 + 12 * 4 * 1024             # 3 batch tiles x 4: 4 slices of 64
    assert q(16, 1008, 768) == 256 + 63 * 4 * 1024           # 63 tiles: the largest split shape
    assert q(16, 37, 48) == 0                                # 3 units: too few to split
    assert q(16, 1024, 768) == 0                             # 64 tiles: no split
    assert q(16, 3072, 768) == 0                             # input projection: 192 tiles
    assert q(16, 50280, 768) == 0
    assert q(0, 768, 1536) == 0
    assert q(16, 768, 24) == -1 and b"16" in lib.ss_last_error()
    for batch, n_out, k_in in [(16, 80, 1536), (1, 1, 1 << 20), (16, 1008, 1 << 20), (64, 240, 2048)]:
        assert q(batch, n_out, k_in) <= 1 << 20                # the Python layer's per-stream workspace


def valid_linear(nat, batch=16, n_out=3072, k_in=768):
    a = nat.DecodeLinearArgs()
    a.batch, a.n_out, a.k_in = batch, n_out, k_in
    a.dtype = a.bias_dtype = nat.SS_BF16
    a.x_row_stride, a.w_row_stride, a.y_row_stride = k_in, k_in, n_out
    a.x, a.weight, a.y = FAKE, FAKE + (1 << 24), FAKE + (1 << 25)
    return a


@pytest.mark.parametrize("case", ["conv_itype", "conv_batch", "conv_dim", "conv_width", "conv_null_state",
                                  "norm_rows", "norm_dim", "norm_k_in", "norm_dtype", "norm_w_dtype",
                                  "norm_misaligned", "norm_stride", "norm_neg_eps", "norm_inplace_residual",
                                  "norm_residual_out_over_x", "norm_y_over_residual", "y_over_x", "ws_misaligned",
                                  "ws_neg", "k_in", "null_y"])
def test_decode_linear_rejects(nat, lib, case):
    # every check runs before any device work, so these calls need no GPU
    a = valid_linear(nat)
    c = nat.Conv1dUpdateArgs()
    c.batch, c.dim, c.width, c.itype, c.has_bias, c.silu = 16, 1536, 4, nat.SS_BF16, 1, 1
    c.state_batch_stride, c.state_dim_stride, c.state_width_stride = 1536 * 4, 4, 1
    c.w_dim_stride, c.w_width_stride = 4, 1
    c.conv_state, c.weight, c.bias = FAKE + (1 << 26), FAKE + (1 << 27), FAKE + (1 << 28)
    n = valid_norm(nat, rows=16, dim=768)
    if case.startswith("conv"):
        a.conv = ctypes.pointer(c)
        if case == "conv_itype":
            c.itype = nat.SS_F16
        elif case == "conv_batch":
            c.batch = 15
        elif case == "conv_dim":
            c.dim = 3073
        elif case == "conv_width":
            c.width = 5
        elif case == "conv_null_state":
            c.conv_state = None
    elif case.startswith("norm"):
        a.norm = ctypes.pointer(n)
        if case == "norm_rows":
            n.rows = 8
        elif case == "norm_dim":
            n.dim = 512
        elif case == "norm_k_in":
            a.k_in = n.dim = 1536
            a.x_row_stride = a.w_row_stride = 1536
        elif case == "norm_dtype":
            n.dtype = nat.SS_F16
        elif case == "norm_w_dtype":
            n.w_dtype = nat.SS_F16
        elif case == "norm_misaligned":
            n.residual = FAKE + 8
        elif case == "norm_stride":
            n.x_row_stride = 772                       # rows not 16-byte aligned
        elif case == "norm_neg_eps":
            n.eps = -1.0
        elif case == "norm_inplace_residual":
            n.residual_out = n.residual                # the residual stream updated in place
        elif case == "norm_residual_out_over_x":
            n.residual_out = n.x + 16 * 768 * 2 - 16   # the last 16 bytes of x
        elif case == "norm_y_over_residual":
            a.y = n.residual + 4096
    elif case == "ws_misaligned":
        a.workspace, a.workspace_bytes = FAKE + 4, 1 << 20
    elif case == "ws_neg":
        a.workspace, a.workspace_bytes = FAKE, -1
    elif case == "k_in":
        a.k_in = 24
    elif case == "null_y":
        a.y = None
    elif case == "y_over_x":
        a.y = a.x + 768 * 2 * 15                       # y's first row is x's last
    rc = lib.ss_decode_linear(ctypes.byref(a), None)
    assert rc in (nat.SS_ERR_INVALID, nat.SS_ERR_UNSUPPORTED), case
    err = lib.ss_last_error().decode()
    assert err
    if "over" in case or "inplace" in case:
        assert rc == nat.SS_ERR_INVALID and "overlaps" in err, (case, err)


def test_rmsnorm_python_boundary_refuses_cpu_tensors():
    from mamba_amd.ops.rms_norm import rms_norm_fn
    with pytest.raises(ValueError, match="no CPU path"):
        rms_norm_fn(torch.randn(2, 8), torch.zeros(8))


def test_forward_workspace_query(nat, lib):
    # sequence segments only when batch x (dim / 16) is below 768 workgroups, the
    # fast path applies and segments keep at least 4 x 64 steps
    a = valid_fwd(nat, batch=1, dim=1536, seqlen=32768)
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == 1 * 8 * 1536 * 17 * 4      # 96 blocks -> 8 segments
    a = valid_fwd(nat, batch=8, dim=1536, seqlen=2048)
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == 0                           # 768 blocks already
    a = valid_fwd(nat, batch=1, dim=64, seqlen=4096)
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == 1 * 16 * 64 * 17 * 4       # 4 blocks: 64 / 16 = 4 sc each
    a = valid_fwd(nat, batch=1, dim=64, seqlen=100)
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == 0                           # too short to split
    # segment counts need not divide the super-chunk count (469 here)
    a = valid_fwd(nat, batch=1, dim=1536, seqlen=30000)
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == 1 * 8 * 1536 * 17 * 4
    a = valid_fwd(nat, batch=1, dim=64, seqlen=30000)
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == 1 * 64 * 64 * 17 * 4
    # seqlen x dim above 2^30 stays on the fast path (65 blocks -> 16 segments)
    a = valid_fwd(nat, batch=1, dim=1040, seqlen=(1 << 20) + 37)
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == 1 * 16 * 1040 * 17 * 4
    a.u = None
    assert lib.ss_fwd_workspace_bytes(ctypes.byref(a)) == -1


def test_noalloc_entry_checks_before_device_work(nat, lib):
    """ss_bwd_noalloc: the scratch limit of the header is the binding's; bad
    arguments and arguments needing more scratch than the fixed buffer are
    rejected before any device work (no GPU is touched here)."""
    text = open(HEADER).read()
    m = re.search(r"#define\s+SS_NOALLOC_SCRATCH_BYTES\s+\((\d+)ll\s*<<\s*(\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == nat.NOALLOC_SCRATCH_BYTES
    bad = valid_bwd(nat)
    bad.dout = None
    assert lib.ss_bwd_noalloc(ctypes.byref(bad), None) == nat.SS_ERR_INVALID
    assert "dout is NULL" in lib.ss_last_error().decode()
    # 1632 channel blocks in one group: 16 dB / dC slices of 16 x 32768 floats
    # each, 64 MiB, twice the fixed buffer
    big = valid_bwd(nat, batch=1, dim=26112, seqlen=32768)
    need = lib.ss_bwd_workspace_bytes(ctypes.byref(big))
    assert need == 2 * 16 * (16 * 32768) * 4 > nat.NOALLOC_SCRATCH_BYTES
    assert lib.ss_bwd_noalloc(ctypes.byref(big), None) == nat.SS_ERR_UNSUPPORTED
    msg = lib.ss_last_error().decode()
    assert str(need) in msg and str(nat.NOALLOC_SCRATCH_BYTES) in msg


def test_deterministic_workspace_query(nat, lib):
    """Deterministic sums: one dB / dC slice per 16-channel block of a group
    plus the dA / dD / ddelta_bias partials of every (batch row, segment);
    shapes the fast kernels do not take are refused before any device work."""
    b = valid_bwd(nat, batch=2, dim=256, seqlen=512)
    b.deterministic = 1
    # (32 workgroups: 2 sequence segments, whose carries sit between the two)
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == (2 * 16 * (2 * 16 * 512) * 4 + 2 * 2 * 256 * 17 * 4
                                                          + 2 * 2 * 256 * 18 * 4)
    # one long sequence: 8 segments, their carries, then 8 rows of partials
    b = valid_bwd(nat, batch=1, dim=1536, seqlen=32768)
    b.deterministic = 1
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == (2 * 96 * (16 * 32768) * 4 + 1 * 8 * 1536 * 17 * 4
                                                          + 1 * 8 * 1536 * 18 * 4)
    # dstate 32: two passes of the fast kernel, one per 16-state slice; what
    # one pass needs (2 dB / dC slices of 16 rows padded to 128 floats, one
    # row of partials) then the two accumulators (batch x dim x seqlen fp32)
    b = valid_bwd(nat, batch=1, dim=32, seqlen=100, dstate=32)
    b.deterministic = 1
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == (2 * 2 * (16 * 128) * 4 + 1 * 32 * 18 * 4
                                                          + 2 * 32 * 100 * 4)
    b = valid_bwd(nat, batch=1, dim=32, seqlen=100, dstate=24)     # dstate 24: the general kernel
    b.deterministic = 1
    assert lib.ss_bwd_workspace_bytes(ctypes.byref(b)) == -1
    assert "deterministic" in lib.ss_last_error().decode()
    assert lib.ss_bwd_noalloc(ctypes.byref(b), None) == nat.SS_ERR_UNSUPPORTED


def test_deterministic_setting_without_workspace(nat, lib):
    """torch.use_deterministic_algorithms with a call that passes no
    workspace: raises as torch's own ops do, or under warn_only warns and
    runs with atomic sums; an explicit flag is passed through untouched (the
    library refuses it), and a call with a workspace keeps the fixed order."""
    import warnings

    import torch
    from mamba_amd import selective_scan as ss
    was, was_warn = torch.are_deterministic_algorithms_enabled(), torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        b = valid_bwd(nat)
        with pytest.raises(RuntimeError, match="need a workspace"):
            ss._set_deterministic(lib, b, None, None)
        b = valid_bwd(nat)
        ss._set_deterministic(lib, b, None, "auto")
        assert b.deterministic == 1
        torch.use_deterministic_algorithms(True, warn_only=True)
        b = valid_bwd(nat)
        with warnings.catch_warnings(record=True) as w:
            warnings.simplefilter("always")
            ss._set_deterministic(lib, b, None, None)
        assert b.deterministic == 0 and any("need a workspace" in str(x.message) for x in w)
        b = valid_bwd(nat)
        ss._set_deterministic(lib, b, True, None)
        assert b.deterministic == 1
    finally:
        torch.use_deterministic_algorithms(was, warn_only=was_warn)
