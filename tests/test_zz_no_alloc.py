"""GPU test of ss_bwd_noalloc, the backward entry point that allocates
nothing: its scratch (dB / dC slices, sequence-segment carries) lives in a
fixed device buffer inside the library instead of a caller workspace.

Two calls in a row through the C ABI, the second on a smaller problem (so
it runs on what the first left in the buffer), each against ss_bwd with a
workspace from torch on the same inputs.  du, ddelta and dz come from the
same kernels in the same order and must match bit for bit; dA, dB, dC, dD
and ddelta_bias are fp32 atomic sums whose order varies between launches,
so they are compared to 1e-5 relative (well inside the fp32 bar of 1e-3).
With deterministic sums on dstate 32 (two passes of the fast kernel, one
per 16-state slice, whose accumulators also sit in the buffer) every
output matches bit for bit, again on two calls, the second smaller.  A
dstate-32 call whose state-slice passes need more than the buffer runs on
the general kernel, as ss_bwd without a workspace; it is held to the
workspace backward at the fp32 bar (1e-3: other kernels, other orders).
"""
import ctypes
import sys

import pytest
import torch

from mamba_amd import _native as nat
from mamba_amd import selective_scan as ss
from oracle.selective_scan_ref import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _grads(x, dev):
    u, dl, A, B, C, D, z, bias = (x[k] for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"))
    g = {"du": torch.empty_like(u), "ddelta": torch.empty_like(dl), "dz": torch.empty_like(z)}
    for k, ref in (("dA", A), ("dB", B), ("dC", C), ("dD", D), ("ddelta_bias", bias)):
        g[k] = torch.full(ref.shape, float("nan"), dtype=torch.float32, device=dev)   # zero_grads ignores these
    return g


def _run(x, g, entry, det=0):
    """One backward through the C ABI: entry 'ss_bwd' (torch workspace) or 'ss_bwd_noalloc'."""
    u, dl, A, B, C, D, z, bias = (x[k] for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias"))
    lib = nat.load()
    b = ss._bwd_into_args(u, dl, A, B, C, D, bias, x["dout"], x["xck"], True, g["du"], g["ddelta"],
                          g["dA"], g["dB"], g["dC"], g["dD"], g["ddelta_bias"], z, x["y"], g["dz"])
    b.zero_grads = 1
    b.deterministic = det
    need = lib.ss_bwd_workspace_bytes(ctypes.byref(b))
    assert need > 0, "the case must use scratch"
    ws = None
    if entry == "ss_bwd":
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        b.workspace, b.workspace_bytes = ctypes.c_void_p(ws.data_ptr()), need
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    rc = getattr(lib, entry)(ctypes.byref(b), stream)
    nat.check(rc, entry)
    torch.cuda.synchronize()
    return need


def _case(batch, dim, seqlen, seed, N=16):
    x = make_inputs(batch, dim, N, seqlen, seed=seed, dtype=torch.float32)
    x = {k: (v.to(DEV) if v is not None else None) for k, v in x.items()}
    out = torch.empty_like(x["delta"])
    x["xck"] = torch.empty((batch, ss.n_chunks(seqlen), dim, N), dtype=torch.float32, device=DEV)
    x["y"] = torch.empty_like(out)
    ss.forward_into(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["delta_bias"], True, out, x["xck"],
                    z=x["z"], y=x["y"])
    return x


# (batch, dim, seqlen): the first uses 2 dB / dC slices and 4 sequence
# segments, the second (smaller) 2 slices and 8 segments
CASES = [(1, 3072, 4096, 2101), (1, 1600, 2048, 2102)]


def test_noalloc_backward_matches_workspace_backward_twice():
    for batch, dim, seqlen, seed in CASES:
        print(f"\n[no_alloc] batch {batch} dim {dim} seqlen {seqlen}", flush=True)
        sys.stdout.flush()
        x = _case(batch, dim, seqlen, seed)
        want = _grads(x, DEV)
        need = _run(x, want, "ss_bwd")
        got = _grads(x, DEV)
        assert _run(x, got, "ss_bwd_noalloc") == need <= nat.NOALLOC_SCRATCH_BYTES
        for k in ("du", "ddelta", "dz"):
            assert torch.equal(got[k], want[k]), k
        for k in ("dA", "dB", "dC", "dD", "ddelta_bias"):
            w = want[k]
            assert_close(got[k], w, 1e-5, 1e-5 * float(w.abs().max()), k)


# (batch, dim, seqlen, dstate): deterministic sums over state slices, the
# second call smaller (ragged seqlen)
DET_CASES = [(2, 256, 1000, 32, 2103), (1, 64, 777, 32, 2104)]


def test_noalloc_deterministic_state_slices_twice():
    for batch, dim, seqlen, N, seed in DET_CASES:
        print(f"\n[no_alloc] deterministic batch {batch} dim {dim} seqlen {seqlen} dstate {N}", flush=True)
        sys.stdout.flush()
        x = _case(batch, dim, seqlen, seed, N=N)
        want = _grads(x, DEV)
        need = _run(x, want, "ss_bwd", det=1)
        got = _grads(x, DEV)
        assert _run(x, got, "ss_bwd_noalloc", det=1) == need <= nat.NOALLOC_SCRATCH_BYTES
        for k in want:
            assert torch.equal(got[k], want[k]), k


def test_noalloc_state_slices_too_large_run_on_the_general_kernel():
    batch, dim, seqlen, N = 2, 1040, 2048, 32
    print(f"\n[no_alloc] general kernel fallback batch {batch} dim {dim} seqlen {seqlen} dstate {N}", flush=True)
    sys.stdout.flush()
    x = _case(batch, dim, seqlen, 2105, N=N)
    want = _grads(x, DEV)
    need = _run(x, want, "ss_bwd")
    assert need > nat.NOALLOC_SCRATCH_BYTES            # the slice passes' accumulators alone pass 32 MiB
    got = _grads(x, DEV)
    _run(x, got, "ss_bwd_noalloc")
    for k in want:
        w = want[k]
        assert_close(got[k], w, 1e-3, 1e-3 * float(w.abs().max()), k)
