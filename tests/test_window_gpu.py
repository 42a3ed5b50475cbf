"""Checkpoint windows of the fast scans.

The fast kernels address the checkpoints x of a batch row through a buffer
resource based at a window of chunks, rebased when a chunk leaves the
window.  At the default span (2^31 bytes) that happens only for rows with
more than 2^31 bytes of checkpoints (seqlen x dim from 2^25), so here the
span is set small through ``ss_fwd_args.x_window_bytes`` and the results
must be the same bits as with the default span: forward out, y, x and
last_state, and (deterministic sums) every gradient.  Cases: ragged
seqlens, so the tail super-chunk / chunk falls in a window of its own;
spans of 64 KiB (several chunks per window) and of 1 byte (a new window
for every super-chunk / chunk); serial and sequence-segmented scans.
"""
import ctypes
import sys

import pytest
import torch

from mamba_amd import _native as nat
from mamba_amd import selective_scan as ss
from oracle.selective_scan_ref import make_inputs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

CASES = [
    # batch, dim, seqlen, dtype, forward / backward workspace (segments)
    (2, 48, 1037, torch.float32, False),
    (1, 32, 3001, torch.bfloat16, True),
    (3, 16, 2048, torch.float16, False),
]


def run(x, dtype, window, seg):
    lib = nat.load()
    t = {k: (v.to(dtype) if k in ("u", "delta", "z", "B", "C", "dout") else v).to(DEV) for k, v in x.items()}
    batch, dim, L = t["u"].shape
    N = t["A"].shape[1]
    out, y = torch.empty_like(t["u"]), torch.empty_like(t["u"])
    xck = torch.full((batch, ss.n_chunks(L), dim, N), float("nan"), device=DEV)
    last = torch.empty((batch, dim, N), device=DEV)
    a = ss._fwd_into_args(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True,
                          out, xck, t["z"], y, last)
    a.x_window_bytes = window
    ws_f = ss._attach_fwd_workspace(lib, a, "auto" if seg else None, DEV)
    nat.check(lib.ss_fwd(ctypes.byref(a), ss._stream(DEV)), "ss_fwd")
    du, dd, dz = torch.empty_like(out), torch.empty_like(out), torch.empty_like(out)
    dA = torch.empty(t["A"].shape, device=DEV)
    dB = torch.empty(t["B"].shape, device=DEV)
    dC = torch.empty(t["C"].shape, device=DEV)
    dD, db = torch.empty(dim, device=DEV), torch.empty(dim, device=DEV)
    b = ss._bwd_into_args(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck,
                          True, du, dd, dA, dB, dC, dD, db, t["z"], y, dz)
    b.f.x_window_bytes = window
    b.deterministic = 1
    b.zero_grads = 1
    n = lib.ss_bwd_workspace_bytes(ctypes.byref(b))
    assert n > 0
    ws_b = torch.empty(n, dtype=torch.uint8, device=DEV)
    b.workspace, b.workspace_bytes = ctypes.c_void_p(ws_b.data_ptr()), n
    nat.check(lib.ss_bwd(ctypes.byref(b), ss._stream(DEV)), "ss_bwd")
    torch.cuda.synchronize()
    del ws_f, ws_b
    return dict(out=out, y=y, x=xck, last_state=last, du=du, ddelta=dd, dz=dz, dA=dA, dB=dB, dC=dC, dD=dD,
                ddelta_bias=db)


@pytest.mark.parametrize("batch,dim,seqlen,dtype,seg", CASES,
                         ids=[f"b{c[0]}_d{c[1]}_l{c[2]}_{str(c[3])[6:]}{'_seg' if c[4] else ''}" for c in CASES])
def test_small_windows_same_bits(batch, dim, seqlen, dtype, seg):
    print(f"\n[window] batch {batch} dim {dim} seqlen {seqlen} {dtype} segments {seg}", flush=True)
    sys.stdout.flush()
    x = make_inputs(batch, dim, 16, seqlen, seed=77 + seqlen)
    base = run(x, dtype, 0, seg)
    for k, v in base.items():
        assert torch.isfinite(v.float()).all(), f"{k}: non-finite values with the default window"
    # one window per super-chunk / chunk, then windows of several chunks
    # (dim x 16 x 4 bytes per chunk)
    for window in (1, 64 << 10):
        got = run(x, dtype, window, seg)
        for k in base:
            assert torch.equal(got[k], base[k]), f"{k}: window of {window} bytes differs from the default"
