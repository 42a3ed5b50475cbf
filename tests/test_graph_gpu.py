"""The selective scan's forward + backward captured into a HIP graph.

The library clears its gradient accumulators and scratch with fill kernels
(never memsets), so a whole training step of the scan can be captured and
replayed.  Each case captures forward_into + backward_into (zero_grads, the
library's workspace) once, then replays the graph three times with eager
work and synchronisations between the replays, and checks every output of
every replay against the eager step: out, y, checkpoints and du / ddelta /
dz exactly; the atomically summed dA, dB, dC, dD, ddelta_bias to 1e-5
relative (their summation order varies from run to run).  Cases: the fast
kernels with the dB / dC workspace slices, the general kernels (ragged
seqlen, dstate 4), and the sequence-parallel kernels of a long single
sequence.
"""
import sys

import pytest
import torch

from oracle.selective_scan_ref import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

CASES = [(1, 3072, 16, 256, torch.float32), (2, 64, 4, 100, torch.float32), (1, 64, 16, 4096, torch.bfloat16)]


@pytest.mark.parametrize("case", CASES, ids=["fast-slices", "general", "segments"])
def test_scan_step_graph_replays(case):
    from mamba_amd import selective_scan as ss
    batch, dim, N, L, dt = case
    print(f"\n[graph] scan fwd+bwd capture b{batch}-d{dim}-n{N}-l{L} {dt}", flush=True)
    sys.stdout.flush()
    x = make_inputs(batch, dim, N, L, seed=41, dtype=dt)
    t = {k: x[k].to(DEV) for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias", "dout")}
    fargs = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True)
    out, y = torch.empty_like(t["delta"]), torch.empty_like(t["delta"])
    xck = torch.empty((batch, ss.n_chunks(L), dim, N), dtype=torch.float32, device=DEV)
    grads = [torch.empty_like(t["u"]), torch.empty_like(t["delta"]), torch.empty(t["A"].shape, device=DEV),
             torch.empty(t["B"].shape, device=DEV), torch.empty(t["C"].shape, device=DEV),
             torch.empty(t["D"].shape, device=DEV), torch.empty(t["delta_bias"].shape, device=DEV)]
    dz = torch.empty_like(t["z"])
    bargs = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck, True, *grads)
    fws = ss.forward_workspace_bytes(*fargs, out, xck, z=t["z"], y=y)
    fwork = torch.empty(max(fws, 16), dtype=torch.uint8, device=DEV) if fws else None
    bws = ss.workspace_bytes(*bargs, z=t["z"], y=y, dz=dz)
    bwork = torch.empty(max(bws, 16), dtype=torch.uint8, device=DEV) if bws else None
    if L == 4096:
        assert fws > 0 and bws > 0, "the long single sequence should use sequence segments"
    if dim == 3072:
        assert fws == 0 and bws == 2 * 2 * 16 * L * 4, "192 channel blocks should use 2 dB / dC slices"

    def step():
        ss.forward_into(*fargs, out, xck, z=t["z"], y=y, workspace=fwork)
        ss.backward_into(*bargs, z=t["z"], y=y, dz=dz, workspace=bwork, zero_grads=True)

    def snapshot():
        return [v.clone() for v in (out, y, xck, dz, *grads)]

    step()
    torch.cuda.synchronize()
    want = snapshot()

    # capture on a side stream, as torch requires
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    names = ("out", "y", "x", "dz", "du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias")
    for rep in range(3):
        for v in (out, y, xck, dz, *grads):          # eager work between replays: poison every output
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = snapshot()
        for name, a, b in zip(names, got, want):
            if name in ("dA", "dB", "dC", "dD", "ddelta_bias"):
                assert_close(a.float().cpu(), b.float().cpu(), 1e-5, 1e-5 * max(1.0, float(b.abs().max())),
                             f"replay {rep} {name}")
            else:
                assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager step"
