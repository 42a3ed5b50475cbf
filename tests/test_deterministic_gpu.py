"""Deterministic sums of the backward (ss_bwd_args.deterministic).

With the flag, dB and dC are summed over channel blocks and dA, dD and
ddelta_bias over batch rows and sequence segments in a fixed order, so the
backward gives the same bits on every run.  Checked, through the C ABI
(``backward_into``):
* three runs bit-identical in every output, on the serial fast kernel, on
  a group with several dB / dC slices and on the sequence-segmented kernel
  (one long sequence);
* the results against the float64 oracle (fp32 rtol / atol 1e-3) and
  against the atomic sums to 1e-5 relative (the same sums in another
  order);
* accumulation (zero_grads off) adds the same bits to what the
  accumulators held;
* a HIP graph of the deterministic forward + backward replays bit for bit;
* torch.use_deterministic_algorithms(True) turns it on for autograd
  (selective_scan_fn), and for arguments the fast kernels do not take it
  raises as torch's own ops do, or warns under warn_only.
"""
import sys

import pytest
import torch

from oracle.selective_scan_ref import make_inputs
from tests._util import NAMES, assert_close, oracle_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GRADS = ("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz")


def _say(msg):
    print(f"\n[deterministic] {msg}", flush=True)
    sys.stdout.flush()


def _setup(batch, dim, L, seed, dtype=torch.float32):
    from mamba_amd import selective_scan as ss
    x = make_inputs(batch, dim, 16, L, seed=seed, dtype=dtype)
    t = {k: x[k].to(DEV) for k in NAMES + ("dout",)}
    out, y = torch.empty_like(t["delta"]), torch.empty_like(t["delta"])
    xck = torch.empty((batch, ss.n_chunks(L), dim, 16), dtype=torch.float32, device=DEV)
    ss.forward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, out, xck,
                    z=t["z"], y=y)
    return x, t, out, y, xck


def _backward(t, y, xck, det, zero=True, init=None):
    from mamba_amd import selective_scan as ss
    g = {"du": torch.empty_like(t["u"]), "ddelta": torch.empty_like(t["delta"]), "dz": torch.empty_like(t["z"])}
    for k, ref in (("dA", "A"), ("dB", "B"), ("dC", "C"), ("dD", "D"), ("ddelta_bias", "delta_bias")):
        g[k] = (init[k].clone() if init is not None else
                torch.full(t[ref].shape, float("nan"), dtype=torch.float32, device=DEV))
    ss.backward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck, True,
                     g["du"], g["ddelta"], g["dA"], g["dB"], g["dC"], g["dD"], g["ddelta_bias"],
                     z=t["z"], y=y, dz=g["dz"], zero_grads=zero, deterministic=det)
    torch.cuda.synchronize()
    return g


# (batch, dim, seqlen): serial fast kernel, 2 channel blocks per slice group
# boundary (192 blocks: 192 slices), one long sequence (8 segments), ragged
# seqlens (1001: identity-padded tail chunks in slices with padded rows;
# 2064: a wholly padded last chunk)
CASES = [(2, 256, 512), (1, 3072, 256), (1, 256, 4096), (1, 256, 1001), (2, 64, 2064)]


@pytest.mark.parametrize("case", CASES, ids=["serial", "many-blocks", "segments", "ragged-1001", "ragged-2064"])
def test_deterministic_backward_is_reproducible_and_correct(case):
    from mamba_amd import selective_scan as ss
    batch, dim, L = case
    _say(f"batch {batch} dim {dim} seqlen {L}")
    x, t, out, y, xck = _setup(batch, dim, L, seed=300 + dim)
    g0 = _backward(t, y, xck, det=True)
    nbytes = ss.workspace_bytes(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck,
                                True, g0["du"], g0["ddelta"], g0["dA"], g0["dB"], g0["dC"], g0["dD"],
                                g0["ddelta_bias"], z=t["z"], y=y, dz=g0["dz"], deterministic=True)
    assert nbytes >= 2 * (dim // 16) * batch * 16 * L * 4       # one dB / dC partial per channel block
    runs = [_backward(t, y, xck, det=True) for _ in range(3)]
    for k in GRADS:
        assert torch.equal(runs[0][k], runs[1][k]) and torch.equal(runs[0][k], runs[2][k]), f"{k} differs between runs"
    atomic = _backward(t, y, xck, det=False)
    for k in GRADS:
        w = atomic[k]
        assert_close(runs[0][k], w, 1e-5, 1e-5 * float(w.abs().max()), f"{k} vs atomic sums")
    if batch * dim * L <= 2 * 256 * 512:
        _, want = oracle_fwd_bwd(x)
        for k in NAMES:
            assert_close(runs[0]["d" + k].cpu(), want[k], 1e-3, 1e-3, f"d{k} vs oracle")
    # accumulation: the same sums added to what the accumulators held
    init = {k: torch.randn(runs[0][k].shape, device=DEV) for k in ("dA", "dB", "dC", "dD", "ddelta_bias")}
    acc = _backward(t, y, xck, det=True, zero=False, init=init)
    for k in init:
        assert torch.equal(acc[k], init[k] + runs[0][k]), k


def test_deterministic_graph_replays_bit_for_bit():
    from mamba_amd import selective_scan as ss
    batch, dim, L = 2, 256, 512
    _say("graph replays of the deterministic step")
    x, t, out, y, xck = _setup(batch, dim, L, seed=321)
    g = _backward(t, y, xck, det=True)
    bargs = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck, True,
             g["du"], g["ddelta"], g["dA"], g["dB"], g["dC"], g["dD"], g["ddelta_bias"])
    ws = torch.empty(ss.workspace_bytes(*bargs, z=t["z"], y=y, dz=g["dz"], deterministic=True),
                     dtype=torch.uint8, device=DEV)

    def step():
        ss.forward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, out, xck,
                        z=t["z"], y=y)
        ss.backward_into(*bargs, z=t["z"], y=y, dz=g["dz"], workspace=ws, zero_grads=True, deterministic=True)

    step()
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in g.items()}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep in range(3):
        for v in g.values():
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k in GRADS:
            assert torch.equal(g[k], eager[k]), f"replay {rep}: {k}"
        _ = (t["u"] * 2).sum().item()            # eager work between replays


def test_torch_deterministic_setting_drives_autograd():
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    _say("torch.use_deterministic_algorithms and selective_scan_fn")
    x = make_inputs(2, 256, 16, 512, seed=331)
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    prev = torch.are_deterministic_algorithms_enabled()
    prev_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)

        def grads(xx):
            p = {k: xx[k].to(DEV).requires_grad_(True) for k in names}
            out = selective_scan_fn(p["u"], p["delta"], p["A"], p["B"], p["C"], p["D"], z=p["z"],
                                    delta_bias=p["delta_bias"], delta_softplus=True)
            out.backward(xx["dout"].to(DEV))
            torch.cuda.synchronize()
            return {k: p[k].grad.clone() for k in names}
        a, b = grads(x), grads(x)
        for k in names:
            assert torch.equal(a[k], b[k]), k
        # dstate 32: the general kernel, which has no deterministic sums
        xr = make_inputs(1, 32, 32, 100, seed=332)
        with pytest.raises(RuntimeError, match="deterministic"):
            grads(xr)
        torch.use_deterministic_algorithms(True, warn_only=True)
        with pytest.warns(UserWarning, match="deterministic"):
            grads(xr)
    finally:
        torch.use_deterministic_algorithms(prev, warn_only=prev_warn)
