"""GPU parity at the committed fixtures and at the full benchmark sizes.

* the golden fixtures (tests/golden/ss_golden.npz, float64 C-oracle outputs)
  against the HIP path in fp32;
* batch 8, dim 1536, dstate 16, seqlen 2048, fp32, z gate, D, delta_bias,
  softplus: every output and gradient against the float64 C oracle on the
  same inputs (about 15 s of CPU time);
* batch 4, dim 5120, dstate 16, seqlen 8192, bf16: per-channel outputs and
  gradients of the first 256 channels against the C oracle on that channel
  slice, dB / dC of the slice run alone against the oracle, and dB / dC of
  the full run equal to the sum of the per-slice runs (the B and C
  gradients are sums over channels, so they add across channel slices).

Tolerances: fp32 rtol 1e-3 / atol 1e-3, bf16 rtol 2e-2 / atol 2e-2.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle.selective_scan_ref import make_inputs
from tests._util import NAMES, assert_close

pytestmark = pytest.mark.gpu

GRADS = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
         "delta_bias": "ddelta_bias"}


def _gpu_fwd_bwd(x, softplus=True):
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    dev = torch.device("cuda:0")
    g = {k: (x[k].to(dev).requires_grad_(True) if x[k] is not None else None) for k in NAMES}
    out, last = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                                  delta_bias=g["delta_bias"], delta_softplus=softplus, return_last_state=True)
    out.backward(x["dout"].to(dev))
    torch.cuda.synchronize()
    grads = {GRADS[k]: g[k].grad.cpu() for k in NAMES if g[k] is not None}
    return out.detach().cpu(), last.cpu(), grads


def _say(msg):
    print(f"\n[parity] {msg}", flush=True)
    sys.stdout.flush()


def test_golden_fixtures():
    from tests.golden import make_golden as mg
    data = np.load(mg.PATH)
    for name, (_, _, _, _, _, _, softplus, grads) in mg.CASES.items():
        _say(f"golden fixture {name}")
        x = mg.case_inputs(name)
        out, last, g = _gpu_fwd_bwd(x, softplus)
        assert_close(out, torch.from_numpy(data[f"{name}/out"]), 1e-3, 1e-3, f"{name}/out")
        assert_close(last, torch.from_numpy(data[f"{name}/last_state"]), 1e-3, 1e-3, f"{name}/last_state")
        if grads:
            for k, v in g.items():
                assert_close(v, torch.from_numpy(data[f"{name}/{k}"]), 1e-3, 1e-3, f"{name}/{k}")


def test_full_size_fp32_against_c_oracle():
    _say("full size fp32 b8-d1536-n16-l2048 (C oracle takes ~15 s)")
    x = make_inputs(8, 1536, 16, 2048, seed=1001)
    out, last, g = _gpu_fwd_bwd(x)
    args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    rout, rlast = c_oracle.fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args)
    assert_close(out, rout, 1e-3, 1e-3, "out")
    assert_close(last, rlast, 1e-3, 1e-3, "last_state")
    rg = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], dout=x["dout"], **args)
    for k, v in g.items():
        assert_close(v, rg[k], 1e-3, 1e-3, k)


def _slice(x, c0, c1):
    y = dict(x)
    for k in ("u", "delta", "z", "dout"):
        y[k] = x[k][:, c0:c1].contiguous()
    for k in ("A", "D", "delta_bias"):
        y[k] = x[k][c0:c1].contiguous()
    return y


def test_full_size_bf16_channel_slices():
    _say("full size bf16 b4-d5120-n16-l8192")
    x = make_inputs(4, 5120, 16, 8192, seed=1002, dtype=torch.bfloat16)
    out, last, g = _gpu_fwd_bwd(x)
    S = 256
    xs = _slice(x, 0, S)
    args = dict(D=xs["D"], z=xs["z"], delta_bias=xs["delta_bias"], delta_softplus=True)
    _say("C oracle on channels 0-255")
    rout, rlast = c_oracle.fwd(xs["u"], xs["delta"], xs["A"], xs["B"], xs["C"], **args)
    rg = c_oracle.bwd(xs["u"], xs["delta"], xs["A"], xs["B"], xs["C"], dout=xs["dout"], **args)
    tol = (2e-2, 2e-2)
    assert_close(out[:, :S].float(), rout, *tol, "out[:, :256]")
    assert_close(last[:, :S], rlast, *tol, "last_state[:, :256]")
    for k in ("du", "ddelta", "dz"):
        assert_close(g[k][:, :S].float(), rg[k], *tol, f"{k}[:, :256]")
    for k in ("dA", "dD", "ddelta_bias"):
        assert_close(g[k][:S], rg[k], *tol, f"{k}[:256]")
    # B / C gradients: the slice alone against the oracle, and additivity over
    # slices of the fp32 accumulators (the autograd layer rounds them to bf16)
    _say("bf16 per-slice runs for dB / dC additivity")
    dB_full, dC_full = _raw_dBC(x)
    assert_close(g["dB"].float(), dB_full, *tol, "dB (bf16 output of the fp32 accumulator)")
    dB = torch.zeros_like(dB_full)
    dC = torch.zeros_like(dC_full)
    for c0 in range(0, 5120, 1024):
        dBs, dCs = _raw_dBC(_slice(x, c0, c0 + 1024))
        dB += dBs
        dC += dCs
    dB0, dC0 = _raw_dBC(xs)
    assert_close(dB0, rg["dB"], *tol, "dB (channels 0-255)")
    assert_close(dC0, rg["dC"], *tol, "dC (channels 0-255)")
    assert_close(dB_full, dB, 1e-4, 1e-3, "dB additivity over channel slices")
    assert_close(dC_full, dC, 1e-4, 1e-3, "dC additivity over channel slices")


def _raw_dBC(x):
    """fp32 dB, dC of the native forward + backward (before any cast to B's dtype)."""
    from mamba_amd import selective_scan as ss
    dev = torch.device("cuda:0")
    t = {k: (x[k].to(dev) if x[k] is not None else None) for k in NAMES}
    dout = x["dout"].to(dev)
    out, xck, y = ss.forward(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, z=t["z"])
    res = ss.backward(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], dout, xck, True,
                      z=t["z"], y=y)
    torch.cuda.synchronize()
    assert res[3].dtype == torch.float32 and res[4].dtype == torch.float32
    return res[3].cpu(), res[4].cpu()
