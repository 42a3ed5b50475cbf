"""GPU parity at a million steps.

One 16-channel block (batch 1, dim 16, dstate 16, fp32, z gate, D,
delta_bias, softplus) over a very long sequence, forward and backward
through selective_scan_fn against the float64 C oracle on the same inputs:
* seqlen 2^20: the largest chunk indices the kernels form at this width and
  the sequence-segmented forward and backward with the most segments (64);
* seqlen 1,000,003: a ragged length (64 segments of unequal length in both
  directions), with the identity-padded tail.
The per-step outputs and gradients are held to rtol / atol 1e-3; dA, dD
and ddelta_bias, sums over a million steps in fp32 on the GPU, to 2e-3.
About 10 s of CPU time per case for the oracle.

Then 1040 channels x 2^20 + 37 steps (seqlen x dim above 2^30, so the
checkpoints of a row span more than 2^32 bytes): three 16-channel blocks of
that launch (first, middle, last) against the same scan run on those blocks
alone, forward outputs and every per-channel gradient, to 1e-4 relative
(the two launches join different numbers of sequence segments).
"""
import sys

import pytest
import torch

from oracle import c_oracle
from oracle.selective_scan_ref import make_inputs
from tests._util import NAMES, assert_close

pytestmark = pytest.mark.gpu
GRADS = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
         "delta_bias": "ddelta_bias"}
SUMS_OVER_TIME = ("dA", "dD", "ddelta_bias")


@pytest.mark.parametrize("seqlen", [1 << 20, 1_000_003], ids=["2^20", "1000003"])
def test_million_steps_against_c_oracle(seqlen):
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    print(f"\n[long] batch 1 dim 16 seqlen {seqlen}", flush=True)
    sys.stdout.flush()
    dev = torch.device("cuda:0")
    x = make_inputs(1, 16, 16, seqlen, seed=1234 + seqlen % 97)
    g = {k: x[k].to(dev).requires_grad_(True) for k in NAMES}
    out, last = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                                  delta_bias=g["delta_bias"], delta_softplus=True, return_last_state=True)
    out.backward(x["dout"].to(dev))
    torch.cuda.synchronize()
    args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    rout, rlast = c_oracle.fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args)
    assert_close(out.detach().cpu(), rout, 1e-3, 1e-3, "out")
    assert_close(last.cpu(), rlast, 1e-3, 1e-3, "last_state")
    rg = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], dout=x["dout"], **args)
    for k in NAMES:
        name = GRADS[k]
        tol = 2e-3 if name in SUMS_OVER_TIME else 1e-3
        assert_close(g[k].grad.cpu(), rg[name], tol, tol, name)


def test_checkpoints_past_4_gib_per_row():
    from mamba_amd import selective_scan as ss
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    dim, L = 1040, (1 << 20) + 37
    print(f"\n[long] batch 1 dim {dim} seqlen {L} (seqlen x dim {dim * L})", flush=True)
    sys.stdout.flush()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(4321)
    r = lambda *s: torch.randn(*s, generator=gen, device=dev)
    u, dl, z, dout = r(1, dim, L), r(1, dim, L) * 0.5, r(1, dim, L), r(1, dim, L)
    B, C = r(1, 1, 16, L), r(1, 1, 16, L)
    A = -torch.rand(dim, 16, generator=gen, device=dev) * 3 - 0.1
    D, bias = r(dim), r(dim) * 0.5 - 3.0
    out = torch.empty_like(dl)
    xck = torch.empty((1, ss.n_chunks(L), dim, 16), device=dev)
    assert ss.forward_kernel_name(u, dl, A, B, C, D, bias, True, out, xck, z=z, y=torch.empty_like(out)) \
        == "ss_fwd_fast"
    del out, xck

    def run(sl):
        p = [t.detach()[..., sl, :].contiguous().requires_grad_(True) if t.dim() == 3 else
             t.detach()[sl].contiguous().requires_grad_(True) for t in (u, dl, A, z, D, bias)]
        uu, dd, AA, zz, DD, bb = p
        o = selective_scan_fn(uu, dd, AA, B, C, DD, z=zz, delta_bias=bb, delta_softplus=True)
        grads = torch.autograd.grad(o, (uu, dd, AA, zz, DD, bb), dout[:, sl].contiguous())
        torch.cuda.synchronize()
        return [o.detach()] + list(grads)

    full = run(slice(0, dim))
    names = ("out", "du", "ddelta", "dA", "dz", "dD", "ddelta_bias")
    for c0 in (0, 512, dim - 16):
        part = run(slice(c0, c0 + 16))
        for name, a, b in zip(names, full, part):
            a = a[:, c0:c0 + 16] if a.dim() == 3 else a[c0:c0 + 16]
            scale = max(1.0, float(b.abs().max()))
            assert_close(a.cpu(), b.cpu(), 1e-4, 1e-4 * scale, f"{name}, channels {c0}..{c0 + 15}")
        del part
