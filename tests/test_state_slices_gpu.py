"""GPU parity of dstate 16 S on the fast kernels (one pass per 16-state slice).

A call with dstate 32, 48, ..., 256 (variable B and C, 16-channel groups)
runs the dstate-16 fast kernels once per slice of 16 states, with the sums
over states that the slices share (the forward's y, the backward's
sum_n g B and sum_n A g a h) carried from pass to pass in an fp32
workspace.  Each case runs selective_scan_fn (which allocates that
workspace) forward and backward, with return_last_state, and holds the
output, the last state and every gradient to the float64 C oracle on the
same inputs (fp32 rtol / atol 1e-3, bf16 and fp16 2e-2).  Shapes: ragged
seqlens (partial tail chunk and a chunk wholly past the sequence), bf16 and
fp16, no z gate, sequence segments (one batch row, long sequence), dB / dC
through workspace slices (97 channel blocks in the group), 16 slices
(dstate 256), two groups.

The checkpoints keep the (batch, chunk, dim, dstate) layout on every path,
so a forward on the slices followed by a backward on the general kernel
(no workspace), and the reverse, give the same results: checked against
the oracle too.

The general kernels' padding lanes (states past dstate in the last group
of 16, or whole groups when dstate is below 16 x the template's group
count: 48, 80, 96, 144, 200) are checked against the oracle at 24 channels
(not a multiple of 16, so only the general kernels apply), with variable
and constant B / C.
"""
import sys

import pytest
import torch

from mamba_amd import selective_scan as ss
from oracle import c_oracle
from oracle.selective_scan_ref import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-3, torch.bfloat16: 2e-2, torch.float16: 2e-2}
GRADS = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
         "delta_bias": "ddelta_bias"}

# (batch, dim, dstate, seqlen, dtype, has_z, n_groups)
CASES = [
    (2, 64, 32, 333, torch.float32, True, 1),      # ragged: a partial chunk and one wholly past the sequence
    (2, 48, 64, 256, torch.bfloat16, True, 1),     # 4 slices, bf16
    (1, 32, 48, 130, torch.float16, False, 1),     # 3 slices, fp16, no z
    (1, 32, 32, 4100, torch.float32, True, 1),     # one row, long: sequence segments in every pass
    (1, 1552, 32, 128, torch.float32, True, 1),    # 97 channel blocks: dB / dC through workspace slices
    (2, 32, 256, 100, torch.float32, True, 1),     # 16 slices, the largest dstate
    (2, 64, 32, 96, torch.float32, True, 2),       # two groups of 32 channels
]


def _ids(c):
    b, d, n, l, dt, z, g = c
    return f"b{b}-d{d}-n{n}-l{l}-{str(dt).split('.')[-1]}{'-z' if z else ''}-g{g}"


def _oracle(x, has_z):
    args = dict(D=x["D"], z=x["z"] if has_z else None, delta_bias=x["delta_bias"], delta_softplus=True)
    out, last = c_oracle.fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args)
    grads = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], dout=x["dout"], **args)
    return out, last, grads


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_state_slices_match_oracle(case):
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    b, d, n, l, dt, hz, G = case
    print(f"\n[slices] selective_scan_fn {_ids(case)}", flush=True)
    sys.stdout.flush()
    x = make_inputs(b, d, n, l, seed=2024 + n + l, dtype=dt, n_groups=G, has_z=hz)
    g = {k: (v.to(DEV).requires_grad_(True) if v is not None else None) for k, v in x.items() if k != "dout"}
    out0 = torch.empty_like(g["u"])
    xck = torch.empty((b, ss.n_chunks(l), d, n), device=DEV)
    assert ss.forward_kernel_name(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["delta_bias"], True,
                                  out0, xck, z=g["z"], y=torch.empty_like(out0) if hz else None) == "ss_fwd_fast"
    out, last = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                                  delta_bias=g["delta_bias"], delta_softplus=True, return_last_state=True)
    out.backward(x["dout"].to(DEV))
    torch.cuda.synchronize()
    rout, rlast, rg = _oracle(x, hz)
    tol = TOL[dt]
    assert out.dtype == dt
    assert_close(out.detach().cpu(), rout, tol, tol, "out")
    assert_close(last.cpu(), rlast, tol, tol, "last_state")
    for k, v in g.items():
        if v is not None:
            assert_close(v.grad.cpu(), rg[GRADS[k]], tol, tol, GRADS[k])


def _fwd(t, fast):
    b, d, l = t["u"].shape
    n = t["A"].shape[1]
    out, y = torch.empty_like(t["u"]), torch.empty_like(t["u"])
    xck = torch.empty((b, ss.n_chunks(l), d, n), device=DEV)
    ss.forward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, out, xck,
                    z=t["z"], y=y, workspace="auto" if fast else None)
    return out, y, xck


def _bwd(t, y, xck, fast):
    du, dd, dz = (torch.empty_like(t["u"]) for _ in range(3))
    dA = torch.empty(t["A"].shape, device=DEV)
    dB, dC = torch.empty(t["B"].shape, device=DEV), torch.empty(t["C"].shape, device=DEV)
    dD, db = torch.empty(t["D"].shape, device=DEV), torch.empty(t["delta_bias"].shape, device=DEV)
    ss.backward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck, True,
                     du, dd, dA, dB, dC, dD, db, z=t["z"], y=y, dz=dz, workspace="auto" if fast else None,
                     zero_grads=True)
    return dict(du=du, ddelta=dd, dz=dz, dA=dA, dB=dB, dC=dC, dD=dD, ddelta_bias=db)


@pytest.mark.parametrize("fwd_fast,bwd_fast", [(True, False), (False, True), (False, False)],
                         ids=["slices-then-general", "general-then-slices", "general"])
def test_paths_share_the_checkpoints(fwd_fast, bwd_fast):
    b, d, n, l = 2, 32, 32, 200
    print(f"\n[slices] forward {'slices' if fwd_fast else 'general'}, backward {'slices' if bwd_fast else 'general'}",
          flush=True)
    sys.stdout.flush()
    x = make_inputs(b, d, n, l, seed=77)
    t = {k: v.to(DEV) for k, v in x.items()}
    out, y, xck = _fwd(t, fwd_fast)
    got = _bwd(t, y, xck, bwd_fast)
    torch.cuda.synchronize()
    rout, _, rg = _oracle(x, True)
    assert_close(out.cpu(), rout, 1e-3, 1e-3, "out")
    for k, v in got.items():
        assert_close(v.cpu(), rg[k], 1e-3, 1e-3, k)


# (dstate, var_B, var_C, seqlen): the general kernels run states in groups of
# 16 per lane row, SPL = 1, 2, 4, 8 or 16 groups; a dstate below 16 SPL
# leaves padding lanes, in the last group (40: 8 of them) or as whole groups
# (48 on SPL 4, 80 and 96 on SPL 8, 144 on SPL 16).  Padding lanes must add
# nothing to y, du or ddelta.
PAD_CASES = [
    (40, True, True, 77),
    (48, True, True, 77),
    (48, False, True, 50),
    (48, True, False, 50),
    (80, True, True, 33),
    (96, True, True, 40),
    (144, True, True, 20),
    (200, True, True, 20),
]


@pytest.mark.parametrize("case", PAD_CASES, ids=[f"n{c[0]}-{'vB' if c[1] else 'cB'}-{'vC' if c[2] else 'cC'}-l{c[3]}"
                                                 for c in PAD_CASES])
def test_general_kernels_with_padding_state_groups(case):
    n, var_B, var_C, l = case
    b, d = 2, 24
    print(f"\n[slices] general kernels dstate {n} var_B {var_B} var_C {var_C} seqlen {l}", flush=True)
    sys.stdout.flush()
    x = make_inputs(b, d, n, l, seed=300 + n + l, var_B=var_B, var_C=var_C)
    t = {k: v.to(DEV) for k, v in x.items()}
    out, y, xck = _fwd(t, False)
    got = _bwd(t, y, xck, False)
    torch.cuda.synchronize()
    rout, _, rg = _oracle(x, True)
    assert_close(out.cpu(), rout, 1e-3, 1e-3, "out")
    for k, v in got.items():
        assert_close(v.cpu(), rg[k], 1e-3, 1e-3, k)
