"""Seeded random shapes: the scan kernels against the float64 C oracle.

Each case draws batch, dim, dstate, seqlen, I/O dtype, group count, which
of B / C vary per step, which of z, D, delta_bias and softplus are present,
and whether the sequence tensors are views with padded rows (a row stride
above seqlen).  The forward and backward run through the C ABI
(``forward_into`` / ``backward_into``, with and without workspace), and every
output and gradient is compared elementwise with ``oracle/ss_oracle.c`` on
the same (already rounded) inputs: fp32 rtol / atol 1e-3, bf16 / fp16
2e-2.  The draw covers both the fast kernels (dstate 16, variable B and C,
16-channel groups) and the general ones, ragged and tiny seqlens, and the
sequence-segmented paths (small batch x dim with long sequences).  A second
draw holds dstate 32 to 128 (multiples of 16) with variable B and C and
16-channel groups: with a workspace those run as one fast-kernel pass per
16-state slice, without one on the general kernels.  A third draws any
dstate from 1 to 256, any channel count per group, constant or variable B
and C, and in about a third of the cases gradient accumulators that hold
seeded values (no zero_grads: the backward must add to them).  A fourth
holds dstate 16 with B and C, or one of them, constant, which the fast
kernels take.

``MAMBA_AMD_RANDOM_SWEEP=N`` adds a sweep of N more seeds over all four
draws (deterministic sums on about a third of the fast-kernel cases with a
workspace); without it the sweep is skipped.
"""
import os
import random
import sys

import pytest
import torch

from oracle import c_oracle
from oracle.selective_scan_ref import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-3, torch.bfloat16: 2e-2, torch.float16: 2e-2}
N_CASES = 96


def _draw(i):
    rnd = random.Random(9000 + i)
    dtype = rnd.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
    fast = rnd.random() < 0.7
    dstate = 16 if fast else rnd.choice([1, 4, 8, 16, 32])
    n_groups = rnd.choice([1, 1, 2])
    per_group = rnd.choice([16, 32, 48]) if fast else rnd.choice([8, 10, 16, 24])
    dim = n_groups * per_group
    batch = rnd.choice([1, 1, 2, 3])
    seqlen = rnd.choice([1, 2, 15, 16, 17, 31, 33, 63, 64, 65, 127, 500, 1001, 2047, 2049, 3000,
                         rnd.randint(1, 4096)])
    var_B = True if fast else rnd.random() < 0.7
    var_C = True if fast else rnd.random() < 0.7
    return dict(batch=batch, dim=dim, dstate=dstate, seqlen=seqlen, dtype=dtype, n_groups=n_groups,
                var_B=var_B, var_C=var_C, has_z=rnd.random() < 0.8, has_D=rnd.random() < 0.8,
                has_bias=rnd.random() < 0.8, softplus=rnd.random() < 0.8, pad=rnd.choice([0, 0, 1, 3, 8]),
                workspace=rnd.choice(["auto", "auto", None]), seed=9100 + i)


def _seq_view(t, pad):
    """t as a view with rows of seqlen + pad elements (the padding NaN)."""
    if pad == 0:
        return t.contiguous()
    b, d, L = t.shape
    buf = torch.full((b, d, L + pad), float("nan"), dtype=t.dtype, device=t.device)
    v = buf[..., :L]
    v.copy_(t)
    return v


def _draw_slices(i):
    rnd = random.Random(9500 + i)
    n_groups = rnd.choice([1, 1, 2])
    return dict(batch=rnd.choice([1, 2, 3]), dim=n_groups * rnd.choice([16, 32]),
                dstate=rnd.choice([32, 32, 48, 64, 64, 128]),
                seqlen=rnd.choice([1, 17, 63, 64, 65, 500, 2047, 2049, rnd.randint(1, 3000)]),
                dtype=rnd.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16]),
                n_groups=n_groups, var_B=True, var_C=True, has_z=rnd.random() < 0.8,
                has_D=rnd.random() < 0.8, has_bias=rnd.random() < 0.8, softplus=rnd.random() < 0.8,
                pad=rnd.choice([0, 0, 1, 8]), workspace=rnd.choice(["auto", "auto", "auto", None]),
                seed=9600 + i)


def _draw_general(i):
    rnd = random.Random(9800 + i)
    n_groups = rnd.choice([1, 1, 2, 3])
    var_B, var_C = rnd.random() < 0.6, rnd.random() < 0.6
    return dict(batch=rnd.choice([1, 2, 3]), dim=n_groups * rnd.randint(1, 24), dstate=rnd.randint(1, 256),
                seqlen=rnd.choice([1, 16, 33, rnd.randint(1, 600)]),
                dtype=rnd.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16]),
                n_groups=n_groups, var_B=var_B, var_C=var_C, has_z=rnd.random() < 0.7,
                has_D=rnd.random() < 0.7, has_bias=rnd.random() < 0.7, softplus=rnd.random() < 0.8,
                pad=rnd.choice([0, 1, 5]), workspace=rnd.choice(["auto", None]), seed=9900 + i,
                accumulate=rnd.random() < 0.3)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape_against_c_oracle(i):
    c = _draw(i)
    print(f"\n[random] case {i}: {c}", flush=True)
    sys.stdout.flush()
    _run_case(c)


@pytest.mark.parametrize("i", range(24))
def test_random_state_slices_against_c_oracle(i):
    c = _draw_slices(i)
    print(f"\n[random slices] case {i}: {c}", flush=True)
    sys.stdout.flush()
    _run_case(c)


def _draw_const_bc(i):
    rnd = random.Random(9700 + i)
    var_B, var_C = rnd.choice([(False, False), (False, False), (True, False), (False, True)])
    dim = rnd.choice([16, 32, 48, 64])
    n_groups = rnd.choice([1, 2]) if (var_B or var_C) and dim % 32 == 0 else 1
    return dict(batch=rnd.choice([1, 2, 3]), dim=dim, dstate=16,
                seqlen=rnd.choice([1, 15, 17, 63, 64, 100, 2047, 2049, rnd.randint(1, 3000)]),
                dtype=rnd.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16]),
                n_groups=n_groups, var_B=var_B, var_C=var_C, has_z=rnd.random() < 0.8,
                has_D=rnd.random() < 0.8, has_bias=rnd.random() < 0.8, softplus=rnd.random() < 0.8,
                pad=rnd.choice([0, 0, 1, 8]), workspace=rnd.choice(["auto", None]), seed=9750 + i,
                accumulate=rnd.random() < 0.3)


@pytest.mark.parametrize("i", range(32))
def test_random_constant_bc_against_c_oracle(i):
    c = _draw_const_bc(i)
    print(f"\n[random constant B / C] case {i}: {c}", flush=True)
    sys.stdout.flush()
    _run_case(c)


@pytest.mark.parametrize("i", range(32))
def test_random_general_shapes_against_c_oracle(i):
    c = _draw_general(i)
    print(f"\n[random general] case {i}: {c}", flush=True)
    sys.stdout.flush()
    _run_case(c)


# channel blocks of 16 on the general kernels: a block with padding channels
# past dim in one group (summed over the block in LDS), blocks that straddle
# two groups (every lane adds its own dB / dC), and a wide row of 1000
# channels in one group
CHANNEL_CASES = [
    dict(batch=2, dim=40, dstate=16, seqlen=300, n_groups=1, dtype=torch.float32),
    dict(batch=2, dim=72, dstate=16, seqlen=211, n_groups=3, dtype=torch.float32),
    dict(batch=1, dim=1000, dstate=16, seqlen=129, n_groups=1, dtype=torch.bfloat16),
    dict(batch=1, dim=120, dstate=20, seqlen=97, n_groups=5, dtype=torch.float16),
]


@pytest.mark.parametrize("i", range(len(CHANNEL_CASES)))
def test_general_kernels_channel_blocks_against_c_oracle(i):
    c = dict(CHANNEL_CASES[i], var_B=True, var_C=True, has_z=True, has_D=True, has_bias=True, softplus=True,
             pad=0, workspace="auto", seed=9960 + i, accumulate=i % 2 == 1)
    print(f"\n[random channel blocks] case {i}: {c}", flush=True)
    sys.stdout.flush()
    _run_case(c)


SWEEP = int(os.environ.get("MAMBA_AMD_RANDOM_SWEEP", "0"))


@pytest.mark.skipif(SWEEP <= 0, reason="set MAMBA_AMD_RANDOM_SWEEP=N for a sweep of N more seeds")
def test_random_sweep_against_c_oracle():
    failures = []
    for i in range(SWEEP):
        rnd = random.Random(100000 + i)
        kind = rnd.choice(["base", "slices", "general", "const"])
        draw = {"base": _draw, "slices": _draw_slices, "general": _draw_general, "const": _draw_const_bc}[kind]
        c = draw(100000 + i)
        fast = (c["dstate"] % 16 == 0 and c["var_B"] and c["var_C"] and c["dim"] % 16 == 0
                and (c["dim"] // c["n_groups"]) % 16 == 0)
        if fast and c["workspace"] == "auto" and rnd.random() < 0.35:
            c["det"] = True
        try:
            _run_case(c)
        except AssertionError as e:
            failures.append(f"seed {100000 + i} ({kind}): {c}: {str(e)[:200]}")
            print(f"\n[random sweep] FAIL {failures[-1]}", flush=True)
        if i % 100 == 99:
            print(f"\n[random sweep] {i + 1}/{SWEEP} cases, {len(failures)} failures", flush=True)
    assert not failures, "\n".join(failures[:10])


def _run_case(c):
    from mamba_amd import selective_scan as ss
    x = make_inputs(c["batch"], c["dim"], c["dstate"], c["seqlen"], seed=c["seed"], dtype=c["dtype"],
                    n_groups=c["n_groups"], var_B=c["var_B"], var_C=c["var_C"], has_z=c["has_z"],
                    has_D=c["has_D"], has_delta_bias=c["has_bias"])
    if not c["softplus"]:
        # without softplus the step size is used as given: keep it positive so
        # the recurrence is stable (a = exp(delta * A) < 1), as the other
        # parity tests do
        x["delta"] = (x["delta"].float().abs() * 0.5).to(c["dtype"])
        if x["delta_bias"] is not None:
            x["delta_bias"] = x["delta_bias"].abs()
    dt, pad, ws = c["dtype"], c["pad"], c["workspace"]
    g = {k: (v.to(DEV) if v is not None else None) for k, v in x.items()}
    u, dl = _seq_view(g["u"], pad), _seq_view(g["delta"], pad)
    z = _seq_view(g["z"], pad) if c["has_z"] else None
    dout = _seq_view(g["dout"], pad)
    A, B, C, D, bias = g["A"], g["B"], g["C"], g["D"], g["delta_bias"]
    batch, dim, L = u.shape
    out = _seq_view(torch.empty(batch, dim, L, dtype=dt, device=DEV), pad)
    y = _seq_view(torch.empty(batch, dim, L, dtype=dt, device=DEV), pad) if z is not None else None
    xck = torch.empty((batch, ss.n_chunks(L), dim, c["dstate"]), dtype=torch.float32, device=DEV)
    ss.forward_into(u, dl, A, B, C, D, bias, c["softplus"], out, xck, z=z, y=y, workspace=ws)
    du, dd = (_seq_view(torch.empty(batch, dim, L, dtype=dt, device=DEV), pad) for _ in range(2))
    dz = _seq_view(torch.empty(batch, dim, L, dtype=dt, device=DEV), pad) if z is not None else None
    acc = c.get("accumulate", False)
    gen = torch.Generator().manual_seed(c["seed"] + 1)
    start = {}

    def grad_buf(shape):
        if not acc:
            return torch.empty(shape, dtype=torch.float32, device=DEV)
        v = torch.randn(shape, generator=gen)
        start[len(start)] = v
        return v.to(DEV)

    dA, dB, dC = grad_buf(A.shape), grad_buf(B.shape), grad_buf(C.shape)
    dD = grad_buf(D.shape) if D is not None else None
    db = grad_buf(bias.shape) if bias is not None else None
    ss.backward_into(u, dl, A, B, C, D, bias, dout, xck, c["softplus"], du, dd, dA, dB, dC, dD, db,
                     z=z, y=y, dz=dz, workspace=ws, zero_grads=not acc, deterministic=c.get("det"))
    torch.cuda.synchronize()

    args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=c["softplus"])
    rout, _ = c_oracle.fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args)
    rg = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], dout=x["dout"], **args)
    tol = TOL[dt]
    assert_close(out.float().cpu(), rout, tol, tol, "out")
    got = dict(du=du, ddelta=dd, dA=dA, dB=dB, dC=dC, dD=dD, ddelta_bias=db, dz=dz)
    if acc:
        # without zero_grads the backward adds to what the accumulators held
        base = dict(zip([k for k in ("dA", "dB", "dC", "dD", "ddelta_bias") if got[k] is not None],
                        start.values()))
        rg = {k: (v + base[k] if k in base else v) for k, v in rg.items() if v is not None}
    for k, v in got.items():
        if v is None:
            continue
        assert_close(v.float().cpu(), rg[k], tol, tol, k)
