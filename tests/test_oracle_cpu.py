"""CPU checks that pin the two oracles (no GPU needed).

The reference ships no tests, golden vectors or fixtures for the selective
scan, and its CUDA kernels cannot be built here, so the oracles
(oracle/selective_scan_ref.py in PyTorch, oracle/ss_oracle.c in float64 C)
are pinned by what the mathematics fixes:

* a brute-force scalar loop over Python floats on tiny inputs;
* closed forms: A = 0 without softplus is a cumulative sum; seqlen 1 is
  y = D u + sum_n C delta u B; dstate 1 with constant delta and B = C = 1 is a
  first-order IIR filter (scipy.signal.lfilter); the softplus threshold;
  the z gate y * silu(z) (scipy.special.expit);
* structure: constant B / C equal variable B / C broadcast over batch and
  time, n_groups equal an explicit per-channel broadcast, causality, and
  linearity in u for fixed delta;
* gradients: fp64 gradcheck of the PyTorch oracle, central finite differences
  of the C oracle, the C backward against autograd, and the identities
  dD = sum dy u, ddelta_bias = sum ddelta, dz = dout y silu'(z);
* the committed fixtures in tests/golden/ as a regression pin.

``test_planted_mistakes_are_caught`` runs the forward checks against
deliberately wrong variants of the oracle (a dropped D term, a flipped A
sign, swapped B and C, reversed time, ...) and requires each to fail at
least one of them.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.signal import lfilter
from scipy.special import expit

from oracle import c_oracle
from oracle.selective_scan_ref import make_inputs, selective_scan_ref

F64 = torch.float64


# ------------------------------------------------------------------ oracles --
def ref64(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    return selective_scan_ref(u, delta, A, B, C, D, z=z, delta_bias=delta_bias,
                              delta_softplus=delta_softplus, compute_dtype=F64)


def c64(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    return c_oracle.fwd(u, delta, A, B, C, D=D, z=z, delta_bias=delta_bias, delta_softplus=delta_softplus)[0]


ORACLES = {"torch": ref64, "c": c64}


def brute_force(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    """Scalar loops over Python floats (float64), one (batch, channel) row at a time."""
    u, delta, A = (t.double().numpy() for t in (u, delta, A))
    var_B, var_C = B.dim() >= 3, C.dim() >= 3
    Bn, Cn = B.double().numpy(), C.double().numpy()
    Dn = D.double().numpy() if D is not None else None
    zn = z.double().numpy() if z is not None else None
    bn = delta_bias.double().numpy() if delta_bias is not None else None
    Bt, dim, L = u.shape
    N = A.shape[1]
    G = B.shape[1] if var_B else (C.shape[1] if var_C else 1)
    out = np.zeros((Bt, dim, L))
    for b in range(Bt):
        for d in range(dim):
            g = d // (dim // G)
            h = [0.0] * N
            for t in range(L):
                x = float(delta[b, d, t]) + (float(bn[d]) if bn is not None else 0.0)
                if delta_softplus and x <= 20.0:
                    x = math.log1p(math.exp(x))
                uu = float(u[b, d, t])
                acc = 0.0
                for n in range(N):
                    bv = float(Bn[b, g, n, t]) if var_B else float(Bn[d, n])
                    cv = float(Cn[b, g, n, t]) if var_C else float(Cn[d, n])
                    h[n] = math.exp(x * float(A[d, n])) * h[n] + x * uu * bv
                    acc += cv * h[n]
                if Dn is not None:
                    acc += float(Dn[d]) * uu
                if zn is not None:
                    zz = float(zn[b, d, t])
                    acc *= zz / (1.0 + math.exp(-zz))
                out[b, d, t] = acc
    return torch.from_numpy(out)


def _close(got, want, rtol=1e-10, atol=1e-12):
    got, want = torch.as_tensor(got).double(), torch.as_tensor(want).double()
    return bool(got.shape == want.shape and torch.allclose(got, want, rtol=rtol, atol=atol))


def _inputs(batch, dim, dstate, seqlen, seed, positive_delta=False, **kw):
    """Seeded fp64 inputs.  Without softplus a negative delta + delta_bias makes
    exp(delta A) grow without bound, so those cases (``positive_delta``) shift
    delta so that delta + delta_bias = |delta| / 2."""
    x = make_inputs(batch, dim, dstate, seqlen, seed=seed, **kw)
    x = {k: (v.double() if v is not None else None) for k, v in x.items()}
    if positive_delta:
        bias = x["delta_bias"][:, None] if x["delta_bias"] is not None else 0.0
        x["delta"] = x["delta"].abs() * 0.5 - bias
    return x


# ------------------------------------------------------- forward pin checks --
# Each returns True when `fwd` agrees with what the check fixes.
def check_brute_force(fwd):
    ok = True
    for kw, sp in (({"n_groups": 2}, True), ({"var_B": False, "has_z": False}, False),
                   ({"var_C": False, "has_D": False, "has_delta_bias": False}, True)):
        x = _inputs(2, 4, 3, 9, seed=11, positive_delta=not sp, **kw)
        args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=sp)
        ok &= _close(fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args),
                     brute_force(x["u"], x["delta"], x["A"], x["B"], x["C"], **args))
    return ok


def check_A_zero_cumsum(fwd):
    """A = 0, no softplus, no bias: h_t = sum_{s<=t} delta_s u_s B_s."""
    x = _inputs(2, 5, 4, 33, seed=12, positive_delta=True, has_z=False, has_delta_bias=False)
    A = torch.zeros_like(x["A"])
    got = fwd(x["u"], x["delta"], A, x["B"], x["C"], D=x["D"], delta_softplus=False)
    h = torch.cumsum((x["delta"] * x["u"])[:, :, None, :] * x["B"], dim=-1)   # (Bt, D, N, L), G = 1
    want = (x["C"] * h).sum(2) + x["D"][:, None] * x["u"]
    return _close(got, want)


def check_seqlen_one(fwd):
    """L = 1: y = D u + sum_n C delta u B with delta = softplus(delta + bias)."""
    x = _inputs(3, 6, 5, 1, seed=13, has_z=False)
    got = fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], delta_bias=x["delta_bias"],
              delta_softplus=True)
    dt = np.logaddexp(0.0, (x["delta"] + x["delta_bias"][:, None]).numpy())   # softplus via logaddexp
    want = (x["C"] * x["B"]).sum(2).numpy() * dt * x["u"].numpy() + x["D"].numpy()[:, None] * x["u"].numpy()
    return _close(got, want)


def check_iir_filter(fwd):
    """dstate 1, constant delta_d, B = C = 1: y = lfilter([delta], [1, -exp(delta a)], u) + D u."""
    g = torch.Generator().manual_seed(14)
    Bt, dim, L = 2, 3, 50
    u = torch.randn(Bt, dim, L, generator=g, dtype=F64)
    dl = torch.rand(dim, generator=g, dtype=F64) * 0.5 + 0.1
    delta = dl[None, :, None].expand(Bt, dim, L).contiguous()
    A = -(torch.rand(dim, 1, generator=g, dtype=F64) * 2 + 0.1)
    one = torch.ones(dim, 1, dtype=F64)
    Dv = torch.randn(dim, generator=g, dtype=F64)
    got = fwd(u, delta, A, one, one, D=Dv, delta_softplus=False)
    want = np.empty((Bt, dim, L))
    for d in range(dim):
        a = math.exp(float(dl[d] * A[d, 0]))
        want[:, d] = lfilter([float(dl[d])], [1.0, -a], u[:, d].numpy(), axis=-1) + float(Dv[d]) * u[:, d].numpy()
    return _close(got, want)


def check_softplus_threshold(fwd):
    """L = 1, N = 1, A = 0, B = C = u = 1: y = softplus(x) for x <= 20, x above."""
    xs = torch.tensor([-30.0, -1.0, 0.0, 3.5, 19.5, 20.0, 20.0001, 25.0, 60.0], dtype=F64)
    dim = xs.numel()
    u = torch.ones(1, dim, 1, dtype=F64)
    delta = xs[None, :, None].clone()
    A = torch.zeros(dim, 1, dtype=F64)
    one = torch.ones(dim, 1, dtype=F64)
    got = fwd(u, delta, A, one, one, delta_softplus=True)
    want = torch.where(xs <= 20.0, torch.from_numpy(np.logaddexp(0.0, xs.numpy())), xs)
    return _close(got.flatten(), want, rtol=1e-14, atol=1e-15)


def check_z_gate(fwd):
    """out(z) = out(no z) * z * sigmoid(z)."""
    x = _inputs(2, 4, 3, 20, seed=15)
    base = dict(D=x["D"], delta_bias=x["delta_bias"], delta_softplus=True)
    got = fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], z=x["z"], **base)
    y = fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **base)
    want = y.numpy() * x["z"].numpy() * expit(x["z"].numpy())
    return _close(got, want)


FORWARD_CHECKS = {
    "brute_force": check_brute_force,
    "A_zero_cumsum": check_A_zero_cumsum,
    "seqlen_one": check_seqlen_one,
    "iir_filter": check_iir_filter,
    "softplus_threshold": check_softplus_threshold,
    "z_gate": check_z_gate,
}


@pytest.mark.parametrize("check", sorted(FORWARD_CHECKS))
@pytest.mark.parametrize("oracle", sorted(ORACLES))
def test_forward_pin(oracle, check):
    assert FORWARD_CHECKS[check](ORACLES[oracle]), f"{oracle} oracle fails {check}"


# Plausible mistakes, each expressed as a wrong variant of the torch oracle.
def _flip(t):
    return None if t is None or t.dim() < 3 else t.flip(-1)


def _shift_right(t):
    out = torch.zeros_like(t)
    out[..., 1:] = t[..., :-1]
    return out


MUTANTS = {
    "dropped_D_term": lambda u, dl, A, B, C, D=None, **k: ref64(u, dl, A, B, C, None, **k),
    "A_sign_flipped": lambda u, dl, A, B, C, D=None, **k: ref64(u, dl, -A, B, C, D, **k),
    "B_C_swapped": lambda u, dl, A, B, C, D=None, **k: ref64(u, dl, A, C, B, D, **k),
    "softplus_ignored": lambda u, dl, A, B, C, D=None, delta_softplus=False, **k: ref64(u, dl, A, B, C, D, **k),
    "bias_ignored": lambda u, dl, A, B, C, D=None, delta_bias=None, **k: ref64(u, dl, A, B, C, D, **k),
    "time_reversed": lambda u, dl, A, B, C, D=None, z=None, **k: ref64(
        u.flip(-1), dl.flip(-1), A, _flip(B) if B.dim() >= 3 else B, _flip(C) if C.dim() >= 3 else C, D,
        z=_flip(z), **k).flip(-1),
    "input_one_step_late": lambda u, dl, A, B, C, D=None, **k: ref64(_shift_right(u), dl, A, B, C, D, **k)
    + (0 if D is None else (D[:, None] * (u - _shift_right(u)))),
    "gate_sigmoid_not_silu": lambda u, dl, A, B, C, D=None, z=None, **k: ref64(u, dl, A, B, C, D, **k)
    * (1 if z is None else torch.sigmoid(z)),
    "exp_of_A_only": lambda u, dl, A, B, C, D=None, **k: _exp_a_only(u, dl, A, B, C, D, **k),
}


def _exp_a_only(u, dl, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    """Mistake: decay exp(A) instead of exp(delta * A) (the state ignores delta's step size)."""
    Bt, dim, L = u.shape
    d = dl + (delta_bias[:, None] if delta_bias is not None else 0)
    if delta_softplus:
        d = F.softplus(d, threshold=20.0)
    Bx = B if B.dim() >= 3 else B[None, :, :, None].expand(Bt, dim, -1, L)
    Cx = C if C.dim() >= 3 else C[None, :, :, None].expand(Bt, dim, -1, L)
    Bx = Bx.repeat_interleave(dim // Bx.shape[1], 1)
    Cx = Cx.repeat_interleave(dim // Cx.shape[1], 1)
    h = torch.zeros(Bt, dim, A.shape[1], dtype=F64)
    ys = []
    for t in range(L):
        h = torch.exp(A)[None] * h + (d[:, :, t] * u[:, :, t])[..., None] * Bx[..., t]
        ys.append((h * Cx[..., t]).sum(-1))
    y = torch.stack(ys, -1)
    if D is not None:
        y = y + D[:, None] * u
    if z is not None:
        y = y * F.silu(z)
    return y


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_planted_mistakes_are_caught(mutant):
    caught = [name for name, chk in FORWARD_CHECKS.items() if not chk(MUTANTS[mutant])]
    assert caught, f"no forward check catches the planted mistake {mutant}"


# -------------------------------------------------------- structural checks --
@pytest.mark.parametrize("oracle", sorted(ORACLES))
def test_constant_BC_equals_broadcast(oracle):
    fwd = ORACLES[oracle]
    x = _inputs(2, 6, 4, 17, seed=21, var_B=False, var_C=False)
    Bt, dim, L = x["u"].shape
    Bv = x["B"][None, :, :, None].expand(Bt, dim, -1, L).contiguous()   # G = dim
    Cv = x["C"][None, :, :, None].expand(Bt, dim, -1, L).contiguous()
    args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    assert _close(fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args),
                  fwd(x["u"], x["delta"], x["A"], Bv, Cv, **args))


@pytest.mark.parametrize("oracle", sorted(ORACLES))
def test_groups_equal_per_channel_broadcast(oracle):
    fwd = ORACLES[oracle]
    x = _inputs(2, 8, 3, 15, seed=22, n_groups=2)
    Bx = x["B"].repeat_interleave(4, dim=1).contiguous()   # (Bt, dim, N, L): channel d uses group d // 4
    Cx = x["C"].repeat_interleave(4, dim=1).contiguous()
    args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    assert _close(fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args),
                  fwd(x["u"], x["delta"], x["A"], Bx, Cx, **args))


@pytest.mark.parametrize("oracle", sorted(ORACLES))
def test_causality_and_prefix(oracle):
    fwd = ORACLES[oracle]
    x = _inputs(1, 4, 5, 40, seed=23)
    args = dict(D=x["D"], delta_bias=x["delta_bias"], delta_softplus=True)
    full = fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], z=x["z"], **args)
    p = 17
    pre = fwd(x["u"][..., :p].contiguous(), x["delta"][..., :p].contiguous(), x["A"],
              x["B"][..., :p].contiguous(), x["C"][..., :p].contiguous(), z=x["z"][..., :p].contiguous(), **args)
    assert _close(full[..., :p], pre)
    u2 = x["u"].clone()
    u2[..., p] += 1.0
    pert = fwd(u2, x["delta"], x["A"], x["B"], x["C"], z=x["z"], **args)
    assert _close(pert[..., :p], full[..., :p], rtol=0, atol=0)
    assert not _close(pert[..., p], full[..., p])


@pytest.mark.parametrize("oracle", sorted(ORACLES))
def test_linear_in_u(oracle):
    fwd = ORACLES[oracle]
    x = _inputs(2, 3, 4, 25, seed=24, has_z=False)
    g = torch.Generator().manual_seed(5)
    u2 = torch.randn(x["u"].shape, generator=g, dtype=F64)
    args = dict(D=x["D"], delta_bias=x["delta_bias"], delta_softplus=True)
    f = lambda u: fwd(u, x["delta"], x["A"], x["B"], x["C"], **args)
    assert _close(f(2.0 * x["u"] - 3.0 * u2), 2.0 * f(x["u"]) - 3.0 * f(u2), rtol=1e-9, atol=1e-10)


def test_last_state_agrees():
    x = _inputs(2, 4, 3, 23, seed=25, n_groups=2)
    args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True)
    out_t, last_t = selective_scan_ref(x["u"], x["delta"], x["A"], x["B"], x["C"], return_last_state=True,
                                       compute_dtype=F64, **args)
    out_c, last_c = c_oracle.fwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args)
    assert _close(out_t, out_c) and _close(last_t, last_c)
    # the last state at L = 1 is delta u B
    x1 = _inputs(1, 3, 4, 1, seed=26, has_z=False, has_delta_bias=False)
    _, last = c_oracle.fwd(x1["u"], x1["delta"], x1["A"], x1["B"], x1["C"], delta_softplus=False)
    want = (x1["delta"] * x1["u"])[:, :, 0, None] * x1["B"][:, 0, None, :, 0]   # (Bt, D, N)
    assert _close(last, want)


# ----------------------------------------------------------------- gradients --
GRAD_NAMES = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")

# (batch, dim, dstate, seqlen, make_inputs keywords, softplus)
GRAD_CASES = [
    (2, 4, 3, 12, {"n_groups": 2}, True),
    (1, 3, 2, 9, {"var_B": False}, True),
    (1, 3, 2, 9, {"var_C": False, "has_z": False}, False),
    (2, 2, 3, 7, {"var_B": False, "var_C": False, "has_D": False, "has_delta_bias": False}, True),
]


def _autograd(x, softplus):
    ins = {k: (x[k].clone().requires_grad_(True) if x[k] is not None else None) for k in GRAD_NAMES}
    out = ref64(ins["u"], ins["delta"], ins["A"], ins["B"], ins["C"], ins["D"], z=ins["z"],
                delta_bias=ins["delta_bias"], delta_softplus=softplus)
    out.backward(x["dout"])
    return {k: ins[k].grad for k in GRAD_NAMES if ins[k] is not None}


@pytest.mark.parametrize("case", range(len(GRAD_CASES)))
def test_gradcheck_torch_oracle(case):
    b, d, n, l, kw, sp = GRAD_CASES[case]
    x = _inputs(b, d, n, l, seed=30 + case, positive_delta=not sp, **kw)
    keys = [k for k in GRAD_NAMES if x[k] is not None]

    def f(*ts):
        a = dict(zip(keys, ts))
        return ref64(a["u"], a["delta"], a["A"], a["B"], a["C"], a.get("D"), z=a.get("z"),
                     delta_bias=a.get("delta_bias"), delta_softplus=sp)
    ts = tuple(x[k].clone().requires_grad_(True) for k in keys)
    assert torch.autograd.gradcheck(f, ts, eps=1e-6, atol=1e-7, rtol=1e-5)


@pytest.mark.parametrize("case", range(len(GRAD_CASES)))
def test_c_backward_equals_autograd(case):
    b, d, n, l, kw, sp = GRAD_CASES[case]
    x = _inputs(b, d, n, l, seed=40 + case, positive_delta=not sp, **kw)
    want = _autograd(x, sp)
    got = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
                       delta_bias=x["delta_bias"], delta_softplus=sp, dout=x["dout"])
    names = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
             "delta_bias": "ddelta_bias"}
    for k, g in want.items():
        assert _close(got[names[k]], g, rtol=1e-9, atol=1e-11), k


@pytest.mark.parametrize("case", range(len(GRAD_CASES)))
def test_c_backward_finite_differences(case):
    """Central differences of sum(dout * out) through the C forward, without torch autograd."""
    b, d, n, l, kw, sp = GRAD_CASES[case]
    x = _inputs(b, d, n, l, seed=50 + case, positive_delta=not sp, **kw)
    grads = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
                         delta_bias=x["delta_bias"], delta_softplus=sp, dout=x["dout"])
    names = {"u": "du", "delta": "ddelta", "A": "dA", "B": "dB", "C": "dC", "D": "dD", "z": "dz",
             "delta_bias": "ddelta_bias"}
    rng = np.random.default_rng(case)
    eps = 1e-6

    def loss(vals):
        out = c64(vals["u"], vals["delta"], vals["A"], vals["B"], vals["C"], D=vals["D"], z=vals["z"],
                  delta_bias=vals["delta_bias"], delta_softplus=sp)
        return float((out * x["dout"]).sum())

    for k in GRAD_NAMES:
        if x[k] is None:
            continue
        for flat in rng.choice(x[k].numel(), size=min(4, x[k].numel()), replace=False):
            vals = dict(x)
            plus, minus = x[k].clone(), x[k].clone()
            plus.view(-1)[flat] += eps
            minus.view(-1)[flat] -= eps
            vals[k] = plus
            lp = loss(vals)
            vals[k] = minus
            lm = loss(vals)
            fd = (lp - lm) / (2 * eps)
            an = float(grads[names[k]].reshape(-1)[flat])
            assert abs(fd - an) <= 1e-6 + 1e-5 * abs(an), f"{k}[{flat}]: fd {fd} vs analytic {an}"


def test_gradient_identities():
    """dD = sum dy u, ddelta_bias = sum ddelta, dz = dout y silu'(z), dy = dout silu(z)."""
    x = _inputs(2, 5, 4, 19, seed=60)
    g = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
                     delta_bias=x["delta_bias"], delta_softplus=True, dout=x["dout"])
    z = x["z"].numpy()
    sg = expit(z)
    dy = x["dout"].numpy() * z * sg
    assert _close(g["dD"], (dy * x["u"].numpy()).sum(axis=(0, 2)))
    assert _close(g["ddelta_bias"], g["ddelta"].sum(dim=(0, 2)))
    y = c64(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], delta_bias=x["delta_bias"],
            delta_softplus=True).numpy()
    assert _close(g["dz"], x["dout"].numpy() * y * sg * (1 + z * (1 - sg)))
    # softplus' = sigmoid: ddelta with softplus = ddelta' (no softplus, delta' given) * sigmoid(delta + bias)
    pre = x["delta"] + x["delta_bias"][:, None]
    g_lin = c_oracle.bwd(x["u"], F.softplus(pre, threshold=20.0), x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
                         delta_softplus=False, dout=x["dout"])
    assert _close(g["ddelta"], g_lin["ddelta"] * torch.sigmoid(pre))


def test_constant_B_gradient_is_broadcast_sum():
    x = _inputs(2, 3, 2, 11, seed=61, var_B=False)
    Bt, dim, L = x["u"].shape
    Bv = x["B"][None, :, :, None].expand(Bt, dim, -1, L).contiguous()
    Cx = x["C"].repeat_interleave(dim, dim=1).contiguous()   # G = dim for the variable-B run
    args = dict(D=x["D"], z=x["z"], delta_bias=x["delta_bias"], delta_softplus=True, dout=x["dout"])
    gc = c_oracle.bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], **args)
    gv = c_oracle.bwd(x["u"], x["delta"], x["A"], Bv, Cx, **args)
    assert _close(gc["dB"], gv["dB"].sum(dim=(0, 3)))
    assert _close(gc["dC"], gv["dC"].reshape(Bt, dim, -1, L).sum(1, keepdim=True))


# ------------------------------------------------------------------ fixtures --
def test_golden_fixtures():
    from tests.golden import make_golden as mg
    data = np.load(mg.PATH)
    for name, (_, _, _, _, _, _, softplus, grads) in mg.CASES.items():
        x = mg.case_inputs(name)
        assert str(data[f"{name}/inputs_sha256"]) == mg.inputs_digest(x), \
            f"{name}: the seeded input generator changed; regenerate only if that change is intended"
        got = mg.compute(name)
        tol = (1e-6, 1e-6) if not grads else (1e-12, 1e-12)
        for k, v in got.items():
            assert _close(v, data[f"{name}/{k}"], *tol), f"{name}/{k}"
        # the PyTorch oracle agrees with the stored C-oracle outputs too
        xd = {k: (t.double() if t is not None else None) for k, t in x.items()}
        out = ref64(xd["u"], xd["delta"], xd["A"], xd["B"], xd["C"], xd["D"], z=xd["z"],
                    delta_bias=xd["delta_bias"], delta_softplus=softplus)
        assert _close(out, data[f"{name}/out"], *(1e-6, 1e-6) if not grads else (1e-10, 1e-12)), name
