"""ctypes wrapper around the float64 C restatement (oracle/ss_oracle.c).

Test infrastructure only.  ``build()`` compiles the library with the
Makefile beside this file; the wrappers take and return torch tensors and
do all arithmetic in float64.  ``scan`` is the same forward / backward as an
autograd function, so the block and model oracles can differentiate through
long sequences without selective_scan_ref's per-step autograd graph.
"""
import ctypes
import os
import subprocess

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libss_oracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "libss_oracle.so"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        i64, ci, p = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
        lib.ss_oracle_fwd.argtypes = [i64] * 5 + [ci] * 3 + [p] * 10
        lib.ss_oracle_fwd.restype = ci
        lib.ss_oracle_bwd.argtypes = [i64] * 5 + [ci] * 3 + [p] * 17
        lib.ss_oracle_bwd.restype = ci
        _lib = lib
    return _lib


def _d(t):
    return None if t is None else t.detach().to("cpu", torch.float64).contiguous()


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _dims(u, A, B, C):
    Bt, D, L = u.shape
    N = A.shape[1]
    var_B, var_C = B.dim() >= 3, C.dim() >= 3
    G = B.shape[1] if var_B else (C.shape[1] if var_C else 1)
    return Bt, D, L, N, G, var_B, var_C


def fwd(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False):
    """Returns (out, last_state) in float64."""
    Bt, Dd, L, N, G, var_B, var_C = _dims(u, A, B, C)
    args = [_d(x) for x in (u, delta, A, B, C, D, delta_bias, z)]
    out = torch.empty(Bt, Dd, L, dtype=torch.float64)
    last = torch.empty(Bt, Dd, N, dtype=torch.float64)
    rc = _load().ss_oracle_fwd(Bt, Dd, L, N, G, int(var_B), int(var_C), int(delta_softplus),
                               *[_ptr(a) for a in args], _ptr(out), _ptr(last))
    if rc != 0:
        raise ValueError("ss_oracle_fwd rejected the shapes")
    return out, last


def bwd(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False, dout=None):
    """Returns a dict of float64 gradients: du, ddelta, dA, dB, dC, dD, ddelta_bias, dz."""
    Bt, Dd, L, N, G, var_B, var_C = _dims(u, A, B, C)
    args = [_d(x) for x in (u, delta, A, B, C, D, delta_bias, z, dout)]
    f64 = dict(dtype=torch.float64)
    du = torch.empty(Bt, Dd, L, **f64)
    dd = torch.empty(Bt, Dd, L, **f64)
    dA = torch.empty(Dd, N, **f64)
    dB = torch.empty(tuple(B.shape), **f64)
    dC = torch.empty(tuple(C.shape), **f64)
    dD = torch.empty(Dd, **f64) if D is not None else None
    db = torch.empty(Dd, **f64) if delta_bias is not None else None
    dz = torch.empty(Bt, Dd, L, **f64) if z is not None else None
    rc = _load().ss_oracle_bwd(Bt, Dd, L, N, G, int(var_B), int(var_C), int(delta_softplus),
                               *[_ptr(a) for a in args],
                               *[_ptr(x) for x in (du, dd, dA, dB, dC, dD, db, dz)])
    if rc != 0:
        raise ValueError("ss_oracle_bwd rejected the shapes")
    return dict(du=du, ddelta=dd, dA=dA, dB=dB, dC=dC, dD=dD, ddelta_bias=db, dz=dz)


class CScanFn(torch.autograd.Function):
    """selective_scan (forward_kernel.cu:174-310, backward_kernel.cu:276-585,
    z gate of modules/mamba_simple.py:143-146) with both directions in the
    float64 C restatement; the output comes back in u's dtype."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, z, delta_bias, delta_softplus):
        out, _ = fwd(u, delta, A, B, C, D, z=z, delta_bias=delta_bias, delta_softplus=delta_softplus)
        ctx.save_for_backward(u, delta, A, B, C, D, z, delta_bias)
        ctx.delta_softplus = delta_softplus
        return out.to(u.dtype)

    @staticmethod
    def backward(ctx, dout):
        u, delta, A, B, C, D, z, bias = ctx.saved_tensors
        g = bwd(u, delta, A, B, C, D, z=z, delta_bias=bias, delta_softplus=ctx.delta_softplus, dout=dout)

        def cast(x, ref):
            return None if x is None or ref is None else x.to(ref.dtype)
        return (cast(g["du"], u), cast(g["ddelta"], delta), cast(g["dA"], A), cast(g["dB"], B),
                cast(g["dC"], C), cast(g["dD"], D), cast(g["dz"], z), cast(g["ddelta_bias"], bias), None)


def scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, delta_softplus=False, compute_dtype=None):
    """selective_scan_ref's signature on the C restatement (compute_dtype is
    ignored: the arithmetic is float64); differentiable."""
    return CScanFn.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus)
