"""One decode step of the selective scan on the HIP library.

``selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None,
dt_softplus=False)`` advances the scan of forward_kernel.cu:216-293 by one
token from a state kept between tokens (the reference has no decode path:
CausalLM.generate is a stub, models/causal_lm.py:61-62):

    dt' = softplus(dt + dt_bias)
    state[b, d, n] <- exp(dt' A[d, n]) state[b, d, n] + dt' x[b, d] B[b, g, n]   (in place, fp32)
    out[b, d] = sum_n C[b, g, n] state[b, d, n] + D[d] x[b, d], times silu(z[b, d])

state: fp32 (batch, dim, dstate); x, dt, z: (batch, dim); A: (dim, dstate);
B, C: (batch, dstate) or (batch, n_groups, dstate), in x's dtype (any
strides); D, dt_bias: (dim,).  Returns out (batch, dim) in x's dtype.

dt may also be a pair (dt_low, dt_weight): the block's delta projection
dt = dt_low @ dt_weight.T (modules/mamba_simple.py:118-119), with dt_low
(batch, rank) and dt_weight (dim, rank) in x's dtype, summed in fp32 inside
the kernel, so a decode step needs no launch for that product.
"""
import ctypes

import torch

from .. import _native as nat
from ..selective_scan import _ITYPES, _ptr, _stream


def _require(cond, msg):
    if not cond:
        raise ValueError(f"selective_state_update: {msg}")


def selective_state_update(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False, out=None):
    lib = nat.load()
    _require(x.dim() == 2 and x.device.type == "cuda", "x must be (batch, dim) on a ROCm GPU device (no CPU path)")
    _require(x.dtype in _ITYPES, f"unsupported dtype {x.dtype}")
    batch, dim = x.shape
    dev = x.device
    _require(state.dim() == 3 and state.shape[:2] == (batch, dim) and state.dtype == torch.float32
             and state.device == dev, f"state must be fp32 ({batch}, {dim}, dstate)")
    dstate = state.shape[2]
    low = isinstance(dt, (tuple, list))
    if low:
        dt_low, dt_w = dt
        _require(dt_low.dim() == 2 and dt_low.shape[0] == batch and dt_low.dtype == x.dtype
                 and dt_low.device == dev, "dt_low must be (batch, rank) in x's dtype")
        _require(dt_w.shape == (dim, dt_low.shape[1]) and dt_w.dtype == x.dtype and dt_w.device == dev,
                 "dt_weight must be (dim, rank) in x's dtype")
    else:
        _require(dt.shape == x.shape and dt.dtype == x.dtype, "dt must match x in shape and dtype")
    _require(A.shape == (dim, dstate), f"A must be ({dim}, {dstate})")
    A32 = A.to(device=dev, dtype=torch.float32)
    if B.dim() == 2:
        B = B.unsqueeze(1)
    if C.dim() == 2:
        C = C.unsqueeze(1)
    _require(B.dim() == 3 and B.shape[0] == batch and B.shape[2] == dstate and B.dtype == x.dtype,
             "B must be (batch, [n_groups,] dstate) in x's dtype")
    _require(C.shape == B.shape and C.dtype == x.dtype, "C must match B")
    n_groups = B.shape[1]
    _require(dim % n_groups == 0, f"dim {dim} is not a multiple of n_groups {n_groups}")
    D32 = D.to(device=dev, dtype=torch.float32).contiguous() if D is not None else None
    db32 = dt_bias.to(device=dev, dtype=torch.float32).contiguous() if dt_bias is not None else None
    for name, t in (("D", D32), ("dt_bias", db32)):
        _require(t is None or t.shape == (dim,), f"{name} must be ({dim},)")
    _require(z is None or (z.shape == x.shape and z.dtype == x.dtype), "z must match x")
    if out is None:
        out = torch.empty(batch, dim, dtype=x.dtype, device=dev)
    a = nat.StateUpdateArgs()
    a.batch, a.dim, a.dstate, a.n_groups = batch, dim, dstate, n_groups
    a.itype = _ITYPES[x.dtype]
    a.has_D, a.has_z, a.has_delta_bias, a.delta_softplus = (int(D32 is not None), int(z is not None),
                                                            int(db32 is not None), int(bool(dt_softplus)))
    a.state_batch_stride, a.state_dim_stride, a.state_dstate_stride = state.stride()
    a.x_batch_stride, a.x_dim_stride = x.stride()
    if low:
        a.delta_rank = dt_low.shape[1]
        a.delta_low_batch_stride, a.delta_low_rank_stride = dt_low.stride()
        a.delta_weight_dim_stride, a.delta_weight_rank_stride = dt_w.stride()
        a.delta_low, a.delta_weight = _ptr(dt_low), _ptr(dt_w)
    else:
        a.delta_batch_stride, a.delta_dim_stride = dt.stride()
    if z is not None:
        a.z_batch_stride, a.z_dim_stride = z.stride()
    a.out_batch_stride, a.out_dim_stride = out.stride()
    a.A_dim_stride, a.A_dstate_stride = A32.stride()
    a.B_batch_stride, a.B_group_stride, a.B_dstate_stride = B.stride()
    a.C_batch_stride, a.C_group_stride, a.C_dstate_stride = C.stride()
    a.state, a.x, a.A, a.B, a.C = _ptr(state), _ptr(x), _ptr(A32), _ptr(B), _ptr(C)
    a.delta = None if low else _ptr(dt)
    a.D, a.z, a.delta_bias, a.out = _ptr(D32), _ptr(z), _ptr(db32), _ptr(out)
    with torch.cuda.device(dev):
        nat.check(lib.ss_state_update(ctypes.byref(a), _stream(dev)), "selective_state_update")
    return out
