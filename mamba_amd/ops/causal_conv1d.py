"""Causal depthwise conv1d (+ SiLU) on the HIP library.

The reference runs this step of the Mamba block in PyTorch
(modules/mamba_simple.py:40-47 builds nn.Conv1d(dim, dim, width,
groups=dim, padding=width - 1); :100-101 cuts the output to seqlen and
applies SiLU):

    out[b, d, t] = act(bias[d] + sum_k weight[d, k] * x[b, d, t - (width - 1) + k])

``causal_conv1d_fn(x, weight, bias=None, activation=None)`` takes x as
(batch, dim, seqlen) with unit stride along seqlen (batch and channel
strides are free, so x may be a channel slice of a packed xz tensor),
weight as (dim, width) or nn.Conv1d's (dim, 1, width), width 1..4, and
returns out in x's dtype.  Gradients: dx in x's dtype, dweight / dbias in
the parameters' dtypes (accumulated in fp32).  Under
``torch.use_deterministic_algorithms(True)`` the backward sums dweight and
dbias in a fixed order (per-workgroup partials added per channel by a second
launch), so they come out with the same bits on every run; otherwise each
workgroup adds its partial with fp32 atomics.
"""
import ctypes

import torch

from .. import _native as nat
from ..selective_scan import _ITYPES, _ptr, _require, _stream


def _weight2d(weight, dim):
    w = weight.reshape(weight.shape[0], weight.shape[-1]) if weight.dim() == 3 else weight
    _require(w.dim() == 2 and w.shape[0] == dim, f"weight must be (dim, width), got {tuple(weight.shape)}")
    return w


def _fill(x, weight32, bias32, silu, out):
    _require(x.dim() == 3, f"x must be (batch, dim, seqlen), got {tuple(x.shape)}")
    _require(x.device.type == "cuda", "tensors must be on a ROCm GPU device (no CPU path)")
    _require(x.dtype in _ITYPES, f"unsupported dtype {x.dtype}")
    _require(x.shape[-1] <= 1 or x.stride(-1) == 1, "x must have unit stride along seqlen")
    batch, dim, seqlen = x.shape
    a = nat.Conv1dArgs()
    a.batch, a.dim, a.seqlen, a.width = batch, dim, seqlen, weight32.shape[1]
    a.itype = _ITYPES[x.dtype]
    a.has_bias, a.silu = int(bias32 is not None), int(bool(silu))
    a.x_batch_stride, a.x_dim_stride = x.stride(0), x.stride(1)
    if out is not None:
        a.out_batch_stride, a.out_dim_stride = out.stride(0), out.stride(1)
    a.w_dim_stride, a.w_width_stride = weight32.stride(0), weight32.stride(1)
    a.x, a.weight, a.bias, a.out = _ptr(x), _ptr(weight32), _ptr(bias32), _ptr(out)
    return a


def _params32(weight, bias, dim, device):
    w = _weight2d(weight, dim).to(device=device, dtype=torch.float32)
    b = bias.to(device=device, dtype=torch.float32).contiguous() if bias is not None else None
    if b is not None:
        _require(b.shape == (dim,), f"bias must be ({dim},), got {tuple(bias.shape)}")
    return w, b


def causal_conv1d_fwd(x, weight, bias=None, silu=False, out=None):
    """Forward into ``out`` (allocated if None, x's dtype and shape)."""
    lib = nat.load()
    w, b = _params32(weight, bias, x.shape[1], x.device)
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _require(out.shape == x.shape and out.dtype == x.dtype and (out.shape[-1] <= 1 or out.stride(-1) == 1),
             "out must match x in shape and dtype, with unit stride along seqlen")
    a = _fill(x, w, b, silu, out)
    with torch.cuda.device(x.device):
        nat.check(lib.ss_conv1d_fwd(ctypes.byref(a), _stream(x.device)), "causal_conv1d_fwd")
    return out


def causal_conv1d_bwd(x, weight, bias, dout, silu=False, dx=None, deterministic=None):
    """Returns (dx, dweight fp32 (dim, width), dbias fp32 or None).
    ``deterministic``: sum dweight / dbias in a fixed order; None follows
    ``torch.use_deterministic_algorithms``."""
    lib = nat.load()
    w, b = _params32(weight, bias, x.shape[1], x.device)
    _require(dout.shape == x.shape and dout.dtype == x.dtype, "dout must match x in shape and dtype")
    if dout.shape[-1] > 1 and dout.stride(-1) != 1:
        dout = dout.contiguous()
    if dx is None:
        dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dw = torch.zeros(w.shape, dtype=torch.float32, device=x.device)
    db = torch.zeros(b.shape, dtype=torch.float32, device=x.device) if b is not None else None
    g = nat.Conv1dBwdArgs()
    g.f = _fill(x, w, b, silu, None)
    g.dout_batch_stride, g.dout_dim_stride = dout.stride(0), dout.stride(1)
    g.dx_batch_stride, g.dx_dim_stride = dx.stride(0), dx.stride(1)
    g.dout, g.dx, g.dweight, g.dbias = _ptr(dout), _ptr(dx), _ptr(dw), _ptr(db)
    if deterministic is None:
        deterministic = torch.are_deterministic_algorithms_enabled()
    ws = None
    if deterministic:
        nbytes = lib.ss_conv1d_bwd_workspace_bytes(ctypes.byref(g))
        _require(nbytes >= 0, "invalid conv1d sizes")
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=x.device)
        g.workspace, g.workspace_bytes = _ptr(ws), ws.numel() * 4
    with torch.cuda.device(x.device):
        nat.check(lib.ss_conv1d_bwd(ctypes.byref(g), _stream(x.device)), "causal_conv1d_bwd")
    del ws                  # the caching allocator keeps it until the stream's work is done
    return dx, dw, db


def _silu_flag(activation):
    _require(activation in (None, "silu", "swish"), f"activation must be None, 'silu' or 'swish', got {activation!r}")
    return activation in ("silu", "swish")


class CausalConv1dFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias=None, activation=None):
        silu = _silu_flag(activation)
        if x.shape[-1] > 1 and x.stride(-1) != 1:
            x = x.contiguous()
        out = causal_conv1d_fwd(x, weight, bias, silu)
        ctx.save_for_backward(x, weight, bias)
        ctx.silu = silu
        return out

    @staticmethod
    def backward(ctx, dout):
        x, weight, bias = ctx.saved_tensors
        dx, dw, db = causal_conv1d_bwd(x, weight, bias, dout, ctx.silu)
        dw = dw.reshape(weight.shape).to(weight.dtype)
        db = db.to(bias.dtype) if bias is not None else None
        return dx, dw, db, None


def causal_conv1d_fn(x, weight, bias=None, activation=None):
    """Causal depthwise conv1d with optional SiLU; see the module docstring."""
    return CausalConv1dFn.apply(x, weight, bias, activation)


def causal_conv1d_update(x, conv_state, weight, bias=None, activation=None, out=None):
    """One decode step of the causal conv: conv_state (batch, dim, width) holds the
    last width inputs; it is shifted by one with x (batch, dim) appended, in place,
    and out[b, d] = act(bias[d] + sum_k weight[d, k] * conv_state[b, d, k]) is
    returned in x's dtype.  Equals step t of causal_conv1d_fn when conv_state
    held inputs t - width .. t - 1 (zeros before the sequence start)."""
    lib = nat.load()
    silu = _silu_flag(activation)
    _require(x.dim() == 2 and x.device.type == "cuda", "x must be (batch, dim) on a ROCm GPU device (no CPU path)")
    _require(x.dtype in _ITYPES, f"unsupported dtype {x.dtype}")
    batch, dim = x.shape
    w, b = _params32(weight, bias, dim, x.device)
    _require(conv_state.shape == (batch, dim, w.shape[1]) and conv_state.dtype == x.dtype
             and conv_state.device == x.device,
             f"conv_state must be ({batch}, {dim}, {w.shape[1]}) of x's dtype, got {tuple(conv_state.shape)}")
    if out is None:
        out = torch.empty(batch, dim, dtype=x.dtype, device=x.device)
    a = nat.Conv1dUpdateArgs()
    a.batch, a.dim, a.width = batch, dim, w.shape[1]
    a.itype, a.has_bias, a.silu = _ITYPES[x.dtype], int(b is not None), int(silu)
    a.x_batch_stride, a.x_dim_stride = x.stride(0), x.stride(1)
    a.out_batch_stride, a.out_dim_stride = out.stride(0), out.stride(1)
    a.state_batch_stride, a.state_dim_stride, a.state_width_stride = conv_state.stride()
    a.w_dim_stride, a.w_width_stride = w.stride(0), w.stride(1)
    a.x, a.conv_state, a.weight, a.bias, a.out = _ptr(x), _ptr(conv_state), _ptr(w), _ptr(b), _ptr(out)
    with torch.cuda.device(x.device):
        nat.check(lib.ss_conv1d_update(ctypes.byref(a), _stream(x.device)), "causal_conv1d_update")
    return out
