"""RMSNorm (+ residual add) on the HIP library.

Replaces the reference's RMSNorm.forward (modules/rms_norm.py:19,29-31) and,
fused into the same pass, the residual add that ends each block
(models/causal_lm.py:31-35):

    s   = x + residual            (rounded to x's dtype; s = x without residual)
    out = s * rsqrt(mean(s**2, -1) + eps) * (1 + weight)    (fp32, rounded to x's dtype)

``rms_norm_fn(x, weight, residual=None, eps=1e-6, prenorm=False)`` returns
out, or (out, s) when ``prenorm`` (s is the residual stream that the next
block adds to).  x and residual share shape and dtype (fp32, bf16 or fp16);
weight is (dim,) of any float dtype (read as fp32 unless it is x's dtype).
Gradients flow to x, residual and weight; the weight gradient is summed over
rows in a fixed order, so it has the same bits on every run.
"""
import ctypes

import torch

from .. import _native as nat
from ..selective_scan import _ITYPES, _ptr, _stream


def _require(cond, msg):
    if not cond:
        raise ValueError(f"rms_norm: {msg}")


def _rows(t, dim):
    """(rows, dim) view of t with unit column stride (a copy only when no such view exists)."""
    if dim > 1 and t.stride(-1) != 1:
        t = t.contiguous()
    v = t.reshape(-1, dim)
    if dim > 1 and v.stride(1) != 1:
        v = v.contiguous()
    return v


def _weight(weight, x):
    _require(weight.dim() == 1 and weight.shape[0] == x.shape[-1],
             f"weight must be ({x.shape[-1]},), got {tuple(weight.shape)}")
    _require(weight.device == x.device, f"weight is on {weight.device}, x on {x.device}")
    w = weight if weight.dtype in (x.dtype, torch.float32) else weight.float()
    return w.contiguous()


def _fwd_args(x2, r2, w, out, rout, rstd, eps):
    a = nat.RmsNormArgs()
    a.rows, a.dim = x2.shape
    a.dtype, a.w_dtype = _ITYPES[x2.dtype], _ITYPES[w.dtype]
    a.eps = float(eps)
    a.x_row_stride, a.out_row_stride = x2.stride(0), out.stride(0)
    if r2 is not None:
        a.residual_row_stride, a.residual_out_row_stride = r2.stride(0), rout.stride(0)
    a.x, a.residual, a.weight = _ptr(x2), _ptr(r2), _ptr(w)
    a.out, a.residual_out, a.rstd = _ptr(out), _ptr(rout), _ptr(rstd)
    return a


def rms_norm_fwd(x, weight, residual=None, eps=1e-6, want_rstd=False, want_s=True):
    """Forward without autograd: returns (out, s or None, rstd or None), all (rows, dim)-shaped.

    s (x + residual) is written only when residual is given and want_s."""
    lib = nat.load()
    _require(x.device.type == "cuda", "tensors must be on a ROCm GPU device (no CPU path)")
    _require(x.dtype in _ITYPES, f"unsupported dtype {x.dtype}")
    _require(x.dim() >= 1, "x must have at least one dimension")
    dim = x.shape[-1]
    w = _weight(weight, x)
    x2 = _rows(x, dim)
    r2 = None
    if residual is not None:
        _require(residual.shape == x.shape and residual.dtype == x.dtype and residual.device == x.device,
                 "residual must match x in shape, dtype and device")
        r2 = _rows(residual, dim)
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    rout = torch.empty_like(out) if r2 is not None and want_s else None
    rstd = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device) if want_rstd else None
    a = _fwd_args(x2, r2, w, out, rout, rstd, eps)
    with torch.cuda.device(x.device):
        nat.check(lib.ss_rmsnorm_fwd(ctypes.byref(a), _stream(x.device)), "rms_norm forward")
    return out, rout, rstd


def rms_norm_bwd(s, weight, rstd, dout, dresidual_out=None):
    """Backward without autograd: returns (ds, dweight); s, dout, dresidual_out are (rows, dim)."""
    lib = nat.load()
    dim = s.shape[-1]
    w = _weight(weight, s)
    s2 = _rows(s, dim)
    dy = _rows(dout.to(s.dtype), dim)
    dr = _rows(dresidual_out.to(s.dtype), dim) if dresidual_out is not None else None
    rows = s2.shape[0]
    _require(dy.shape == s2.shape and (dr is None or dr.shape == s2.shape), "dout must match s")
    _require(rstd.dtype == torch.float32 and rstd.shape == (rows,) and rstd.is_contiguous(),
             "rstd must be fp32 (rows,) contiguous")
    dx = torch.empty(s2.shape, dtype=s.dtype, device=s.device)
    dw = torch.empty(dim, dtype=w.dtype, device=s.device)
    nbytes = int(lib.ss_rmsnorm_bwd_workspace_bytes(rows, dim))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=s.device)
    g = nat.RmsNormBwdArgs()
    g.rows, g.dim = rows, dim
    g.dtype, g.w_dtype = _ITYPES[s.dtype], _ITYPES[w.dtype]
    g.s_row_stride, g.dout_row_stride, g.dx_row_stride = s2.stride(0), dy.stride(0), dx.stride(0)
    if dr is not None:
        g.dresidual_out_row_stride = dr.stride(0)
    g.s, g.weight, g.rstd, g.dout, g.dresidual_out = _ptr(s2), _ptr(w), _ptr(rstd), _ptr(dy), _ptr(dr)
    g.dx, g.dweight, g.workspace, g.workspace_bytes = _ptr(dx), _ptr(dw), _ptr(ws), nbytes
    with torch.cuda.device(s.device):
        nat.check(lib.ss_rmsnorm_bwd(ctypes.byref(g), _stream(s.device)), "rms_norm backward")
    return dx, dw


def prepare_rms_norm_fwd(x, weight, residual, eps, out, residual_out, rstd):
    """Checks and packs the forward arguments once (x, residual, out, residual_out: (rows, dim)
    with unit column stride; weight as for rms_norm_fn; rstd fp32 (rows,) or None) and
    returns a callable that only makes the C call, on the stream current now."""
    lib = nat.load()
    _require(x.device.type == "cuda" and x.dim() == 2 and x.dtype in _ITYPES, "x must be a (rows, dim) GPU tensor")
    w = _weight(weight, x)
    for t in (residual, out, residual_out):
        _require(t is None or (t.shape == x.shape and t.dtype == x.dtype and (x.shape[1] <= 1 or t.stride(1) == 1)),
                 "residual / out / residual_out must match x, with unit column stride")
    a = _fwd_args(x, residual, w, out, residual_out, rstd, eps)
    stream = _stream(x.device)
    keep = (x, residual, w, out, residual_out, rstd)

    def launch():
        nat.check(lib.ss_rmsnorm_fwd(ctypes.byref(a), stream), "rms_norm forward")
        return keep
    return launch


def prepare_rms_norm_bwd(s, weight, rstd, dout, dresidual_out, dx, dweight, workspace):
    """As prepare_rms_norm_fwd, for the backward (all row tensors (rows, dim), unit column
    stride; dweight (dim,) of weight's dtype or fp32; workspace a uint8 tensor of at least
    ss_rmsnorm_bwd_workspace_bytes(rows, dim) bytes)."""
    lib = nat.load()
    w = _weight(weight, s)
    rows, dim = s.shape
    _require(dweight.dtype == w.dtype and dweight.shape == (dim,), "dweight must be (dim,) of the weight's dtype")
    g = nat.RmsNormBwdArgs()
    g.rows, g.dim = rows, dim
    g.dtype, g.w_dtype = _ITYPES[s.dtype], _ITYPES[w.dtype]
    g.s_row_stride, g.dout_row_stride, g.dx_row_stride = s.stride(0), dout.stride(0), dx.stride(0)
    if dresidual_out is not None:
        g.dresidual_out_row_stride = dresidual_out.stride(0)
    g.s, g.weight, g.rstd, g.dout, g.dresidual_out = _ptr(s), _ptr(w), _ptr(rstd), _ptr(dout), _ptr(dresidual_out)
    g.dx, g.dweight, g.workspace, g.workspace_bytes = _ptr(dx), _ptr(dweight), _ptr(workspace), workspace.numel()
    stream = _stream(s.device)
    keep = (s, w, rstd, dout, dresidual_out, dx, dweight, workspace)

    def launch():
        nat.check(lib.ss_rmsnorm_bwd(ctypes.byref(g), stream), "rms_norm backward")
        return keep
    return launch


class RMSNormFn(torch.autograd.Function):
    """Autograd of rms_norm_fn; outputs (out,) or (out, s) when prenorm."""

    @staticmethod
    def forward(ctx, x, weight, residual, eps, prenorm):
        want_rstd = any(ctx.needs_input_grad[:3])
        out, rout, rstd = rms_norm_fwd(x, weight, residual, eps, want_rstd, want_s=prenorm or want_rstd)
        s = rout if residual is not None else x
        if want_rstd:
            ctx.save_for_backward(_rows(s, x.shape[-1]) if residual is None else s, weight, rstd)
        ctx.shape = x.shape
        ctx.has_residual = residual is not None
        ctx.set_materialize_grads(False)
        out = out.view(x.shape)
        if prenorm:
            return out, rout.view(x.shape)
        return out

    @staticmethod
    def backward(ctx, dout, dres=None):
        s, weight, rstd = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros(s.shape, dtype=s.dtype, device=s.device)
        dx, dw = rms_norm_bwd(s, weight, rstd, dout.reshape(s.shape),
                              dres.reshape(s.shape) if dres is not None else None)
        dx = dx.view(ctx.shape)
        dweight = dw.to(weight.dtype) if ctx.needs_input_grad[1] else None
        dres_in = dx if ctx.has_residual and ctx.needs_input_grad[2] else None
        return (dx if ctx.needs_input_grad[0] else None), dweight, dres_in, None, None


def rms_norm_fn(x, weight, residual=None, eps=1e-6, prenorm=False):
    """RMSNorm of x (+ residual) on the HIP kernels; see the module docstring."""
    if residual is None and prenorm:
        return RMSNormFn.apply(x, weight, None, eps, False), x
    return RMSNormFn.apply(x, weight, residual, eps, prenorm)
