"""Decode-size linear layer on the HIP library's matrix-core kernel.

``decode_linear(x, weight, bias=None, conv=None)`` computes
``F.linear(x, weight, bias)`` for the few rows of a single-token step (x:
(batch, k_in), weight: (n_out, k_in), nn.Linear's layout).  bf16 / fp16 rows
with k_in a multiple of 16 and unit column strides take ``ss_decode_linear``
(one pass over the weight on the matrix cores, K split over several
workgroups per output tile when there are few tiles); other shapes and
dtypes take torch's library GEMM, which computes the same product.

``conv=(conv_state, conv_weight, conv_bias, activation)`` fuses the block's
conv step into the product: outputs ``n < conv_state.shape[1]`` are replaced
by ``causal_conv1d_update`` of the product rounded to x's dtype (the conv
state advances in place), the rest are returned as they are.  This is the
block's input projection and conv update in one launch.

``norm=(residual, norm_weight, eps)`` fuses the RMSNorm in front of the
product: x is then the RMSNorm input, the product's input rows are
``rms_norm_fn(x, norm_weight, residual, eps, prenorm=True)``'s output, bit for
bit, computed in the same launch, and the call returns ``(y, s)`` with s =
x + residual (x itself without residual), the residual stream that the
prenorm RMSNorm returns.  Shapes the fused launch does not take (rows that
are not 16-byte aligned, k_in above 1024) run the RMSNorm kernel first.

The split needs a small workspace (its tile counters and fp32 partial tiles,
at most about 0.25 MiB); one is kept per (device, stream), allocated zeroed
the first time that stream calls outside a graph capture, and reused by every
later call on it, captured ones included (the kernel leaves it ready for the
next call).  A call captured on a stream that has none yet runs without the
split.  Calls that share a stream run in order, so they never use the
workspace at the same time.  Work that may run beside that stream's own
(a captured graph replayed on another stream) brings its own workspace:
``private_workspace(ws)`` makes the calls of the current thread inside it
use ``ws`` (from ``new_workspace``) instead, which is how ``GraphedStep``
gives every captured step a workspace of its own.
"""
import contextlib
import ctypes
import threading

import torch
import torch.nn.functional as F

from .. import _native as nat
from ..selective_scan import _ITYPES, _ptr, _stream
from .causal_conv1d import _params32, _require, _silu_flag, causal_conv1d_update

_MAX_ROWS = 64
_WS_BYTES = 1 << 20            # covers every split the library picks (at most 63 tiles x 4 slices x 1 KiB + counters)
_workspaces = {}
_ws_lock = threading.Lock()
_private = threading.local()


def new_workspace(device):
    """A zeroed split workspace, for ``private_workspace``."""
    return torch.zeros(_WS_BYTES, dtype=torch.uint8, device=device)


@contextlib.contextmanager
def private_workspace(ws):
    """Calls of this thread inside the block use ``ws`` (on its device) as
    their split workspace instead of the per-stream one."""
    prev = getattr(_private, "ws", None)
    _private.ws = ws
    try:
        yield ws
    finally:
        _private.ws = prev


def _fits(x, weight, bias):
    return (x.is_cuda and x.dim() == 2 and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype
            and weight.dim() == 2 and weight.shape[1] == x.shape[1] and x.shape[1] % 16 == 0
            and 0 < x.shape[0] <= _MAX_ROWS and x.stride(1) == 1 and weight.stride(1) == 1
            and x.stride(0) % 4 == 0 and weight.stride(0) % 4 == 0
            and x.data_ptr() % 8 == 0 and weight.data_ptr() % 8 == 0
            and (bias is None or (bias.dtype in (x.dtype, torch.float32) and bias.is_contiguous())))


def _workspace(device):
    """The split workspace of (device, current stream), or None while a graph
    is being captured on a stream that has none yet; inside
    ``private_workspace`` the one given there."""
    ws = getattr(_private, "ws", None)
    if ws is not None and ws.device == device:
        return ws
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    ws = _workspaces.get(key)
    if ws is not None or torch.cuda.is_current_stream_capturing():
        return ws
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None:
            ws = torch.zeros(_WS_BYTES, dtype=torch.uint8, device=device)
            _workspaces[key] = ws
    return ws


def _conv_args(conv, batch, n_out, dtype, device):
    conv_state, weight, bias, activation = conv
    silu = _silu_flag(activation)
    dim = conv_state.shape[1]
    w, b = _params32(weight, bias, dim, device)
    _require(conv_state.dim() == 3 and conv_state.shape == (batch, dim, w.shape[1]) and conv_state.dtype == dtype
             and conv_state.device == device and dim <= n_out,
             f"conv_state must be ({batch}, dim <= {n_out}, width) of x's dtype, got {tuple(conv_state.shape)}")
    c = nat.Conv1dUpdateArgs()
    c.batch, c.dim, c.width = batch, dim, w.shape[1]
    c.itype, c.has_bias, c.silu = _ITYPES[dtype], int(b is not None), int(silu)
    c.state_batch_stride, c.state_dim_stride, c.state_width_stride = conv_state.stride()
    c.w_dim_stride, c.w_width_stride = w.stride(0), w.stride(1)
    c.conv_state, c.weight, c.bias = _ptr(conv_state), _ptr(w), _ptr(b)
    return c, (w, b)


def _rows16(t):
    return t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def _norm_fits(x, residual, norm_weight):
    return (x.shape[1] <= 1024 and _rows16(x) and (residual is None or (
                residual.shape == x.shape and residual.dtype == x.dtype and _rows16(residual)))
            and norm_weight.dim() == 1 and norm_weight.shape[0] == x.shape[1]
            and norm_weight.dtype in (x.dtype, torch.float32) and norm_weight.is_contiguous()
            and norm_weight.data_ptr() % 16 == 0)


def decode_linear(x, weight, bias=None, conv=None, split=True, norm=None):
    """See the module docstring; ``split=False`` runs without the K split (one
    workgroup per output tile)."""
    if norm is not None:
        residual, norm_weight, eps = norm
        if not (_fits(x, weight, bias) and _norm_fits(x, residual, norm_weight)):
            from .rms_norm import rms_norm_fn
            normed, s = rms_norm_fn(x, norm_weight, residual, eps, prenorm=True)
            return decode_linear(normed, weight, bias, conv=conv, split=split), s
    if not _fits(x, weight, bias):
        y = F.linear(x, weight, bias)
        if conv is not None:
            dim = conv[0].shape[1]
            y[:, :dim] = causal_conv1d_update(y[:, :dim], *conv)
        return y
    lib = nat.load()
    batch, k_in = x.shape
    n_out = weight.shape[0]
    y = torch.empty(batch, n_out, dtype=x.dtype, device=x.device)
    a = nat.DecodeLinearArgs()
    a.batch, a.n_out, a.k_in = batch, n_out, k_in
    a.dtype = _ITYPES[x.dtype]
    a.bias_dtype = _ITYPES[bias.dtype] if bias is not None else a.dtype
    a.x_row_stride, a.w_row_stride, a.y_row_stride = x.stride(0), weight.stride(0), y.stride(0)
    a.x, a.weight, a.bias, a.y = _ptr(x), _ptr(weight), _ptr(bias), _ptr(y)
    keep = None
    if conv is not None:
        c, keep = _conv_args(conv, batch, n_out, x.dtype, x.device)
        a.conv = ctypes.pointer(c)
    s = None
    if norm is not None:
        residual, norm_weight, eps = norm
        s = torch.empty_like(x) if residual is not None else x
        na = nat.RmsNormArgs()
        na.rows, na.dim = batch, k_in
        na.dtype, na.w_dtype = _ITYPES[x.dtype], _ITYPES[norm_weight.dtype]
        na.eps = float(eps)
        na.x_row_stride = x.stride(0)
        if residual is not None:
            na.residual_row_stride, na.residual_out_row_stride = residual.stride(0), s.stride(0)
            na.residual, na.residual_out = _ptr(residual), _ptr(s)
        na.x, na.weight = _ptr(x), _ptr(norm_weight)
        a.norm = ctypes.pointer(na)
        a.x, a.x_row_stride = None, 0
    with torch.cuda.device(x.device):
        if split and lib.ss_decode_linear_workspace_bytes(ctypes.byref(a)) > 0:
            ws = _workspace(x.device)
            if ws is not None:
                a.workspace, a.workspace_bytes = _ptr(ws), ws.numel()
        nat.check(lib.ss_decode_linear(ctypes.byref(a), _stream(x.device)), "decode_linear")
    del keep
    return (y, s) if norm is not None else y
