"""Decode-size linear layer on the HIP library's matrix-core kernel.

``decode_linear(x, weight, bias=None)`` computes ``F.linear(x, weight, bias)``
for the few rows of a single-token step (x: (batch, k_in), weight:
(n_out, k_in), nn.Linear's layout).  bf16 / fp16 rows with k_in a multiple of
16 and unit column strides take ``ss_decode_linear`` (one pass over the
weight on the matrix cores); other shapes and dtypes take torch's library
GEMM, which computes the same product.
"""
import ctypes

import torch
import torch.nn.functional as F

from .. import _native as nat
from ..selective_scan import _ITYPES, _ptr, _stream

_MAX_ROWS = 64


def _fits(x, weight, bias):
    return (x.is_cuda and x.dim() == 2 and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype
            and weight.dim() == 2 and weight.shape[1] == x.shape[1] and x.shape[1] % 16 == 0
            and 0 < x.shape[0] <= _MAX_ROWS and x.stride(1) == 1 and weight.stride(1) == 1
            and x.stride(0) % 4 == 0 and weight.stride(0) % 4 == 0
            and x.data_ptr() % 8 == 0 and weight.data_ptr() % 8 == 0
            and (bias is None or (bias.dtype in (x.dtype, torch.float32) and bias.is_contiguous())))


def decode_linear(x, weight, bias=None):
    if not _fits(x, weight, bias):
        return F.linear(x, weight, bias)
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
    with torch.cuda.device(x.device):
        nat.check(lib.ss_decode_linear(ctypes.byref(a), _stream(x.device)), "decode_linear")
    return y
