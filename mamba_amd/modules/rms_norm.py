"""RMSNorm with the reference's parameterisation (modules/rms_norm.py:4-31).

out = x * rsqrt(mean(x^2, -1) + eps) * (1 + weight), computed in fp32 and
cast back to x's dtype; weight starts at zero.

``forward(x, residual=None, prenorm=False)`` also takes the residual add
that ends the reference's Block (models/causal_lm.py:31-35): with a
residual it normalises s = x + residual (rounded to x's dtype), and with
``prenorm`` it returns (out, s).  On a ROCm device with ``use_fast_path``
(the default) this is one HIP kernel (``mamba_amd.ops.rms_norm``);
otherwise it is the reference's own sequence of PyTorch ops.
"""
import torch
import torch.nn as nn

from ..ops.rms_norm import rms_norm_fn


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6, device=None, dtype=None, use_fast_path: bool = True):
        super().__init__()
        self.eps = eps
        self.use_fast_path = use_fast_path
        self.weight = nn.Parameter(torch.zeros(dim, device=device, dtype=dtype))

    def forward(self, x, residual=None, prenorm=False):
        if self.use_fast_path and x.is_cuda:
            return rms_norm_fn(x, self.weight, residual, self.eps, prenorm)
        if residual is not None:
            x = x + residual
        xf = x.float()
        out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * (1.0 + self.weight.float())
        out = out.type_as(x)
        return (out, x) if prenorm else out
