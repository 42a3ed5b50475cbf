"""RMSNorm with the reference's parameterisation (modules/rms_norm.py:4-31).

out = x * rsqrt(mean(x^2, -1) + eps) * (1 + weight), computed in fp32 and
cast back to x's dtype; weight starts at zero.
"""
import torch
import torch.nn as nn


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6, device=None, dtype=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.zeros(dim, device=device, dtype=dtype))

    def forward(self, x):
        xf = x.float()
        out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * (1.0 + self.weight.float())
        return out.type_as(x)
