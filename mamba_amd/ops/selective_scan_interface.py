"""Autograd interface of the selective scan.

``SelectiveScanFn`` keeps the reference's class, argument order and return
values (ops/selective_scan_interface.py:7-49):

    SelectiveScanFn.apply(u, delta, A, B, C, D, delta_bias=None,
                          use_delta_softplus=True) -> out

with ``backward`` returning (du, ddelta, dA, dB, dC, dD, ddelta_bias, None).

``selective_scan_fn`` is the mamba_ssm-style entry point named by the
Mamba block API: it adds the fused z gate (out = y * silu(z), which the
reference applies in PyTorch in modules/mamba_simple.py:143-146) and
``return_last_state`` (h at the last step, shape (batch, dim, dstate)).

Both run on libmamba_ss.so through ``mamba_amd.selective_scan``.
"""
import torch

from .. import selective_scan
from ..utils.tensor_utils import ensure_contiguous


class SelectiveScanFn(torch.autograd.Function):
    """Reference-compatible autograd function (no z gate)."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D, delta_bias=None, use_delta_softplus=True):
        """
        Args:
            u: [batch_size, num_channels, seq_len]
            delta: [batch_size, num_channels, seq_len]
            A: [num_channels, state_dim]
            B: [batch_size, num_groups, state_dim, seq_len] or [num_channels, state_dim]
            C: [batch_size, num_groups, state_dim, seq_len] or [num_channels, state_dim]
            D: [num_channels]
            delta_bias: [num_channels]
        """
        u = ensure_contiguous(u)
        delta = ensure_contiguous(delta)
        A = ensure_contiguous(A)
        B = ensure_contiguous(B)
        C = ensure_contiguous(C)
        D = ensure_contiguous(D)
        delta_bias = ensure_contiguous(delta_bias)
        out, x = selective_scan.forward(u, delta, A, B, C, D, delta_bias, use_delta_softplus)
        ctx.use_delta_softplus = use_delta_softplus
        ctx.save_for_backward(u, delta, A, B, C, D, delta_bias, x)
        return out

    @staticmethod
    def backward(ctx, dout):
        dout = ensure_contiguous(dout)
        u, delta, A, B, C, D, delta_bias, x = ctx.saved_tensors
        du, ddelta, dA, dB, dC, dD, ddelta_bias = selective_scan.backward(
            u, delta, A, B, C, D, delta_bias, dout, x, ctx.use_delta_softplus)
        return du, ddelta, dA, dB, dC, dD, ddelta_bias, None


def _seq_ok(t):
    """True if t is (batch, dim, seqlen) with unit stride along seqlen."""
    return t.shape[-1] <= 1 or t.stride(-1) == 1


class SelectiveScanZFn(torch.autograd.Function):
    """Selective scan with optional fused z gate and last-state output."""

    @staticmethod
    def forward(ctx, u, delta, A, B, C, D=None, z=None, delta_bias=None,
                delta_softplus=False, return_last_state=False):
        # batch / channel strides are passed to the kernels, so only tensors
        # whose seqlen stride is not 1 need a copy
        u = u if _seq_ok(u) else u.contiguous()
        delta = delta if _seq_ok(delta) else delta.contiguous()
        z = z if z is None or _seq_ok(z) else z.contiguous()
        if B.dim() == 3:
            B = B.unsqueeze(1)
            ctx.squeeze_B = True
        else:
            ctx.squeeze_B = False
        if C.dim() == 3:
            C = C.unsqueeze(1)
            ctx.squeeze_C = True
        else:
            ctx.squeeze_C = False
        B = B if B.dim() < 3 or _seq_ok(B) else B.contiguous()
        C = C if C.dim() < 3 or _seq_ok(C) else C.contiguous()
        if B.dim() < 3:
            B = B.float().contiguous()
        if C.dim() < 3:
            C = C.float().contiguous()
        A = A.float()
        D = D.float().contiguous() if D is not None else None
        delta_bias = delta_bias.float().contiguous() if delta_bias is not None else None
        res = selective_scan.forward(u, delta, A, B, C, D, delta_bias, delta_softplus, z=z)
        out, x = res[0], res[1]
        y = res[2] if z is not None else None
        ctx.delta_softplus = delta_softplus
        ctx.has_z = z is not None
        ctx.save_for_backward(u, delta, A, B, C, D, delta_bias, z, x, y)
        ctx.mark_non_differentiable(x)
        if return_last_state:
            # x is (batch, n_chunks, dim, dstate); its last chunk holds h at the last step
            last_state = x[:, -1] if x.shape[1] > 0 else x.new_zeros(x.shape[0], x.shape[2], x.shape[3])
            ctx.mark_non_differentiable(last_state)
            return out, last_state
        return out

    @staticmethod
    def backward(ctx, dout, *unused):
        u, delta, A, B, C, D, delta_bias, z, x, y = ctx.saved_tensors
        if not _seq_ok(dout) or dout.dtype != delta.dtype:
            dout = dout.to(delta.dtype).contiguous()
        res = selective_scan.backward(u, delta, A, B, C, D, delta_bias, dout, x,
                                      ctx.delta_softplus, z=z, y=y)
        du, ddelta, dA, dB, dC, dD, ddelta_bias = res[:7]
        dz = res[7] if ctx.has_z else None
        if B.dim() >= 3:
            dB = dB.to(B.dtype)
        if C.dim() >= 3:
            dC = dC.to(C.dtype)
        if ctx.squeeze_B:
            dB = dB.squeeze(1)
        if ctx.squeeze_C:
            dC = dC.squeeze(1)
        return du, ddelta, dA, dB, dC, dD, dz, ddelta_bias, None, None


def selective_scan_fn(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                      delta_softplus=False, return_last_state=False):
    """Selective scan with fused z gate.

    u, delta, z: (batch, dim, seqlen); A: (dim, dstate) (used in fp32);
    B, C: (batch, n_groups, dstate, seqlen), (batch, dstate, seqlen) for one
    group, or constant (dim, dstate); D, delta_bias: (dim,).
    Returns out (delta's dtype), plus last_state (batch, dim, dstate) fp32
    when ``return_last_state``.
    """
    return SelectiveScanZFn.apply(u, delta, A, B, C, D, z, delta_bias, delta_softplus, return_last_state)
