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
        # the checkpoints x and the pre-gate output y exist for the backward:
        # without a gradient to compute they are neither allocated nor written
        need_bwd = any(ctx.needs_input_grad)
        batch, dim, seqlen = u.shape
        dstate = A.shape[1]
        out = torch.empty_like(delta, memory_format=torch.contiguous_format)
        x = (torch.empty((batch, selective_scan.n_chunks(seqlen), dim, dstate), dtype=torch.float32,
                         device=u.device) if need_bwd else None)
        y = torch.empty_like(out) if z is not None and need_bwd else None
        last_state = None
        if return_last_state:
            last_state = (torch.empty if seqlen > 0 else torch.zeros)(
                (batch, dim, dstate), dtype=torch.float32, device=u.device)
        selective_scan.forward_into(u, delta, A, B, C, D, delta_bias, delta_softplus, out, x, z=z, y=y,
                                    last_state=last_state)
        ctx.delta_softplus = delta_softplus
        ctx.has_z = z is not None
        if need_bwd:
            ctx.save_for_backward(u, delta, A, B, C, D, delta_bias, z, x, y)
        if return_last_state:
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


# ------------------------------------------------------------ Mamba block --
def _cm_view(buf, batch, L):
    """(dim, batch * L) channel-major buffer as a (batch, dim, L) view (unit seqlen stride)."""
    return buf.view(buf.shape[0], batch, L).permute(1, 0, 2)


def _inner_forward(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                   out_proj_bias, A, D, delta_bias, B_proj_bias, C_proj_bias, delta_softplus, save=True,
                   last_state=None):
    """The Mamba block's forward between the projections (see MambaInnerFn); returns
    (out (batch, seqlen, out_features), dict of the intermediates the backward keeps).
    xz: (batch, 2 * dim, seqlen) with unit seqlen stride.  Without ``save`` the scan
    writes no checkpoints and no pre-gate output (nothing for a backward);
    ``last_state`` (fp32 (batch, dim, dstate) contiguous) receives the final state."""
    from .causal_conv1d import causal_conv1d_fwd
    batch, two_d, L = xz.shape
    dim = two_d // 2
    R = delta_proj_weight.shape[1]
    N = A.shape[-1]
    dt, dev = xz.dtype, xz.device
    BL = batch * L
    x, z = xz[:, :dim], xz[:, dim:]

    conv_buf = torch.empty(dim, BL, dtype=dt, device=dev)
    conv_out = _cm_view(conv_buf, batch, L)
    causal_conv1d_fwd(x, conv1d_weight, conv1d_bias, silu=True, out=conv_out)
    x_dblT = x_proj_weight.to(dt) @ conv_buf                          # (R + 2N, b l)
    if B_proj_bias is not None:
        x_dblT[R:R + N] += B_proj_bias.to(dt)[:, None]
    if C_proj_bias is not None:
        x_dblT[R + N:] += C_proj_bias.to(dt)[:, None]
    delta_buf = delta_proj_weight.to(dt) @ x_dblT[:R]                # (dim, b l)
    delta = _cm_view(delta_buf, batch, L)
    Bv = _cm_view(x_dblT[R:R + N], batch, L).unsqueeze(1)           # (batch, 1, N, L)
    Cv = _cm_view(x_dblT[R + N:R + 2 * N], batch, L).unsqueeze(1)
    A32 = A.float().contiguous()
    D32 = D.float().contiguous() if D is not None else None
    db32 = delta_bias.float().contiguous() if delta_bias is not None else None

    out_buf = torch.empty(dim, BL, dtype=dt, device=dev)
    y_buf = torch.empty(dim, BL, dtype=dt, device=dev) if save else None
    xck = (torch.empty((batch, selective_scan.n_chunks(L), dim, N), dtype=torch.float32, device=dev)
           if save else None)
    selective_scan.forward_into(conv_out, delta, A32, Bv, Cv, D32, db32, delta_softplus,
                                _cm_view(out_buf, batch, L), xck, z=z,
                                y=_cm_view(y_buf, batch, L) if save else None, last_state=last_state)
    out_w = out_proj_weight.to(dt)
    res = torch.nn.functional.linear(out_buf.t(), out_w,
                                     out_proj_bias.to(dt) if out_proj_bias is not None else None)
    return res.view(batch, L, -1), {
        "conv_buf": conv_buf, "x_dblT": x_dblT, "delta_buf": delta_buf, "A32": A32, "D32": D32, "db32": db32,
        "xck": xck, "y_buf": y_buf, "out_buf": out_buf, "dims": (batch, dim, L, R, N)}


def mamba_inner_prefill(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                        out_proj_bias, A, D=None, delta_bias=None, B_proj_bias=None, C_proj_bias=None,
                        delta_softplus=True, conv_state=None, ssm_state=None):
    """mamba_inner_fn's forward (no autograd) that also leaves the decode state of the
    sequence's end: conv_state (batch, dim, width) receives the last `width` inputs of
    the conv (zeros before the sequence start) and ssm_state (batch, dim, dstate) fp32
    the scan's state after the last step, so that decoding continues from there."""
    if xz.shape[-1] > 1 and xz.stride(-1) != 1:
        xz = xz.contiguous()
    with torch.no_grad():
        last = None
        if ssm_state is not None:
            direct = ssm_state.dtype == torch.float32 and ssm_state.is_contiguous() and xz.shape[-1] > 0
            last = ssm_state if direct else torch.zeros(ssm_state.shape, dtype=torch.float32, device=xz.device)
        res, t = _inner_forward(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                                out_proj_weight, out_proj_bias, A, D, delta_bias, B_proj_bias, C_proj_bias,
                                delta_softplus, save=False, last_state=last)
        batch, dim, L, _, _ = t["dims"]
        if ssm_state is not None and last is not ssm_state:
            ssm_state.copy_(last)
        if conv_state is not None:
            W = conv_state.shape[-1]
            x = xz[:, :dim]
            tail = x[..., max(0, L - W):]
            conv_state.zero_()
            conv_state[..., W - tail.shape[-1]:].copy_(tail)
    return res


class MambaInnerFn(torch.autograd.Function):
    """The Mamba block between in- and out-projection, with the scan fused.

    Same computation as the reference's MambaSimple.forward after its
    input_proj (modules/mamba_simple.py:98-149), in the mamba_ssm
    ``mamba_inner_fn`` argument order: causal conv1d + SiLU on the x half of
    xz, x_proj into (dt, B, C), delta = delta_proj_weight @ dt, the selective
    scan with the delta bias, softplus and the z gate fused, and the
    out-projection.

    Every (batch, dim, seqlen) intermediate lives channel-major, as a
    (dim, batch * seqlen) buffer viewed as (batch, dim, seqlen) with unit
    seqlen stride: the HIP conv and scan kernels take those strides
    directly, and every projection (x_proj, delta_proj, out_proj and their
    gradients) is then one plain GEMM with no layout copies.  B and C are
    strided views of x_proj's output.  Intermediates are kept for the
    backward (no recomputation: HBM capacity is not the constraint here).
    """

    @staticmethod
    def forward(ctx, xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None,
                B_proj_bias=None, C_proj_bias=None, delta_softplus=True):
        if B is not None or C is not None:
            raise ValueError("mamba_inner_fn: B and C must come from x_proj (pass B=None, C=None)")
        if xz.shape[-1] > 1 and xz.stride(-1) != 1:
            xz = xz.contiguous()
        save = any(ctx.needs_input_grad)
        res, t = _inner_forward(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                                out_proj_weight, out_proj_bias, A, D, delta_bias, B_proj_bias, C_proj_bias,
                                delta_softplus, save=save)
        if not save:
            return res
        ctx.save_for_backward(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
                              t["conv_buf"], t["x_dblT"], t["delta_buf"], t["A32"], t["D32"], t["db32"], t["xck"],
                              t["y_buf"], t["out_buf"], A, D, delta_bias, out_proj_bias, B_proj_bias, C_proj_bias)
        ctx.delta_softplus = delta_softplus
        ctx.dims = t["dims"]
        return res

    @staticmethod
    def backward(ctx, dres):
        from .causal_conv1d import causal_conv1d_bwd
        (xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight, out_proj_weight,
         conv_buf, x_dblT, delta_buf, A32, D32, db32, xck, y_buf, out_buf,
         A, D, delta_bias, out_proj_bias, B_proj_bias, C_proj_bias) = ctx.saved_tensors
        batch, dim, L, R, N = ctx.dims
        dt, dev = xz.dtype, xz.device
        BL = batch * L
        dres2 = dres.reshape(BL, -1).to(dt)
        if not dres2.is_contiguous():
            dres2 = dres2.contiguous()
        out_w = out_proj_weight.to(dt)

        # out-projection
        dout_buf = out_w.t() @ dres2.t()                                 # (dim, b l)
        dout_proj_weight = dres2.t() @ out_buf.t()                       # (out, dim)
        dout_proj_bias = dres2.sum(0) if out_proj_bias is not None else None

        # scan (writes du / ddelta channel-major, dz into the z half of dxz)
        dxz = torch.empty_like(xz)
        dconv_buf = torch.empty(dim, BL, dtype=dt, device=dev)
        ddelta_buf = torch.empty(dim, BL, dtype=dt, device=dev)
        Bv = _cm_view(x_dblT[R:R + N], batch, L).unsqueeze(1)
        Cv = _cm_view(x_dblT[R + N:R + 2 * N], batch, L).unsqueeze(1)
        dA = torch.empty(A32.shape, dtype=torch.float32, device=dev)
        dB = torch.empty((batch, 1, N, L), dtype=torch.float32, device=dev)
        dC = torch.empty((batch, 1, N, L), dtype=torch.float32, device=dev)
        dD = torch.empty(D32.shape, dtype=torch.float32, device=dev) if D32 is not None else None
        ddb = torch.empty(db32.shape, dtype=torch.float32, device=dev) if db32 is not None else None
        selective_scan.backward_into(_cm_view(conv_buf, batch, L), _cm_view(delta_buf, batch, L), A32, Bv, Cv,
                                     D32, db32, _cm_view(dout_buf, batch, L), xck, ctx.delta_softplus,
                                     _cm_view(dconv_buf, batch, L), _cm_view(ddelta_buf, batch, L),
                                     dA, dB, dC, dD, ddb, z=xz[:, dim:], y=_cm_view(y_buf, batch, L),
                                     dz=dxz[:, dim:], zero_grads=True)

        # x_proj / delta_proj
        dx_dblT = torch.empty(R + 2 * N, BL, dtype=dt, device=dev)
        dx_dblT[R:R + N].view(N, batch, L).copy_(dB[:, 0].permute(1, 0, 2))
        dx_dblT[R + N:].view(N, batch, L).copy_(dC[:, 0].permute(1, 0, 2))
        ddelta_proj_weight = ddelta_buf @ x_dblT[:R].t()                 # (dim, R)
        torch.matmul(delta_proj_weight.to(dt).t(), ddelta_buf, out=dx_dblT[:R])
        dx_proj_weight = dx_dblT @ conv_buf.t()                          # (R + 2N, dim)
        dconv_buf.addmm_(x_proj_weight.to(dt).t(), dx_dblT)
        dB_proj_bias = dx_dblT[R:R + N].sum(1) if B_proj_bias is not None else None
        dC_proj_bias = dx_dblT[R + N:].sum(1) if C_proj_bias is not None else None

        # conv1d + SiLU (dx into the x half of dxz)
        _, dconv_w, dconv_b = causal_conv1d_bwd(xz[:, :dim], conv1d_weight, conv1d_bias,
                                                _cm_view(dconv_buf, batch, L), silu=True, dx=dxz[:, :dim])

        def like(g, ref):
            return None if g is None or ref is None else g.reshape(ref.shape).to(ref.dtype)
        return (dxz, like(dconv_w, conv1d_weight), like(dconv_b, conv1d_bias), like(dx_proj_weight, x_proj_weight),
                like(ddelta_proj_weight, delta_proj_weight), like(dout_proj_weight, out_proj_weight),
                like(dout_proj_bias, out_proj_bias), like(dA, A), None, None, like(dD, D),
                like(ddb, delta_bias), like(dB_proj_bias, B_proj_bias), like(dC_proj_bias, C_proj_bias), None)


def mamba_inner_fn(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                   out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None,
                   B_proj_bias=None, C_proj_bias=None, delta_softplus=True):
    """Mamba block (conv, projections, scan with z gate) on the HIP kernels.

    xz: (batch, 2 * dim, seqlen) with unit seqlen stride (the channel-major
    output of the in-projection, viewed as (batch, 2 * dim, seqlen), is used
    without a copy); conv1d_weight: (dim, 1, width) or (dim, width);
    x_proj_weight: (dt_rank + 2 * dstate, dim); delta_proj_weight:
    (dim, dt_rank); out_proj_weight: (out_features, dim); A: (dim, dstate).
    Returns (batch, seqlen, out_features).
    """
    return MambaInnerFn.apply(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                              out_proj_weight, out_proj_bias, A, B, C, D, delta_bias, B_proj_bias,
                              C_proj_bias, delta_softplus)
