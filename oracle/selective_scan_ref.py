"""CPU oracle for the selective scan (test infrastructure only).

This module is test infrastructure, never the product: only ``tests/``, the
``__graft_entry__.smoke()`` check and the ``cpu_baseline`` leg of ``bench.py``
may import it.  The product path (``mamba_amd``) runs on the HIP library and
fails loudly when that library is missing.

``selective_scan_ref`` restates, in plain PyTorch fp32, the arithmetic of the
reference's two CUDA kernels plus the caller-side z gate:

* delta + delta_bias, then softplus with the threshold-20 rule
  (csrc/selective_scan/forward_kernel.cu:216-221);
* deltaA = exp(delta * A) (computed there as exp2(delta * A * log2 e),
  forward_kernel.cu:228,264);
* deltaB_u = delta * B * u, with constant B (shape (D, N)) or variable B
  (shape (Bt, G, N, L), channel d uses group d // (D // G),
  forward_kernel.cu:144,265; selective_scan.cpp:194,202);
* h_t = deltaA_t * h_{t-1} + deltaB_u_t, h_{-1} = 0
  (scan operator common.h:75-81, identity forward_kernel.cu:277);
* y_t = sum_n C_t * h_t (+ D * u_t) (forward_kernel.cu:223,287-293);
* optional z gate out = y * silu(z) (modules/mamba_simple.py:143-146);
* output dtype = delta's dtype (selective_scan.cpp:206).

Gradients come from torch.autograd through this function.  The closed-form
backward of backward_kernel.cu:276-585 is restated separately in
``oracle/ss_oracle.c`` (float64), and the tests pin each against the other and
against fp64 gradcheck.
"""
import torch
import torch.nn.functional as F


def _expand_groups(M, dim):
    """(Bt, G, N, L) -> (Bt, D, N, L); channel d reads group d // (D // G)."""
    G = M.shape[1]
    if dim % G != 0:
        raise ValueError(f"dim {dim} is not a multiple of n_groups {G}")
    return M.repeat_interleave(dim // G, dim=1)


def selective_scan_ref(u, delta, A, B, C, D=None, z=None, delta_bias=None,
                       delta_softplus=False, return_last_state=False,
                       compute_dtype=torch.float32):
    """Sequential selective scan.

    u, delta, z: (Bt, D, L); A: (D, N); B, C: (Bt, G, N, L) or (D, N);
    D, delta_bias: (D,).  Returns out (Bt, D, L) in delta's dtype, and the
    final state h_{L-1} (Bt, D, N) in ``compute_dtype`` when
    ``return_last_state``.
    """
    out_dtype = delta.dtype
    ct = compute_dtype
    u = u.to(ct)
    delta = delta.to(ct)
    if delta_bias is not None:
        delta = delta + delta_bias.to(ct)[:, None]
    if delta_softplus:
        # softplus(x) = log1p(exp(x)) for x <= 20, x above (forward_kernel.cu:217-221)
        delta = F.softplus(delta, beta=1.0, threshold=20.0)
    Bt, dim, L = u.shape
    A = A.to(ct)
    N = A.shape[1]
    var_B = B.dim() >= 3
    var_C = C.dim() >= 3
    deltaA = torch.exp(delta.unsqueeze(-1) * A[None, :, None, :])       # (Bt, D, L, N)
    if var_B:
        Bx = _expand_groups(B.to(ct), dim)                                # (Bt, D, N, L)
        deltaB_u = (delta * u).unsqueeze(-1) * Bx.transpose(2, 3)        # (Bt, D, L, N)
    else:
        deltaB_u = (delta * u).unsqueeze(-1) * B.to(ct)[None, :, None, :]
    if var_C:
        Cx = _expand_groups(C.to(ct), dim).transpose(2, 3)               # (Bt, D, L, N)
    else:
        Cx = C.to(ct)[None, :, None, :].expand(Bt, dim, L, N)
    h = u.new_zeros((Bt, dim, N))
    ys = []
    for t in range(L):
        h = deltaA[:, :, t] * h + deltaB_u[:, :, t]
        ys.append((h * Cx[:, :, t]).sum(-1))
    y = torch.stack(ys, dim=2) if L > 0 else u.new_zeros((Bt, dim, 0))
    out = y if D is None else y + u * D.to(ct)[:, None]
    if z is not None:
        out = out * F.silu(z.to(ct))
    out = out.to(out_dtype)
    if return_last_state:
        return out, h
    return out


def make_inputs(batch, dim, dstate, seqlen, *, seed, dtype=torch.float32,
                n_groups=1, var_B=True, var_C=True, has_z=True, has_D=True,
                has_delta_bias=True, dt_min=1e-3, dt_max=1e-1):
    """Seeded synthetic inputs with the benchmark distributions.

    A CPU generator seeded with ``seed`` draws, in this order, u, delta, z,
    B, C, dt and dout, each N(0,1) fp32 (dt uniform), so GPU and CPU runs see
    bit-identical tensors.  delta_bias = dt + log(-expm1(-dt)) is the inverse
    softplus of dt ~ U[dt_min, dt_max] (the form of
    modules/mamba_simple.py:76); A = -(1..N) per channel
    (modules/mamba_simple.py:80-82,128); D = ones.
    """
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(batch, dim, seqlen, generator=g)
    delta = torch.randn(batch, dim, seqlen, generator=g)
    z = torch.randn(batch, dim, seqlen, generator=g)
    if var_B:
        B = torch.randn(batch, n_groups, dstate, seqlen, generator=g)
    else:
        B = torch.randn(dim, dstate, generator=g)
    if var_C:
        C = torch.randn(batch, n_groups, dstate, seqlen, generator=g)
    else:
        C = torch.randn(dim, dstate, generator=g)
    dt = torch.rand(dim, generator=g) * (dt_max - dt_min) + dt_min
    dout = torch.randn(batch, dim, seqlen, generator=g)
    delta_bias = dt + torch.log(-torch.expm1(-dt))
    A = -torch.arange(1, dstate + 1, dtype=torch.float32).repeat(dim, 1)
    Dv = torch.ones(dim)
    cast = lambda t: t.to(dtype)
    return dict(
        u=cast(u), delta=cast(delta), A=A,
        B=cast(B) if var_B else B, C=cast(C) if var_C else C,
        D=Dv if has_D else None,
        z=cast(z) if has_z else None,
        delta_bias=delta_bias if has_delta_bias else None,
        dout=cast(dout),
    )
