"""CPU oracle for single-token decode (test infrastructure only).

Only tests/ import this module; the product path (mamba_amd) never does.

The reference has no decode path (CausalLM.generate is a stub,
models/causal_lm.py:61-62).  These functions restate one step of the two
recurrences the reference computes over whole sequences, so that a step
applied token after token from a zero state reproduces them:

* ``selective_state_update_ref``: one step of the selective scan
  (forward_kernel.cu:216-293; the scan oracle is selective_scan_ref):
  h <- exp(dt A) h + dt x B, y = C . h + D x, times silu(z);
* ``causal_conv1d_update_ref``: one step of the depthwise causal conv
  (modules/mamba_simple.py:40-47,100-101; the sequence oracle is
  causal_conv1d_ref), with the state holding the last `width` inputs.

Both are functional (they return the new state rather than updating it).
"""
import torch
import torch.nn.functional as F


def selective_state_update_ref(state, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=False,
                               compute_dtype=torch.float64):
    """state (batch, dim, N); x, dt, z (batch, dim); A (dim, N); B, C (batch, N) or
    (batch, G, N); D, dt_bias (dim,).  Returns (out (batch, dim) in x's dtype, new state
    in compute_dtype)."""
    ct = compute_dtype
    batch, dim = x.shape
    if B.dim() == 2:
        B = B.unsqueeze(1)
    if C.dim() == 2:
        C = C.unsqueeze(1)
    g = B.shape[1]
    Bx = B.to(ct).repeat_interleave(dim // g, dim=1)                 # (batch, dim, N)
    Cx = C.to(ct).repeat_interleave(dim // g, dim=1)
    d = dt.to(ct)
    if dt_bias is not None:
        d = d + dt_bias.to(ct)
    if dt_softplus:
        d = F.softplus(d, beta=1.0, threshold=20.0)
    xx = x.to(ct)
    h = torch.exp(d[..., None] * A.to(ct)) * state.to(ct) + (d * xx)[..., None] * Bx
    y = (Cx * h).sum(-1)
    if D is not None:
        y = y + D.to(ct) * xx
    if z is not None:
        y = y * F.silu(z.to(ct))
    return y.to(x.dtype), h


def causal_conv1d_update_ref(x, conv_state, weight, bias=None, activation=None):
    """x (batch, dim); conv_state (batch, dim, width); weight (dim, width) or
    (dim, 1, width).  Returns (out (batch, dim), new conv_state)."""
    w = weight.reshape(weight.shape[0], weight.shape[-1]).to(x.dtype)
    st = torch.cat([conv_state[..., 1:], x[..., None].to(conv_state.dtype)], dim=-1)
    out = (st.to(x.dtype) * w).sum(-1)
    if bias is not None:
        out = out + bias.to(x.dtype)
    if activation in ("silu", "swish"):
        out = F.silu(out)
    return out, st
