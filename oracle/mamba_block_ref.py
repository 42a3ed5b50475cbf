"""CPU oracle for the Mamba block around the scan (test infrastructure only).

Only tests/, the __graft_entry__ smoke check and bench.py's cpu_baseline leg
import this module; the product path (mamba_amd) never does.

* ``causal_conv1d_ref`` restates the reference's depthwise causal conv
  (nn.Conv1d(dim, dim, width, groups=dim, padding=width - 1) cut to seqlen,
  then SiLU: modules/mamba_simple.py:40-47,100-101) as an explicit sum over
  taps.
* ``mamba_inner_ref`` is the Mamba block between in-projection and
  out-projection, as the reference's MambaSimple.forward computes it
  (modules/mamba_simple.py:95-149) but starting from the packed xz tensor:
  conv + SiLU on x, x_proj (the reference's ssm_param_proj) split into
  delta / B / C, delta = W_delta @ dt without bias (the bias goes into the
  scan as delta_bias with softplus), the selective scan, the z gate
  y * silu(z), and the out-projection.
* ``mamba_simple_ref`` is MambaSimple.forward from a dict of the reference
  module's parameters (the same names), and ``rms_norm_ref`` /
  ``causal_lm_ref`` restate modules/rms_norm.py:19-31 and
  models/causal_lm.py:30-59; ``add_rms_norm_ref`` is a block's residual add
  (models/causal_lm.py:31-35) followed by the next RMSNorm.
"""
import torch
import torch.nn.functional as F

from .selective_scan_ref import selective_scan_ref


def causal_conv1d_ref(x, weight, bias=None, activation=None):
    """x: (batch, dim, seqlen); weight: (dim, width) or (dim, 1, width)."""
    w = weight.reshape(weight.shape[0], weight.shape[-1]).to(x.dtype)
    width = w.shape[1]
    L = x.shape[-1]
    xp = F.pad(x, (width - 1, 0))
    out = torch.zeros_like(x)
    for k in range(width):
        out = out + w[:, k, None] * xp[..., k:k + L]
    if bias is not None:
        out = out + bias.to(x.dtype)[:, None]
    if activation in ("silu", "swish"):
        out = F.silu(out)
    return out


def mamba_inner_ref(xz, conv1d_weight, conv1d_bias, x_proj_weight, delta_proj_weight,
                    out_proj_weight, out_proj_bias, A, B=None, C=None, D=None, delta_bias=None,
                    B_proj_bias=None, C_proj_bias=None, delta_softplus=True, scan=None):
    """xz: (batch, 2 * dim, seqlen) -> (batch, seqlen, out_features).  ``scan``
    replaces selective_scan_ref (same signature), e.g. c_oracle.scan for
    long sequences."""
    L = xz.shape[-1]
    R = delta_proj_weight.shape[1]
    N = A.shape[-1]
    x, z = xz.chunk(2, dim=1)
    x = causal_conv1d_ref(x, conv1d_weight, conv1d_bias, activation="silu")
    batch, dim, _ = x.shape
    x_dbl = F.linear(x.transpose(1, 2).reshape(batch * L, dim), x_proj_weight)      # (b l, R + 2N)
    delta = (delta_proj_weight @ x_dbl[:, :R].t()).reshape(dim, batch, L).transpose(0, 1)
    if B is None:
        B = x_dbl[:, R:R + N]
        if B_proj_bias is not None:
            B = B + B_proj_bias.to(B.dtype)
        B = B.reshape(batch, L, N).transpose(1, 2).unsqueeze(1)
    if C is None:
        C = x_dbl[:, R + N:R + 2 * N]
        if C_proj_bias is not None:
            C = C + C_proj_bias.to(C.dtype)
        C = C.reshape(batch, L, N).transpose(1, 2).unsqueeze(1)
    ct = torch.float64 if x.dtype == torch.float64 else torch.float32
    y = (scan or selective_scan_ref)(x, delta, A, B, C, D, z=z, delta_bias=delta_bias,
                                     delta_softplus=delta_softplus, compute_dtype=ct)
    return F.linear(y.transpose(1, 2), out_proj_weight, out_proj_bias)


def mamba_simple_ref(p, hidden, state_dim=16, scan=None):
    """MambaSimple.forward (modules/mamba_simple.py:95-149) from its parameters.

    p: dict with the reference module's parameter names: input_proj.weight
    (+ .bias), short_conv.weight (+ .bias), ssm_param_proj.weight,
    delta_proj.weight, delta_proj.bias, log_A, D, output_proj.weight (+ .bias).
    """
    # A, D and the delta bias enter the scan in fp32 (modules/mamba_simple.py:128,137-138)
    ft = torch.float64 if hidden.dtype == torch.float64 else torch.float32
    xz = F.linear(hidden, p["input_proj.weight"], p.get("input_proj.bias")).transpose(1, 2)
    A = -torch.exp(p["log_A"].to(ft))
    return mamba_inner_ref(xz, p["short_conv.weight"], p.get("short_conv.bias"), p["ssm_param_proj.weight"],
                           p["delta_proj.weight"], p["output_proj.weight"], p.get("output_proj.bias"), A,
                           D=p["D"].to(ft), delta_bias=p["delta_proj.bias"].to(ft), delta_softplus=True,
                           scan=scan)


def rms_norm_ref(x, weight, eps=1e-6):
    """modules/rms_norm.py:19-31: x * rsqrt(mean(x^2) + eps) * (1 + weight), in fp32, cast back."""
    xf = x.double() if x.dtype == torch.float64 else x.float()
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + weight.to(xf.dtype))
    return out.to(x.dtype)


def add_rms_norm_ref(x, residual, weight, eps=1e-6):
    """The residual add that ends a block (models/causal_lm.py:31-35, ``hidden_states += residual``
    in x's dtype) followed by the next block's RMSNorm: returns (rms_norm_ref(s), s), s = x + residual."""
    s = x if residual is None else x + residual
    return rms_norm_ref(s, weight, eps), s


def causal_lm_ref(p, input_ids, num_layers, state_dim=16, eps=1e-6, scan=None):
    """CausalLM.forward in eval mode (dropout off): models/causal_lm.py:30-59.

    p holds the reference model's state_dict names: embedding.weight,
    layers.{i}.norm.weight, layers.{i}.mamba.*, norm.weight, lm_head.weight.
    """
    h = F.embedding(input_ids, p["embedding.weight"])
    for i in range(num_layers):
        sub = {k[len(f"layers.{i}.mamba."):]: v for k, v in p.items() if k.startswith(f"layers.{i}.mamba.")}
        h = h + mamba_simple_ref(sub, rms_norm_ref(h, p[f"layers.{i}.norm.weight"], eps), state_dim, scan=scan)
    h = rms_norm_ref(h, p["norm.weight"], eps)
    return F.linear(h, p.get("lm_head.weight", p["embedding.weight"]))
