"""MambaSimple with the reference's constructor, parameters and forward.

The module mirrors modules/mamba_simple.py:8-149: the same constructor
arguments, parameter names and shapes (input_proj, short_conv,
ssm_param_proj, delta_proj, log_A, D, output_proj) and the same
initialisation, so the reference's state_dict loads unchanged.  Two
forward paths compute the same function:

* ``use_fast_path=True`` (default): in-projection as one GEMM straight into
  the channel-major xz layout, then ``mamba_inner_fn`` (HIP conv1d + SiLU,
  projections, HIP selective scan with the z gate fused, out-projection);
* ``use_fast_path=False``: the reference's own sequence of PyTorch ops
  around ``SelectiveScanFn`` (modules/mamba_simple.py:95-149), with the scan
  on the HIP library.

Decoding (absent in the reference, whose CausalLM.generate is a stub):
``allocate_inference_cache`` gives a (conv_state, ssm_state) pair,
``forward(hidden, inference_cache=...)`` fills it from a whole prompt, and
``step`` advances the block by one token on the HIP state-update kernels.
"""
import math

import torch
import torch.nn as nn

from ..ops.decode_linear import decode_linear
from ..ops.selective_scan_interface import SelectiveScanFn, mamba_inner_fn, mamba_inner_prefill
from ..ops.selective_state_update import selective_state_update


class MambaSimple(nn.Module):
    def __init__(
        self,
        model_dim: int,
        state_dim: int = 16,
        conv_kernel: int = 4,
        expansion_factor: int = 2,
        delta_rank="auto",
        delta_min: float = 0.001,
        delta_max: float = 0.1,
        delta_init: str = "random",
        delta_scale: float = 1.0,
        delta_init_floor: float = 1e-4,
        conv_bias: bool = False,
        bias: bool = False,
        device=None,
        dtype=None,
        use_fast_path: bool = True,
    ):
        super().__init__()
        fk = {"device": device, "dtype": dtype}
        self.model_dim = model_dim
        self.state_dim = state_dim
        self.conv_kernel = conv_kernel
        self.expansion_factor = expansion_factor
        self.inner_dim = int(expansion_factor * model_dim)
        self.delta_rank = math.ceil(model_dim / 16) if delta_rank == "auto" else delta_rank
        self.use_fast_path = use_fast_path

        self.input_proj = nn.Linear(self.model_dim, self.inner_dim * 2, bias=bias, **fk)
        self.short_conv = nn.Conv1d(self.inner_dim, self.inner_dim, kernel_size=conv_kernel,
                                    padding=conv_kernel - 1, groups=self.inner_dim, bias=conv_bias, **fk)
        self.act = nn.SiLU()
        self.ssm_param_proj = nn.Linear(self.inner_dim, self.delta_rank + self.state_dim * 2, bias=False, **fk)
        self.delta_proj = nn.Linear(self.delta_rank, self.inner_dim, bias=True, **fk)

        # initialisation of modules/mamba_simple.py:61-85
        delta_std = self.delta_rank ** -0.5 * delta_scale
        if delta_init == "constant":
            nn.init.constant_(self.delta_proj.weight, delta_std)
        elif delta_init == "random":
            nn.init.uniform_(self.delta_proj.weight, -delta_std, delta_std)
        else:
            raise NotImplementedError
        delta = torch.exp(
            torch.rand(self.inner_dim, device=device, dtype=torch.float32)
            * (math.log(delta_max) - math.log(delta_min)) + math.log(delta_min)
        ).clamp(min=delta_init_floor)
        inv_delta = delta + torch.log(-torch.expm1(-delta))
        with torch.no_grad():
            self.delta_proj.bias.copy_(inv_delta)
        A = torch.arange(1, state_dim + 1, device=device, dtype=torch.float32)
        A = A.unsqueeze(0).expand(self.inner_dim, state_dim).contiguous()
        self.log_A = nn.Parameter(torch.log(A))
        self.D = nn.Parameter(torch.ones(self.inner_dim, device=device))
        self.output_proj = nn.Linear(self.inner_dim, model_dim, bias=bias, **fk)

    def forward(self, hidden_states, inference_cache=None):
        """(batch, seqlen, model_dim) -> (batch, seqlen, model_dim).

        With ``inference_cache`` (a (conv_state, ssm_state) pair from
        allocate_inference_cache) the pair is left holding the state after the
        last token, for ``step``; this needs the fast path on a ROCm device."""
        if inference_cache is not None:
            if not (self.use_fast_path and hidden_states.is_cuda):
                raise ValueError("MambaSimple: filling an inference cache needs the fast path on a ROCm device")
            return self._forward_fast(hidden_states, inference_cache)
        if self.use_fast_path and hidden_states.is_cuda:
            return self._forward_fast(hidden_states)
        return self._forward_reference(hidden_states)

    def _forward_fast(self, hidden_states, inference_cache=None):
        batch, seqlen, _ = hidden_states.shape
        # xz = W_in @ h^T: (2 * inner_dim, batch * seqlen), viewed as (batch, 2 * inner_dim, seqlen)
        xz = self.input_proj.weight @ hidden_states.reshape(batch * seqlen, self.model_dim).t()
        if self.input_proj.bias is not None:
            xz = xz + self.input_proj.bias[:, None]
        xz = xz.view(2 * self.inner_dim, batch, seqlen).permute(1, 0, 2)
        if torch.is_grad_enabled():
            A = -torch.exp(self.log_A.float())
            D, delta_bias = self.D.float(), self.delta_proj.bias.float()
            conv_w, conv_b = self.short_conv.weight, self.short_conv.bias
        else:
            # no autograd graph: the fp32 parameters of the last call, unless one changed
            A, D, delta_bias, conv_w, conv_b = self._decode_params()
        args = (xz, conv_w, conv_b, self.ssm_param_proj.weight,
                self.delta_proj.weight, self.output_proj.weight, self.output_proj.bias, A)
        kw = dict(D=D, delta_bias=delta_bias, delta_softplus=True)
        if inference_cache is not None:
            conv_state, ssm_state = inference_cache
            return mamba_inner_prefill(*args, **kw, conv_state=conv_state, ssm_state=ssm_state)
        return mamba_inner_fn(*args, **kw)

    def allocate_inference_cache(self, batch_size, dtype=None, device=None):
        """(conv_state (batch, inner_dim, conv_kernel) in the weights' dtype, ssm_state
        (batch, inner_dim, state_dim) fp32), zero: the state before a sequence starts."""
        device = self.input_proj.weight.device if device is None else device
        dtype = self.input_proj.weight.dtype if dtype is None else dtype
        conv_state = torch.zeros(batch_size, self.inner_dim, self.conv_kernel, dtype=dtype, device=device)
        ssm_state = torch.zeros(batch_size, self.inner_dim, self.state_dim, dtype=torch.float32, device=device)
        return conv_state, ssm_state

    def step(self, hidden_states, conv_state, ssm_state):
        """One token: hidden_states (batch, model_dim) or (batch, 1, model_dim) -> the same
        shape; conv_state and ssm_state are advanced in place."""
        squeeze = hidden_states.dim() == 3
        h = hidden_states.reshape(-1, self.model_dim)
        *_, conv_w, conv_b = self._decode_params()
        # the input projection with the conv step fused in: xz[:, :inner] is
        # already the conv output (the conv state advanced), xz[:, inner:] is z
        xz = decode_linear(h, self.input_proj.weight, self.input_proj.bias,
                           conv=(conv_state, conv_w, conv_b, "silu"))                # (batch, 2 * inner)
        out = self._step_tail(xz, ssm_state)
        return out.unsqueeze(1) if squeeze else out

    def step_prenorm(self, hidden_states, residual, norm, conv_state, ssm_state):
        """step() of ``norm(hidden_states, residual=residual, prenorm=True)``'s output
        (the block's RMSNorm in front of it, as CausalLM's blocks apply it): returns
        (out, hidden_states + residual), the second the residual stream the prenorm
        RMSNorm returns (hidden_states itself without residual).  With the norm's
        fast path the RMSNorm runs inside the input projection's launch."""
        squeeze = hidden_states.dim() == 3
        h = hidden_states.reshape(-1, self.model_dim)
        r = residual.reshape(-1, self.model_dim) if residual is not None else None
        *_, conv_w, conv_b = self._decode_params()
        conv = (conv_state, conv_w, conv_b, "silu")
        if norm.use_fast_path and h.is_cuda:
            xz, s = decode_linear(h, self.input_proj.weight, self.input_proj.bias, conv=conv,
                                  norm=(r, norm.weight, norm.eps))
        else:
            normed, s = norm(h, residual=r, prenorm=True)
            xz = decode_linear(normed, self.input_proj.weight, self.input_proj.bias, conv=conv)
        out = self._step_tail(xz, ssm_state)
        if squeeze:
            return out.unsqueeze(1), s.view(hidden_states.shape)
        return out, s.view(hidden_states.shape)

    def _step_tail(self, xz, ssm_state):
        """The step after the input projection and conv: xz (batch, 2 * inner) holds the
        conv output and z; returns the block output (batch, model_dim)."""
        A, D, dt_bias, _, _ = self._decode_params()
        x, z = xz[:, :self.inner_dim], xz[:, self.inner_dim:]
        x_db = decode_linear(x, self.ssm_param_proj.weight)                          # (batch, R + 2N)
        R, N = self.delta_rank, self.state_dim
        # the delta projection (x_db[:, :R] @ W.T) is summed inside the state
        # update; its bias goes in there too
        y = selective_state_update(ssm_state, x, (x_db[:, :R], self.delta_proj.weight), A, x_db[:, R:R + N],
                                   x_db[:, R + N:], D, z=z, dt_bias=dt_bias, dt_softplus=True)
        return decode_linear(y, self.output_proj.weight, self.output_proj.bias)

    def _decode_params(self):
        """A = -exp(log_A), D, the delta bias and the conv weight / bias in fp32, computed
        once and reused by every decode step and no-grad forward until one of those
        parameters changes (their version counters move on any in-place update, an
        optimizer step included).  Parameters created under torch.inference_mode
        carry no version counter, so for them the values are computed on every call."""
        params = [self.log_A, self.D, self.delta_proj.bias, self.short_conv.weight]
        if self.short_conv.bias is not None:
            params.append(self.short_conv.bias)
        if any(p.is_inference() for p in params):
            return self._fp32_params()
        key = tuple((p.data_ptr(), p._version) for p in params)
        cached = getattr(self, "_decode_cache", None)
        if cached is None or cached[0] != key:
            self._decode_cache = (key, self._fp32_params())
            cached = self._decode_cache
        return cached[1]

    def _fp32_params(self):
        with torch.no_grad():
            w = self.short_conv.weight
            return (-torch.exp(self.log_A.float()), self.D.float().contiguous(),
                    self.delta_proj.bias.float().contiguous(),
                    w.reshape(w.shape[0], w.shape[-1]).float().contiguous(),
                    self.short_conv.bias.float().contiguous() if self.short_conv.bias is not None else None)

    def _forward_reference(self, hidden_states):
        # the reference's op sequence (modules/mamba_simple.py:95-149)
        batch_size, seq_len, _ = hidden_states.shape
        state_inputs, gate_logits = torch.chunk(
            self.input_proj(hidden_states).permute(0, 2, 1).contiguous(), chunks=2, dim=1)
        state_inputs = self.act(self.short_conv(state_inputs)[..., :seq_len])
        ssm_params = self.ssm_param_proj(
            state_inputs.permute(0, 2, 1).contiguous().view(batch_size * seq_len, self.inner_dim))
        delta, B, C = torch.split(ssm_params, [self.delta_rank, self.state_dim, self.state_dim], dim=-1)
        delta = self.delta_proj.weight @ delta.t()
        delta = delta.view(self.inner_dim, batch_size, seq_len).permute(1, 0, 2).contiguous()
        B = B.view(batch_size, seq_len, self.state_dim).permute(0, 2, 1).contiguous().unsqueeze(1)
        C = C.view(batch_size, seq_len, self.state_dim).permute(0, 2, 1).contiguous().unsqueeze(1)
        A = -torch.exp(self.log_A.float())
        state_outputs = SelectiveScanFn.apply(state_inputs, delta, A, B, C, self.D.float(),
                                              self.delta_proj.bias.float(), True)
        hidden_states = state_outputs.permute(0, 2, 1).contiguous()
        hidden_states = hidden_states * self.act(gate_logits.permute(0, 2, 1).contiguous())
        return self.output_proj(hidden_states)
