"""CausalLM with the reference's configuration, structure and parameter names.

Mirrors models/causal_lm.py:7-62 (CausalLMConfig, Block, CausalLM): token
embedding, ``num_layers`` pre-norm residual blocks RMSNorm -> MambaSimple ->
dropout, a final RMSNorm and an lm_head tied to the embedding.  The
state_dict keys are the reference's.  On a ROCm device each block's
residual add is fused into the next RMSNorm kernel (the residual stream is
carried between blocks instead of being added at the end of each one).
``generate`` is a stub in the reference (:61-62) and is not provided here.
"""
from dataclasses import dataclass

import torch.nn as nn

from ..modules import MambaSimple, RMSNorm


@dataclass
class CausalLMConfig:
    vocab_size: int = 32000
    model_dim: int = 512
    state_dim: int = 16
    conv_kernel: int = 4
    expansion_factor: int = 2
    dropout_rate: float = 0.15
    num_layers: int = 5
    tie_embeddings: bool = True


class Block(nn.Module):
    def __init__(self, config: CausalLMConfig, device=None, dtype=None, use_fast_path=True):
        super().__init__()
        self.norm = RMSNorm(config.model_dim, device=device, dtype=dtype)
        self.mamba = MambaSimple(model_dim=config.model_dim, state_dim=config.state_dim,
                                 conv_kernel=config.conv_kernel, expansion_factor=config.expansion_factor,
                                 device=device, dtype=dtype, use_fast_path=use_fast_path)
        self.dropout = nn.Dropout(config.dropout_rate)

    def forward(self, hidden_states):
        residual = hidden_states
        hidden_states = self.norm(hidden_states)
        hidden_states = self.mamba(hidden_states)
        hidden_states = self.dropout(hidden_states)
        return hidden_states + residual


class CausalLM(nn.Module):
    def __init__(self, config: CausalLMConfig, device=None, dtype=None, use_fast_path=True):
        super().__init__()
        self.config = config
        self.embedding = nn.Embedding(config.vocab_size, config.model_dim, device=device, dtype=dtype)
        self.layers = nn.ModuleList([Block(config, device, dtype, use_fast_path) for _ in range(config.num_layers)])
        self.norm = RMSNorm(config.model_dim, device=device, dtype=dtype)
        self.lm_head = nn.Linear(config.model_dim, config.vocab_size, bias=False, device=device, dtype=dtype)
        if config.tie_embeddings:
            self.lm_head.weight = self.embedding.weight

    def _fused_residual(self, hidden_states):
        return hidden_states.is_cuda and self.norm.use_fast_path and all(
            layer.norm.use_fast_path for layer in self.layers)

    def forward(self, input_ids):
        hidden_states = self.embedding(input_ids)
        if self._fused_residual(hidden_states):
            # the same function as the loop below, with each block's residual
            # add moved into the next RMSNorm kernel: block i computes
            # h_{i+1} = dropout(mamba(norm(h_i))) + h_i, and norm(h_{i+1}) is
            # one pass over (dropout(mamba(...)), h_i) that also writes h_{i+1}
            residual = None
            for layer in self.layers:
                normed, residual = layer.norm(hidden_states, residual=residual, prenorm=True)
                hidden_states = layer.dropout(layer.mamba(normed))
            hidden_states = self.norm(hidden_states, residual=residual)
        else:
            for layer in self.layers:
                hidden_states = layer(hidden_states)
            hidden_states = self.norm(hidden_states)
        return self.lm_head(hidden_states)
