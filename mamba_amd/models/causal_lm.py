"""CausalLM with the reference's configuration, structure and parameter names.

Mirrors models/causal_lm.py:7-62 (CausalLMConfig, Block, CausalLM): token
embedding, ``num_layers`` pre-norm residual blocks RMSNorm -> MambaSimple ->
dropout, a final RMSNorm and an lm_head tied to the embedding.  The
state_dict keys are the reference's.  On a ROCm device each block's
residual add is fused into the next RMSNorm kernel (the residual stream is
carried between blocks instead of being added at the end of each one).
``generate`` is a stub in the reference (:61-62); here it decodes with a
per-block state cache (``allocate_inference_cache``, ``step``) on the HIP
state-update kernels.
"""
from dataclasses import dataclass

import torch
import torch.nn as nn

from ..modules import MambaSimple, RMSNorm
from ..ops import decode_linear as decode_linear_ops


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

    def forward(self, input_ids, inference_cache=None):
        """Logits (batch, seqlen, vocab).  With ``inference_cache`` (from
        allocate_inference_cache) every block's decode state is left at the last
        token, so that ``step`` continues the sequence."""
        hidden_states = self.embedding(input_ids)
        if inference_cache is not None:
            residual = None
            for layer, cache in zip(self.layers, inference_cache):
                normed, residual = layer.norm(hidden_states, residual=residual, prenorm=True)
                hidden_states = layer.dropout(layer.mamba(normed, inference_cache=cache))
            return self.lm_head(self.norm(hidden_states, residual=residual))
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

    def allocate_inference_cache(self, batch_size, dtype=None, device=None):
        """One (conv_state, ssm_state) pair per block, zero (no tokens seen yet)."""
        return [layer.mamba.allocate_inference_cache(batch_size, dtype, device) for layer in self.layers]

    def step(self, input_ids, inference_cache):
        """One token per sequence: input_ids (batch,) -> logits (batch, vocab); the
        cache advances in place.  The same function as the last position of
        forward() over the whole sequence."""
        hidden_states = self.embedding(input_ids)
        residual = None
        for layer, (conv_state, ssm_state) in zip(self.layers, inference_cache):
            # normed, residual = layer.norm(hidden_states, residual, prenorm=True), then
            # the block step on normed: one call, the norm inside the input projection
            out, residual = layer.mamba.step_prenorm(hidden_states, residual, layer.norm, conv_state, ssm_state)
            hidden_states = layer.dropout(out)
        return self.lm_head(self.norm(hidden_states, residual=residual))

    @torch.no_grad()
    def generate(self, input_ids, max_new_tokens=50, temperature=1.0, generator=None, use_graph=None):
        """input_ids (batch, seqlen) -> (batch, seqlen + max_new_tokens): the prompt is
        run once (filling the decode cache), then one token at a time is sampled
        from softmax(logits / temperature) (temperature 0: the argmax) and fed back
        through ``step``.  ``use_graph`` (default: on a ROCm device when at least 8
        tokens are generated) replays the step as one captured HIP graph
        (``GraphedStep``).  The reference declares this method without a body
        (models/causal_lm.py:61-62)."""
        if max_new_tokens <= 0:
            return input_ids
        cache = self.allocate_inference_cache(input_ids.shape[0], device=input_ids.device)
        logits = self(input_ids, inference_cache=cache)[:, -1]
        if use_graph is None:
            use_graph = input_ids.is_cuda and max_new_tokens >= 8
        step = GraphedStep(self, cache, input_ids.shape[0]) if use_graph else (lambda ids: self.step(ids, cache))
        tokens = [input_ids]
        for i in range(max_new_tokens):
            if temperature == 0:
                nxt = logits.argmax(-1)
            else:
                probs = torch.softmax(logits.float() / temperature, dim=-1)
                nxt = torch.multinomial(probs, 1, generator=generator)[:, 0]
            tokens.append(nxt[:, None])
            if i + 1 < max_new_tokens:
                logits = step(nxt)
        return torch.cat(tokens, dim=1)


class GraphedStep:
    """``CausalLM.step`` for a fixed batch and cache, captured once into a HIP graph.

    A decode step is four small launches per block (the norm, input
    projection and conv step in one, the x-projection, the state update, the
    output projection); replaying them as one graph removes the host launch
    cost.  Each call copies the token ids into the captured input,
    replays, and returns the captured logits buffer (overwritten by the next
    call).  The cache tensors are the captured ones: keep using the same
    cache object.  Nothing in a step clears memory with a memset, so the
    graph replays correctly any number of times.  The decode linear layers'
    split workspace (tile counters and partial tiles) is the graph's own,
    allocated before the capture, so a replay shares it with no other graph
    and no eager call; replays of one graph must not overlap each other.
    """

    def __init__(self, model, inference_cache, batch_size, warmup=2):
        dev = next(model.parameters()).device
        self.ids = torch.zeros(batch_size, dtype=torch.long, device=dev)
        saved = [(c.clone(), s.clone()) for c, s in inference_cache]
        # warm-up outside the capture (library handles, allocator pools); it
        # advances the cache, which is put back afterwards
        self.workspace = decode_linear_ops.new_workspace(dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad(), decode_linear_ops.private_workspace(self.workspace):
            for _ in range(warmup):
                model.step(self.ids, inference_cache)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side), torch.no_grad(), \
                decode_linear_ops.private_workspace(self.workspace):
            self.logits = model.step(self.ids, inference_cache)
        with torch.no_grad():
            for (c, s), (c0, s0) in zip(inference_cache, saved):
                c.copy_(c0)
                s.copy_(s0)

    def __call__(self, input_ids):
        self.ids.copy_(input_ids)
        self.graph.replay()
        return self.logits
