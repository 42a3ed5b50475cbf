from .causal_lm import Block, CausalLM, CausalLMConfig

__all__ = ["Block", "CausalLM", "CausalLMConfig"]
