from .causal_lm import Block, CausalLM, CausalLMConfig, GraphedStep

__all__ = ["Block", "CausalLM", "CausalLMConfig", "GraphedStep"]
