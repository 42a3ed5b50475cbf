"""Tensor helpers (mirrors utils/tensor_utils.py:3-6 of the reference)."""
import torch


def ensure_contiguous(x: torch.Tensor | None):
    """Returns x unchanged when it is None or contiguous, else a contiguous copy."""
    if x is None or x.is_contiguous():
        return x
    return x.contiguous()
