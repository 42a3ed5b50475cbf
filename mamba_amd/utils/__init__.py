from .tensor_utils import ensure_contiguous

__all__ = ["ensure_contiguous"]
