from .mamba_simple import MambaSimple
from .rms_norm import RMSNorm

__all__ = ["MambaSimple", "RMSNorm"]
