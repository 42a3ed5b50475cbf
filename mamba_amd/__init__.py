"""MI355X-native selective scan for Mamba.

The hot path (selective-scan forward and backward) runs in hand-written
gfx950 HIP kernels in ``_lib/libmamba_ss.so``, reached through the C ABI of
``include/mamba_ss.h``.  Python API:

* ``mamba_amd.selective_scan`` -- drop-in for the reference's native module
  ``selective_scan`` (``forward`` / ``backward``);
* ``mamba_amd.ops.selective_scan_interface`` -- ``SelectiveScanFn`` (the
  reference's autograd function) and ``selective_scan_fn`` (fused z gate,
  ``return_last_state``).
"""
from . import selective_scan
from .ops.selective_scan_interface import SelectiveScanFn, selective_scan_fn

__all__ = ["selective_scan", "SelectiveScanFn", "selective_scan_fn"]
