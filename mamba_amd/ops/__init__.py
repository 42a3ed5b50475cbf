from .selective_scan_interface import SelectiveScanFn, selective_scan_fn

__all__ = ["SelectiveScanFn", "selective_scan_fn"]
