"""ctypes binding of libmamba_ss.so (declared in include/mamba_ss.h).

The library is loaded lazily from ``mamba_amd/_lib/libmamba_ss.so``.  There
is no fallback: if the library is missing or the tensors are not on a ROCm
device, the call raises.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libmamba_ss.so")

SS_F32, SS_BF16, SS_F16 = 0, 1, 2
SS_OK, SS_ERR_INVALID, SS_ERR_UNSUPPORTED, SS_ERR_HIP = 0, 1, 2, 3
ABI_VERSION = 16
# bytes of the fixed device scratch of ss_bwd_noalloc (SS_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 32 << 20

EXPORTED = (
    "ss_abi_version", "ss_chunk_size", "ss_max_dstate", "ss_struct_sizes",
    "ss_last_error", "ss_fwd_check", "ss_bwd_check", "ss_bwd_workspace_bytes", "ss_fwd_workspace_bytes",
    "ss_fwd_kernel_name", "ss_bwd_kernel_name",
    "ss_fwd", "ss_bwd", "ss_bwd_noalloc", "ss_conv1d_fwd", "ss_conv1d_bwd",
    "ss_rmsnorm_fwd", "ss_rmsnorm_bwd", "ss_rmsnorm_bwd_workspace_bytes",
    "ss_state_update", "ss_conv1d_update", "ss_decode_linear", "ss_decode_linear_workspace_bytes",
    "ss_conv1d_bwd_workspace_bytes",
)

_i64, _i32, _p = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("dim", _i64), ("seqlen", _i64), ("dstate", _i64), ("n_groups", _i64),
        ("itype", _i32), ("is_var_B", _i32), ("is_var_C", _i32),
        ("has_D", _i32), ("has_delta_bias", _i32), ("has_z", _i32), ("delta_softplus", _i32),
        ("n_chunks", _i64),
        ("u_batch_stride", _i64), ("u_dim_stride", _i64),
        ("delta_batch_stride", _i64), ("delta_dim_stride", _i64),
        ("z_batch_stride", _i64), ("z_dim_stride", _i64),
        ("out_batch_stride", _i64), ("out_dim_stride", _i64),
        ("A_dim_stride", _i64), ("A_dstate_stride", _i64),
        ("B_batch_stride", _i64), ("B_group_stride", _i64), ("B_dstate_stride", _i64),
        ("C_batch_stride", _i64), ("C_group_stride", _i64), ("C_dstate_stride", _i64),
        ("u", _p), ("delta", _p), ("A", _p), ("B", _p), ("C", _p),
        ("D", _p), ("delta_bias", _p), ("z", _p), ("out", _p), ("x", _p),
        ("y", _p), ("y_batch_stride", _i64), ("y_dim_stride", _i64),
        ("last_state", _p), ("workspace", _p), ("workspace_bytes", _i64),
        ("x_window_bytes", _i64),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("f", FwdArgs),
        ("dout_batch_stride", _i64), ("dout_dim_stride", _i64),
        ("du_batch_stride", _i64), ("du_dim_stride", _i64),
        ("ddelta_batch_stride", _i64), ("ddelta_dim_stride", _i64),
        ("dz_batch_stride", _i64), ("dz_dim_stride", _i64),
        ("dout", _p), ("du", _p), ("ddelta", _p), ("dz", _p),
        ("dA", _p), ("dB", _p), ("dC", _p), ("dD", _p), ("ddelta_bias", _p),
        ("workspace", _p), ("workspace_bytes", _i64),
        ("zero_grads", _i32), ("deterministic", _i32),
    ]


class Conv1dArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("dim", _i64), ("seqlen", _i64), ("width", _i64),
        ("itype", _i32), ("has_bias", _i32), ("silu", _i32), ("pad_", _i32),
        ("x_batch_stride", _i64), ("x_dim_stride", _i64),
        ("out_batch_stride", _i64), ("out_dim_stride", _i64),
        ("w_dim_stride", _i64), ("w_width_stride", _i64),
        ("x", _p), ("weight", _p), ("bias", _p), ("out", _p),
    ]


class Conv1dBwdArgs(ctypes.Structure):
    _fields_ = [
        ("f", Conv1dArgs),
        ("dout_batch_stride", _i64), ("dout_dim_stride", _i64),
        ("dx_batch_stride", _i64), ("dx_dim_stride", _i64),
        ("dout", _p), ("dx", _p), ("dweight", _p), ("dbias", _p),
        ("workspace", _p), ("workspace_bytes", _i64),
    ]


class RmsNormArgs(ctypes.Structure):
    _fields_ = [
        ("rows", _i64), ("dim", _i64),
        ("dtype", _i32), ("w_dtype", _i32), ("eps", ctypes.c_float), ("pad_", _i32),
        ("x_row_stride", _i64), ("residual_row_stride", _i64),
        ("out_row_stride", _i64), ("residual_out_row_stride", _i64),
        ("x", _p), ("residual", _p), ("weight", _p), ("out", _p), ("residual_out", _p), ("rstd", _p),
    ]


class RmsNormBwdArgs(ctypes.Structure):
    _fields_ = [
        ("rows", _i64), ("dim", _i64),
        ("dtype", _i32), ("w_dtype", _i32),
        ("s_row_stride", _i64), ("dout_row_stride", _i64),
        ("dresidual_out_row_stride", _i64), ("dx_row_stride", _i64),
        ("s", _p), ("weight", _p), ("rstd", _p), ("dout", _p), ("dresidual_out", _p),
        ("dx", _p), ("dweight", _p), ("workspace", _p), ("workspace_bytes", _i64),
    ]


class StateUpdateArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("dim", _i64), ("dstate", _i64), ("n_groups", _i64),
        ("itype", _i32), ("has_D", _i32), ("has_z", _i32), ("has_delta_bias", _i32),
        ("delta_softplus", _i32), ("pad_", _i32),
        ("state_batch_stride", _i64), ("state_dim_stride", _i64), ("state_dstate_stride", _i64),
        ("x_batch_stride", _i64), ("x_dim_stride", _i64),
        ("delta_batch_stride", _i64), ("delta_dim_stride", _i64),
        ("z_batch_stride", _i64), ("z_dim_stride", _i64),
        ("out_batch_stride", _i64), ("out_dim_stride", _i64),
        ("A_dim_stride", _i64), ("A_dstate_stride", _i64),
        ("B_batch_stride", _i64), ("B_group_stride", _i64), ("B_dstate_stride", _i64),
        ("C_batch_stride", _i64), ("C_group_stride", _i64), ("C_dstate_stride", _i64),
        ("state", _p), ("x", _p), ("delta", _p), ("A", _p), ("B", _p), ("C", _p),
        ("D", _p), ("z", _p), ("delta_bias", _p), ("out", _p),
        ("delta_rank", _i64), ("delta_low_batch_stride", _i64), ("delta_low_rank_stride", _i64),
        ("delta_weight_dim_stride", _i64), ("delta_weight_rank_stride", _i64),
        ("delta_low", _p), ("delta_weight", _p),
    ]


class Conv1dUpdateArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("dim", _i64), ("width", _i64),
        ("itype", _i32), ("has_bias", _i32), ("silu", _i32), ("pad_", _i32),
        ("x_batch_stride", _i64), ("x_dim_stride", _i64),
        ("out_batch_stride", _i64), ("out_dim_stride", _i64),
        ("state_batch_stride", _i64), ("state_dim_stride", _i64), ("state_width_stride", _i64),
        ("w_dim_stride", _i64), ("w_width_stride", _i64),
        ("x", _p), ("conv_state", _p), ("weight", _p), ("bias", _p), ("out", _p),
    ]


class DecodeLinearArgs(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("n_out", _i64), ("k_in", _i64),
        ("dtype", _i32), ("bias_dtype", _i32),
        ("x_row_stride", _i64), ("w_row_stride", _i64), ("y_row_stride", _i64),
        ("x", _p), ("weight", _p), ("bias", _p), ("y", _p),
        ("workspace", _p), ("workspace_bytes", _i64), ("conv", ctypes.POINTER(Conv1dUpdateArgs)),
        ("norm", ctypes.POINTER(RmsNormArgs)),
    ]


_lib = None
_lock = threading.Lock()


def load():
    """Loads and type-annotates the library; raises if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"mamba_amd: HIP library not built ({LIB_PATH} missing); "
                "run `python -m mamba_amd.build` or __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        lib.ss_abi_version.restype = ctypes.c_int
        lib.ss_chunk_size.restype = _i64
        lib.ss_max_dstate.restype = _i64
        lib.ss_struct_sizes.argtypes = [ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
        lib.ss_struct_sizes.restype = None
        lib.ss_last_error.restype = ctypes.c_char_p
        for name, T in (("ss_fwd_check", FwdArgs), ("ss_bwd_check", BwdArgs)):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.POINTER(T)]
            fn.restype = ctypes.c_int
        for name, T in (("ss_fwd_kernel_name", FwdArgs), ("ss_bwd_kernel_name", BwdArgs)):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.POINTER(T)]
            fn.restype = ctypes.c_char_p
        lib.ss_conv1d_fwd.argtypes = [ctypes.POINTER(Conv1dArgs), _p]
        lib.ss_conv1d_fwd.restype = ctypes.c_int
        lib.ss_conv1d_bwd.argtypes = [ctypes.POINTER(Conv1dBwdArgs), _p]
        lib.ss_conv1d_bwd.restype = ctypes.c_int
        lib.ss_conv1d_bwd_workspace_bytes.argtypes = [ctypes.POINTER(Conv1dBwdArgs)]
        lib.ss_conv1d_bwd_workspace_bytes.restype = _i64
        lib.ss_decode_linear.argtypes = [ctypes.POINTER(DecodeLinearArgs), _p]
        lib.ss_decode_linear.restype = ctypes.c_int
        lib.ss_decode_linear_workspace_bytes.argtypes = [ctypes.POINTER(DecodeLinearArgs)]
        lib.ss_decode_linear_workspace_bytes.restype = _i64
        lib.ss_state_update.argtypes = [ctypes.POINTER(StateUpdateArgs), _p]
        lib.ss_state_update.restype = ctypes.c_int
        lib.ss_conv1d_update.argtypes = [ctypes.POINTER(Conv1dUpdateArgs), _p]
        lib.ss_conv1d_update.restype = ctypes.c_int
        lib.ss_rmsnorm_fwd.argtypes = [ctypes.POINTER(RmsNormArgs), _p]
        lib.ss_rmsnorm_fwd.restype = ctypes.c_int
        lib.ss_rmsnorm_bwd.argtypes = [ctypes.POINTER(RmsNormBwdArgs), _p]
        lib.ss_rmsnorm_bwd.restype = ctypes.c_int
        lib.ss_rmsnorm_bwd_workspace_bytes.argtypes = [_i64, _i64]
        lib.ss_rmsnorm_bwd_workspace_bytes.restype = _i64
        lib.ss_fwd_workspace_bytes.argtypes = [ctypes.POINTER(FwdArgs)]
        lib.ss_fwd_workspace_bytes.restype = _i64
        lib.ss_bwd_workspace_bytes.argtypes = [ctypes.POINTER(BwdArgs)]
        lib.ss_bwd_workspace_bytes.restype = _i64
        lib.ss_fwd.argtypes = [ctypes.POINTER(FwdArgs), _p]
        lib.ss_fwd.restype = ctypes.c_int
        lib.ss_bwd.argtypes = [ctypes.POINTER(BwdArgs), _p]
        lib.ss_bwd.restype = ctypes.c_int
        lib.ss_bwd_noalloc.argtypes = [ctypes.POINTER(BwdArgs), _p]
        lib.ss_bwd_noalloc.restype = ctypes.c_int
        if lib.ss_abi_version() != ABI_VERSION:
            raise RuntimeError(f"mamba_amd: library ABI {lib.ss_abi_version()} != binding ABI {ABI_VERSION}")
        fs, bs = _i64(), _i64()
        lib.ss_struct_sizes(ctypes.byref(fs), ctypes.byref(bs))
        if fs.value != ctypes.sizeof(FwdArgs) or bs.value != ctypes.sizeof(BwdArgs):
            raise RuntimeError("mamba_amd: ctypes struct layout does not match the library")
        _lib = lib
    return _lib


def check(rc, what):
    """Maps a status code to an exception carrying ss_last_error()."""
    if rc == SS_OK:
        return
    msg = load().ss_last_error().decode(errors="replace")
    if rc in (SS_ERR_INVALID, SS_ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")
