"""Drop-in for the reference's native module ``selective_scan``.

The reference builds a pybind extension named ``selective_scan``
(setup.py:10-16, csrc/selective_scan/selective_scan.cpp:331-334) with

    forward(u, delta, A, B, C, D, delta_bias, use_delta_softplus) -> [out, x]
    backward(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus)
        -> [du, ddelta, dA, dB, dC, dD, ddelta_bias]

This module keeps those positional signatures and return lists and runs
them on libmamba_ss.so through its C ABI.  Host-side rules mirror
selective_scan.cpp:184-329: B (or C) with fewer than 3 dims is constant
(dim, dstate) (:194-195); n_groups = B.size(1) (:202); out has delta's
dtype (:206); du / ddelta have the dtypes of u / delta, dA / dD /
ddelta_bias are zero-initialised fp32 accumulators and variable dB / dC are
fp32 (:271-287).  Unlike the reference, inputs are validated, and a fused z
gate is available through the keyword-only ``z`` (forward then also returns
the pre-gate output y, which ``backward`` needs to produce dz).

There is no CPU fallback: tensors must live on a ROCm device and the
library must be built.
"""
import ctypes

import torch

from . import _native as nat

_ITYPES = {torch.float32: nat.SS_F32, torch.bfloat16: nat.SS_BF16, torch.float16: nat.SS_F16}


def chunk_size():
    """Steps per checkpoint of the state h in x."""
    return int(nat.load().ss_chunk_size())


def n_chunks(seqlen):
    cs = chunk_size()
    return (seqlen + cs - 1) // cs


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require(cond, msg):
    if not cond:
        raise ValueError(f"selective_scan: {msg}")


def _check_seq_tensor(name, t, shape, itype_dtype, device):
    _require(t.device == device, f"{name} is on {t.device}, expected {device}")
    _require(tuple(t.shape) == tuple(shape), f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    _require(t.dtype == itype_dtype, f"{name} has dtype {t.dtype}, expected {itype_dtype}")
    _require(t.shape[-1] <= 1 or t.stride(-1) == 1, f"{name} must have unit stride along seqlen")


def _fill_fwd_args(u, delta, A, B, C, D, delta_bias, delta_softplus, z, out, x, y):
    _require(u.dim() == 3, f"u must be (batch, dim, seqlen), got shape {tuple(u.shape)}")
    device = u.device
    _require(device.type == "cuda", "tensors must be on a ROCm GPU device (no CPU path)")
    _require(u.dtype in _ITYPES, f"unsupported dtype {u.dtype}")
    itype = u.dtype
    batch, dim, seqlen = u.shape
    _check_seq_tensor("delta", delta, u.shape, itype, device)
    _require(A.dim() == 2 and A.shape[0] == dim, f"A must be (dim, dstate), got {tuple(A.shape)}")
    _require(A.dtype == torch.float32 and A.device == device, "A must be fp32 on the same device")
    dstate = A.shape[1]
    var_B, var_C = B.dim() >= 3, C.dim() >= 3
    n_groups = B.shape[1] if var_B else (C.shape[1] if var_C else 1)
    for name, M, var in (("B", B, var_B), ("C", C, var_C)):
        _require(M.device == device, f"{name} is on {M.device}, expected {device}")
        if var:
            _require(M.dim() == 4 and M.shape[0] == batch and M.shape[1] == n_groups
                     and M.shape[2] == dstate and M.shape[3] == seqlen,
                     f"{name} must be (batch, n_groups, dstate, seqlen), got {tuple(M.shape)}")
            _require(M.dtype == itype, f"{name} has dtype {M.dtype}, expected {itype}")
            _require(seqlen <= 1 or M.stride(3) == 1, f"{name} must have unit stride along seqlen")
        else:
            _require(M.dim() == 2 and tuple(M.shape) == (dim, dstate),
                     f"constant {name} must be (dim, dstate), got {tuple(M.shape)}")
            _require(M.dtype == torch.float32, f"constant {name} must be fp32")
    for name, v in (("D", D), ("delta_bias", delta_bias)):
        if v is not None:
            _require(v.shape == (dim,) and v.dtype == torch.float32 and v.device == device
                     and v.is_contiguous(), f"{name} must be a contiguous fp32 ({dim},) tensor")
    if z is not None:
        _check_seq_tensor("z", z, u.shape, itype, device)
    a = nat.FwdArgs()
    a.batch, a.dim, a.seqlen, a.dstate, a.n_groups = batch, dim, seqlen, dstate, n_groups
    a.itype = _ITYPES[itype]
    a.is_var_B, a.is_var_C = int(var_B), int(var_C)
    a.has_D, a.has_delta_bias, a.has_z = int(D is not None), int(delta_bias is not None), int(z is not None)
    a.delta_softplus = int(bool(delta_softplus))
    a.n_chunks = n_chunks(seqlen)
    a.u_batch_stride, a.u_dim_stride = u.stride(0), u.stride(1)
    a.delta_batch_stride, a.delta_dim_stride = delta.stride(0), delta.stride(1)
    if z is not None:
        a.z_batch_stride, a.z_dim_stride = z.stride(0), z.stride(1)
    if out is not None:
        a.out_batch_stride, a.out_dim_stride = out.stride(0), out.stride(1)
    if y is not None:
        a.y_batch_stride, a.y_dim_stride = y.stride(0), y.stride(1)
    a.A_dim_stride, a.A_dstate_stride = A.stride(0), A.stride(1)
    if var_B:
        a.B_batch_stride, a.B_group_stride, a.B_dstate_stride = B.stride(0), B.stride(1), B.stride(2)
    else:
        a.B_batch_stride, a.B_group_stride, a.B_dstate_stride = 0, B.stride(0), B.stride(1)
    if var_C:
        a.C_batch_stride, a.C_group_stride, a.C_dstate_stride = C.stride(0), C.stride(1), C.stride(2)
    else:
        a.C_batch_stride, a.C_group_stride, a.C_dstate_stride = 0, C.stride(0), C.stride(1)
    a.u, a.delta, a.A, a.B, a.C = _ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C)
    a.D, a.delta_bias, a.z = _ptr(D), _ptr(delta_bias), _ptr(z)
    a.out, a.x, a.y = _ptr(out), _ptr(x), _ptr(y)
    return a


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _fwd_into_args(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, z, y, last_state=None):
    _require(out is not None, "out is required")
    _check_seq_tensor("out", out, u.shape, delta.dtype, u.device)
    batch, dim, seqlen = u.shape
    if x is not None:
        _require(x.dtype == torch.float32 and x.is_contiguous() and x.device == u.device
                 and tuple(x.shape) == (batch, n_chunks(seqlen), dim, A.shape[1]),
                 "x must be a contiguous fp32 (batch, n_chunks, dim, dstate) tensor")
    if y is not None:
        _check_seq_tensor("y", y, u.shape, delta.dtype, u.device)
    if last_state is not None:
        _require(last_state.dtype == torch.float32 and last_state.is_contiguous() and last_state.device == u.device
                 and tuple(last_state.shape) == (batch, dim, A.shape[1]),
                 "last_state must be a contiguous fp32 (batch, dim, dstate) tensor")
    a = _fill_fwd_args(u, delta, A, B, C, D, delta_bias, use_delta_softplus, z, out, x, y)
    a.last_state = _ptr(last_state)
    return a


def _attach_fwd_workspace(lib, a, workspace, device):
    """Sets the forward's optional workspace: "auto" allocates what the library
    asks for (torch's caching allocator; none for most shapes), a tensor is
    used as given, None runs the serial scan.  Returns the tensor to keep."""
    if isinstance(workspace, str):
        _require(workspace == "auto", f"workspace must be 'auto', None or a tensor, got {workspace!r}")
        n = int(lib.ss_fwd_workspace_bytes(ctypes.byref(a)))
        if n < 0:
            nat.check(nat.SS_ERR_INVALID, "selective_scan.forward")
        workspace = torch.empty(n, dtype=torch.uint8, device=device) if n > 0 else None
    if workspace is not None:
        _require(workspace.is_cuda and workspace.is_contiguous(), "workspace must be a contiguous GPU tensor")
        a.workspace, a.workspace_bytes = _ptr(workspace), workspace.numel() * workspace.element_size()
    return workspace


def forward_into(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, *, z=None, y=None,
                 last_state=None, workspace="auto"):
    """Forward into caller-allocated ``out`` (delta's dtype), ``x`` (fp32
    (batch, n_chunks, dim, dstate) contiguous) and, with ``z``, ``y``.

    ``x`` and ``y`` are what the backward needs; either may be None for a
    forward that no backward follows (they are then not written at all).
    ``last_state`` (fp32 (batch, dim, dstate), optional) receives the state
    after the last step.  ``workspace`` ("auto", a tensor or None) lets a
    forward with few (batch, channel) rows scan sequence segments in
    parallel (see ``forward_workspace_bytes``)."""
    lib = nat.load()
    a = _fwd_into_args(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, z, y, last_state)
    ws = _attach_fwd_workspace(lib, a, workspace, u.device)
    with torch.cuda.device(u.device):
        nat.check(lib.ss_fwd(ctypes.byref(a), _stream(u.device)), "selective_scan.forward")
    del ws   # the caching allocator keeps it valid for the work queued on this stream


def forward_workspace_bytes(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, *, z=None, y=None):
    """Bytes of scratch ``forward_into`` can use for these tensors (0: none;
    nonzero when the batch has too few channel rows to fill the GPU and the
    sequence is long enough to cut into segments)."""
    lib = nat.load()
    a = _fwd_into_args(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, z, y)
    n = lib.ss_fwd_workspace_bytes(ctypes.byref(a))
    if n < 0:
        nat.check(nat.SS_ERR_INVALID, "selective_scan.forward_workspace_bytes")
    return int(n)


def prepare_forward(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, *, z=None, y=None,
                    last_state=None, workspace="auto"):
    """Validates the arguments of ``forward_into`` once and returns a callable
    that launches the same forward again, on the stream that is current now,
    with no host-side work beyond the C call (the tensors must stay alive
    and keep their storage).  For repeated launches over fixed buffers."""
    lib = nat.load()
    a = _fwd_into_args(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, z, y, last_state)
    ws = _attach_fwd_workspace(lib, a, workspace, u.device)
    dev = u.device
    stream = torch.cuda.current_stream(dev)
    handle = ctypes.c_void_p(stream.cuda_stream)
    ref = ctypes.byref(a)

    def launch():
        nat.check(lib.ss_fwd(ref, handle), "selective_scan.forward")
    launch.args = a
    launch.workspace = ws
    return launch


def forward_kernel_name(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, *, z=None, y=None):
    """Base name of the kernel ``forward_into`` launches for these tensors
    ("" when there is no work).  No device work."""
    lib = nat.load()
    a = _fwd_into_args(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, z, y)
    name = lib.ss_fwd_kernel_name(ctypes.byref(a))
    if name is None:
        nat.check(nat.SS_ERR_INVALID, "selective_scan.forward_kernel_name")
    return name.decode()


def forward(u, delta, A, B, C, D=None, delta_bias=None, use_delta_softplus=True, *, z=None):
    """selective_scan.forward (selective_scan.cpp:184-244).

    Returns [out, x]; with ``z`` given, [out, x, y] where out = y * silu(z)
    and y is the pre-gate output saved for ``backward``.
    """
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    out = torch.empty_like(delta, memory_format=torch.contiguous_format)
    x = torch.empty((batch, n_chunks(seqlen), dim, dstate), dtype=torch.float32, device=u.device)
    y = torch.empty_like(out) if z is not None else None
    forward_into(u, delta, A, B, C, D, delta_bias, use_delta_softplus, out, x, z=z, y=y)
    return [out, x] if z is None else [out, x, y]


def _bwd_into_args(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                   du, ddelta, dA, dB, dC, dD, ddelta_bias, z, y, dz):
    _require(x is not None, "x (the forward's checkpoints) is required")
    _require(z is None or (y is not None and dz is not None), "y from the forward and dz are required with z")
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    _require(x.dtype == torch.float32 and tuple(x.shape) == (batch, n_chunks(seqlen), dim, dstate)
             and x.is_contiguous() and x.device == u.device, "x does not come from forward")
    _check_seq_tensor("dout", dout, u.shape, delta.dtype, u.device)
    _check_seq_tensor("du", du, u.shape, u.dtype, u.device)
    _check_seq_tensor("ddelta", ddelta, u.shape, delta.dtype, u.device)
    if y is not None:
        _check_seq_tensor("y", y, u.shape, delta.dtype, u.device)
    if dz is not None:
        _check_seq_tensor("dz", dz, u.shape, delta.dtype, u.device)
    for name, g, ref in (("dA", dA, A), ("dB", dB, B), ("dC", dC, C), ("dD", dD, D),
                         ("ddelta_bias", ddelta_bias, delta_bias)):
        if ref is None:
            continue
        _require(g is not None and g.dtype == torch.float32 and g.is_contiguous()
                 and tuple(g.shape) == tuple(ref.shape) and g.device == u.device,
                 f"{name} must be a contiguous fp32 tensor of shape {tuple(ref.shape)}")
    b = nat.BwdArgs()
    b.f = _fill_fwd_args(u, delta, A, B, C, D, delta_bias, use_delta_softplus, z, None, x, y)
    b.dout_batch_stride, b.dout_dim_stride = dout.stride(0), dout.stride(1)
    b.du_batch_stride, b.du_dim_stride = du.stride(0), du.stride(1)
    b.ddelta_batch_stride, b.ddelta_dim_stride = ddelta.stride(0), ddelta.stride(1)
    if dz is not None:
        b.dz_batch_stride, b.dz_dim_stride = dz.stride(0), dz.stride(1)
    b.dout, b.du, b.ddelta, b.dz = _ptr(dout), _ptr(du), _ptr(ddelta), _ptr(dz)
    b.dA, b.dB, b.dC, b.dD, b.ddelta_bias = _ptr(dA), _ptr(dB), _ptr(dC), _ptr(dD), _ptr(ddelta_bias)
    return b


def workspace_bytes(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                    du, ddelta, dA, dB, dC, dD, ddelta_bias, *, z=None, y=None, dz=None, deterministic=None):
    """Bytes of scratch ``backward_into`` can use for these tensors (0: none)."""
    lib = nat.load()
    b = _bwd_into_args(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                       du, ddelta, dA, dB, dC, dD, ddelta_bias, z, y, dz)
    _set_deterministic(lib, b, deterministic)
    n = lib.ss_bwd_workspace_bytes(ctypes.byref(b))
    if n < 0:
        nat.check(nat.SS_ERR_INVALID, "selective_scan.workspace_bytes")
    return int(n)


def _set_deterministic(lib, b, flag, workspace="auto"):
    """Sets b.deterministic: the flag, or with None torch.use_deterministic_algorithms.
    An explicit request the kernels cannot honour raises (from the library);
    one that comes from torch's setting raises as torch's own ops do, or
    warns and runs with atomic sums under warn_only.  The deterministic sums
    need a workspace: a call made with ``workspace=None`` cannot have them."""
    if flag is not None:
        b.deterministic = int(bool(flag))
        return
    b.deterministic = int(torch.are_deterministic_algorithms_enabled())
    if not b.deterministic:
        return
    msg = None
    if lib.ss_bwd_workspace_bytes(ctypes.byref(b)) < 0:
        msg = ("selective_scan.backward has no deterministic implementation for these arguments: "
               + lib.ss_last_error().decode())
    elif workspace is None:
        msg = ("selective_scan.backward: the deterministic sums need a workspace, and this call passes "
               "workspace=None")
    if msg is not None:
        if not torch.is_deterministic_algorithms_warn_only_enabled():
            raise RuntimeError(msg)
        import warnings
        warnings.warn(msg)
        b.deterministic = 0


def backward_into(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                  du, ddelta, dA, dB, dC, dD, ddelta_bias, *, z=None, y=None, dz=None, workspace="auto",
                  zero_grads=False, deterministic=None):
    """Backward into caller-allocated gradients.  du, ddelta (and dz) are
    overwritten; dA, dB, dC, dD, ddelta_bias are fp32 and accumulated into,
    or, with ``zero_grads``, cleared by the library first (their contents on
    entry are ignored, so ``torch.empty`` buffers will do).

    ``workspace``: "auto" allocates the scratch the library asks for (see
    ``workspace_bytes``) from torch's caching allocator; a uint8 / any CUDA
    tensor is used as given; None runs without one (same results).

    ``deterministic``: sum dB, dC, dA, dD and ddelta_bias in a fixed order
    (the same bits on every run; needs the fast kernels and a workspace);
    None follows ``torch.use_deterministic_algorithms``.
    """
    lib = nat.load()
    b = _bwd_into_args(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                       du, ddelta, dA, dB, dC, dD, ddelta_bias, z, y, dz)
    _set_deterministic(lib, b, deterministic, workspace)
    if isinstance(workspace, str):
        _require(workspace == "auto", f"workspace must be 'auto', None or a tensor, got {workspace!r}")
        n = lib.ss_bwd_workspace_bytes(ctypes.byref(b))
        if n < 0:
            nat.check(nat.SS_ERR_INVALID, "selective_scan.backward")
        workspace = torch.empty(n, dtype=torch.uint8, device=u.device) if n > 0 else None
    if workspace is not None:
        _require(workspace.device == u.device and workspace.is_contiguous(),
                 "workspace must be a contiguous tensor on the inputs' device")
        b.workspace = _ptr(workspace)
        b.workspace_bytes = workspace.numel() * workspace.element_size()
    b.zero_grads = int(bool(zero_grads))
    with torch.cuda.device(u.device):
        nat.check(lib.ss_bwd(ctypes.byref(b), _stream(u.device)), "selective_scan.backward")


def prepare_backward(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                     du, ddelta, dA, dB, dC, dD, ddelta_bias, *, z=None, y=None, dz=None, workspace="auto",
                     zero_grads=False, deterministic=None):
    """``backward_into`` validated once, as a callable that relaunches it on
    the stream that is current now (see ``prepare_forward``); the workspace,
    if any, is allocated here and kept by the callable."""
    lib = nat.load()
    b = _bwd_into_args(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                       du, ddelta, dA, dB, dC, dD, ddelta_bias, z, y, dz)
    _set_deterministic(lib, b, deterministic, workspace)
    if isinstance(workspace, str):
        _require(workspace == "auto", f"workspace must be 'auto', None or a tensor, got {workspace!r}")
        n = lib.ss_bwd_workspace_bytes(ctypes.byref(b))
        if n < 0:
            nat.check(nat.SS_ERR_INVALID, "selective_scan.backward")
        workspace = torch.empty(n, dtype=torch.uint8, device=u.device) if n > 0 else None
    if workspace is not None:
        _require(workspace.device == u.device and workspace.is_contiguous(),
                 "workspace must be a contiguous tensor on the inputs' device")
        b.workspace = _ptr(workspace)
        b.workspace_bytes = workspace.numel() * workspace.element_size()
    b.zero_grads = int(bool(zero_grads))
    stream = torch.cuda.current_stream(u.device)
    handle = ctypes.c_void_p(stream.cuda_stream)
    ref = ctypes.byref(b)

    def launch():
        nat.check(lib.ss_bwd(ref, handle), "selective_scan.backward")
    launch.args = b
    launch.workspace = workspace
    return launch


def backward_kernel_name(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                         du, ddelta, dA, dB, dC, dD, ddelta_bias, *, z=None, y=None, dz=None):
    """Base name of the kernel ``backward_into`` launches for these tensors
    ("" when there is no work).  No device work."""
    lib = nat.load()
    b = _bwd_into_args(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                       du, ddelta, dA, dB, dC, dD, ddelta_bias, z, y, dz)
    name = lib.ss_bwd_kernel_name(ctypes.byref(b))
    if name is None:
        nat.check(nat.SS_ERR_INVALID, "selective_scan.backward_kernel_name")
    return name.decode()


def backward(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus, *, z=None, y=None):
    """selective_scan.backward (selective_scan.cpp:246-329).

    Returns [du, ddelta, dA, dB, dC, dD, ddelta_bias]; with ``z`` (and the
    forward's ``y``) also dz as an eighth entry.
    """
    du = torch.empty_like(u, memory_format=torch.contiguous_format)
    ddelta = torch.empty_like(delta, memory_format=torch.contiguous_format)
    # the accumulators are cleared by the library in the launch that clears
    # its workspace (zero_grads), not by separate torch fills
    dA = torch.empty(A.shape, dtype=torch.float32, device=A.device)
    dB = torch.empty(B.shape, dtype=torch.float32, device=B.device)
    dC = torch.empty(C.shape, dtype=torch.float32, device=C.device)
    dD = torch.empty(D.shape, dtype=torch.float32, device=D.device) if D is not None else None
    ddelta_bias = (torch.empty(delta_bias.shape, dtype=torch.float32, device=delta_bias.device)
                   if delta_bias is not None else None)
    dz = torch.empty_like(z, memory_format=torch.contiguous_format) if z is not None else None
    backward_into(u, delta, A, B, C, D, delta_bias, dout, x, use_delta_softplus,
                  du, ddelta, dA, dB, dC, dD, ddelta_bias, z=z, y=y, dz=dz, zero_grads=True)
    res = [du, ddelta, dA, dB, dC, dD, ddelta_bias]
    if z is not None:
        res.append(dz)
    return res
