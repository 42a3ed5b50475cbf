"""Deterministic sums of the backward (ss_bwd_args.deterministic).

With the flag, dB and dC are summed over channel blocks and dA, dD and
ddelta_bias over batch rows and sequence segments in a fixed order, so the
backward gives the same bits on every run.  Checked, through the C ABI
(``backward_into``):
* three runs bit-identical in every output, on the serial fast kernel, on
  a group with several dB / dC slices, on the sequence-segmented kernel
  (one long sequence) and on dstate 32 / 64 (one pass of the fast kernel
  per 16-state slice, fixed-order sums in each);
* the results against the float64 oracle (fp32 rtol / atol 1e-3) and
  against the atomic sums to 1e-5 relative (the same sums in another
  order);
* accumulation (zero_grads off) adds the same bits to what the
  accumulators held;
* a HIP graph of the deterministic forward + backward replays bit for bit;
* torch.use_deterministic_algorithms(True) turns it on for autograd
  (selective_scan_fn), and for arguments the fast kernels do not take it
  raises as torch's own ops do, or warns under warn_only.

The causal conv1d backward (ss_conv1d_bwd_args.workspace) likewise: three
runs with the fixed-order dweight / dbias sums bit-identical, equal to the
atomic sums to 1e-5 relative and to float64 autograd of the conv oracle,
accumulating onto what dweight / dbias held; and mamba_inner_fn's gradients
(scan and conv together) bit-identical across runs under
torch.use_deterministic_algorithms(True).
"""
import ctypes
import sys

import pytest
import torch

from oracle.mamba_block_ref import causal_conv1d_ref
from oracle.selective_scan_ref import make_inputs
from tests._util import NAMES, assert_close, oracle_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GRADS = ("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz")


def _say(msg):
    print(f"\n[deterministic] {msg}", flush=True)
    sys.stdout.flush()


def _setup(batch, dim, L, seed, dtype=torch.float32, N=16):
    from mamba_amd import selective_scan as ss
    x = make_inputs(batch, dim, N, L, seed=seed, dtype=dtype)
    t = {k: x[k].to(DEV) for k in NAMES + ("dout",)}
    out, y = torch.empty_like(t["delta"]), torch.empty_like(t["delta"])
    xck = torch.empty((batch, ss.n_chunks(L), dim, N), dtype=torch.float32, device=DEV)
    ss.forward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, out, xck,
                    z=t["z"], y=y)
    return x, t, out, y, xck


def _backward(t, y, xck, det, zero=True, init=None):
    from mamba_amd import selective_scan as ss
    g = {"du": torch.empty_like(t["u"]), "ddelta": torch.empty_like(t["delta"]), "dz": torch.empty_like(t["z"])}
    for k, ref in (("dA", "A"), ("dB", "B"), ("dC", "C"), ("dD", "D"), ("ddelta_bias", "delta_bias")):
        g[k] = (init[k].clone() if init is not None else
                torch.full(t[ref].shape, float("nan"), dtype=torch.float32, device=DEV))
    ss.backward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck, True,
                     g["du"], g["ddelta"], g["dA"], g["dB"], g["dC"], g["dD"], g["ddelta_bias"],
                     z=t["z"], y=y, dz=g["dz"], zero_grads=zero, deterministic=det)
    torch.cuda.synchronize()
    return g


# (batch, dim, seqlen, dstate): serial fast kernel, 2 channel blocks per
# slice group boundary (192 blocks: 192 slices), one long sequence (8
# segments), ragged seqlens (1001: identity-padded tail chunks in slices with
# padded rows; 2064: a wholly padded last chunk); dstate 32 and 64 (state
# slices, one with sequence segments and one ragged)
CASES = [(2, 256, 512, 16), (1, 3072, 256, 16), (1, 256, 4096, 16), (1, 256, 1001, 16), (2, 64, 2064, 16),
         (2, 64, 300, 32), (1, 256, 4096, 32), (1, 32, 1001, 64)]


@pytest.mark.parametrize("case", CASES, ids=["serial", "many-blocks", "segments", "ragged-1001", "ragged-2064",
                                             "n32", "n32-segments", "n64-ragged"])
def test_deterministic_backward_is_reproducible_and_correct(case):
    from mamba_amd import selective_scan as ss
    batch, dim, L, N = case
    _say(f"batch {batch} dim {dim} seqlen {L} dstate {N}")
    x, t, out, y, xck = _setup(batch, dim, L, seed=300 + dim + N, N=N)
    g0 = _backward(t, y, xck, det=True)
    nbytes = ss.workspace_bytes(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck,
                                True, g0["du"], g0["ddelta"], g0["dA"], g0["dB"], g0["dC"], g0["dD"],
                                g0["ddelta_bias"], z=t["z"], y=y, dz=g0["dz"], deterministic=True)
    assert nbytes >= 2 * (dim // 16) * batch * 16 * L * 4       # one dB / dC partial per channel block
    runs = [_backward(t, y, xck, det=True) for _ in range(3)]
    for k in GRADS:
        assert torch.equal(runs[0][k], runs[1][k]) and torch.equal(runs[0][k], runs[2][k]), f"{k} differs between runs"
    atomic = _backward(t, y, xck, det=False)
    for k in GRADS:
        w = atomic[k]
        assert_close(runs[0][k], w, 1e-5, 1e-5 * float(w.abs().max()), f"{k} vs atomic sums")
    if batch * dim * L <= 2 * 256 * 512:
        _, want = oracle_fwd_bwd(x)
        for k in NAMES:
            assert_close(runs[0]["d" + k].cpu(), want[k], 1e-3, 1e-3, f"d{k} vs oracle")
    # accumulation: the same sums added to what the accumulators held
    init = {k: torch.randn(runs[0][k].shape, device=DEV) for k in ("dA", "dB", "dC", "dD", "ddelta_bias")}
    acc = _backward(t, y, xck, det=True, zero=False, init=init)
    for k in init:
        assert torch.equal(acc[k], init[k] + runs[0][k]), k


def test_deterministic_graph_replays_bit_for_bit():
    from mamba_amd import selective_scan as ss
    batch, dim, L = 2, 256, 512
    _say("graph replays of the deterministic step")
    x, t, out, y, xck = _setup(batch, dim, L, seed=321)
    g = _backward(t, y, xck, det=True)
    bargs = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck, True,
             g["du"], g["ddelta"], g["dA"], g["dB"], g["dC"], g["dD"], g["ddelta_bias"])
    ws = torch.empty(ss.workspace_bytes(*bargs, z=t["z"], y=y, dz=g["dz"], deterministic=True),
                     dtype=torch.uint8, device=DEV)

    def step():
        ss.forward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, out, xck,
                        z=t["z"], y=y)
        ss.backward_into(*bargs, z=t["z"], y=y, dz=g["dz"], workspace=ws, zero_grads=True, deterministic=True)

    step()
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in g.items()}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for rep in range(3):
        for v in g.values():
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k in GRADS:
            assert torch.equal(g[k], eager[k]), f"replay {rep}: {k}"
        _ = (t["u"] * 2).sum().item()            # eager work between replays


def test_torch_deterministic_setting_drives_autograd():
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    _say("torch.use_deterministic_algorithms and selective_scan_fn")
    x = make_inputs(2, 256, 16, 512, seed=331)
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    prev = torch.are_deterministic_algorithms_enabled()
    prev_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)

        def grads(xx):
            p = {k: xx[k].to(DEV).requires_grad_(True) for k in names}
            out = selective_scan_fn(p["u"], p["delta"], p["A"], p["B"], p["C"], p["D"], z=p["z"],
                                    delta_bias=p["delta_bias"], delta_softplus=True)
            out.backward(xx["dout"].to(DEV))
            torch.cuda.synchronize()
            return {k: p[k].grad.clone() for k in names}
        a, b = grads(x), grads(x)
        for k in names:
            assert torch.equal(a[k], b[k]), k
        # dstate 24: the general kernel, which has no deterministic sums
        xr = make_inputs(1, 32, 24, 100, seed=332)
        with pytest.raises(RuntimeError, match="deterministic"):
            grads(xr)
        torch.use_deterministic_algorithms(True, warn_only=True)
        with pytest.warns(UserWarning, match="deterministic"):
            grads(xr)
    finally:
        torch.use_deterministic_algorithms(prev, warn_only=prev_warn)


# (batch, dim, seqlen, width, bias, dtype): several sequence tiles per row
# (2048 steps per bf16 workgroup, 1024 fp32), a ragged last tile, width 2
CONV_CASES = [(3, 96, 5000, 4, True, torch.bfloat16), (2, 40, 3001, 2, False, torch.float32),
              (4, 16, 1028, 3, True, torch.float16)]


def _conv_bwd(x, w, b, dout, det, init=None):
    from mamba_amd import _native as nat
    from mamba_amd.ops import causal_conv1d as cc
    from mamba_amd.selective_scan import _ptr, _stream
    if init is None:
        return cc.causal_conv1d_bwd(x, w, b, dout, silu=True, deterministic=det)
    # accumulation: the C ABI adds into dweight / dbias
    lib = nat.load()
    w2, b2 = cc._params32(w, b, x.shape[1], x.device)
    dx = torch.empty_like(x)
    dw, db = init[0].clone(), (init[1].clone() if b is not None else None)
    g = nat.Conv1dBwdArgs()
    g.f = cc._fill(x, w2, b2, True, None)
    g.dout_batch_stride, g.dout_dim_stride = dout.stride(0), dout.stride(1)
    g.dx_batch_stride, g.dx_dim_stride = dx.stride(0), dx.stride(1)
    g.dout, g.dx, g.dweight, g.dbias = _ptr(dout), _ptr(dx), _ptr(dw), _ptr(db)
    ws = torch.empty(lib.ss_conv1d_bwd_workspace_bytes(ctypes.byref(g)) // 4, dtype=torch.float32, device=DEV)
    g.workspace, g.workspace_bytes = _ptr(ws), ws.numel() * 4
    assert lib.ss_conv1d_bwd(ctypes.byref(g), _stream(DEV)) == nat.SS_OK
    torch.cuda.synchronize()
    return dx, dw, db


@pytest.mark.parametrize("case", CONV_CASES, ids=["bf16-w4-bias", "fp32-w2", "fp16-w3-bias"])
def test_conv1d_backward_fixed_order_sums(case):
    batch, dim, L, width, has_bias, dt = case
    _say(f"conv1d backward batch {batch} dim {dim} seqlen {L} width {width} {dt}")
    g = torch.Generator().manual_seed(dim * 7 + L)
    x = torch.randn(batch, dim, L, generator=g).to(dt)
    w = torch.randn(dim, width, generator=g) * 0.5
    b = torch.randn(dim, generator=g) if has_bias else None
    dout = torch.randn(batch, dim, L, generator=g).to(dt)
    xd, wd, dd = x.to(DEV), w.to(DEV), dout.to(DEV)
    bd = b.to(DEV) if b is not None else None
    runs = [_conv_bwd(xd, wd, bd, dd, det=True) for _ in range(3)]
    torch.cuda.synchronize()
    for i, what in ((0, "dx"), (1, "dweight"), (2, "dbias")):
        if runs[0][i] is not None:
            assert torch.equal(runs[0][i], runs[1][i]) and torch.equal(runs[0][i], runs[2][i]), f"{what} differs"
    atomic = _conv_bwd(xd, wd, bd, dd, det=False)
    torch.cuda.synchronize()
    assert torch.equal(runs[0][0], atomic[0])                   # dx has no sums across workgroups
    for i, what in ((1, "dweight"), (2, "dbias")):
        if atomic[i] is not None:
            assert_close(runs[0][i], atomic[i], 1e-5, 1e-5 * float(atomic[i].abs().max()), f"{what} vs atomic")
    xr, wr = x.double(), w.double().requires_grad_(True)
    br = b.double().requires_grad_(True) if b is not None else None
    causal_conv1d_ref(xr, wr, br, activation="silu").backward(dout.double())
    tol = 1e-3 if dt == torch.float32 else 2e-2
    assert_close(runs[0][1].cpu(), wr.grad, tol, tol * max(1.0, float(wr.grad.abs().max())), "dweight vs oracle")
    if b is not None:
        assert_close(runs[0][2].cpu(), br.grad, tol, tol * max(1.0, float(br.grad.abs().max())), "dbias vs oracle")
    init = (torch.randn(dim, width, device=DEV), torch.randn(dim, device=DEV))
    _, dw, db = _conv_bwd(xd, wd, bd, dd, det=True, init=init)
    assert torch.equal(dw, init[0] + runs[0][1])
    if b is not None:
        assert torch.equal(db, init[1] + runs[0][2])


def test_mamba_inner_fn_deterministic_setting():
    from mamba_amd.ops.selective_scan_interface import mamba_inner_fn
    batch, d_model, dim, L, R, N, width = 2, 32, 64, 4104, 4, 16, 4
    _say(f"mamba_inner_fn under torch.use_deterministic_algorithms, seqlen {L}")
    g = torch.Generator().manual_seed(341)
    p = {
        "conv1d_weight": torch.randn(dim, 1, width, generator=g) * 0.3,
        "conv1d_bias": torch.randn(dim, generator=g) * 0.1,
        "x_proj_weight": torch.randn(R + 2 * N, dim, generator=g) * dim ** -0.5,
        "delta_proj_weight": torch.rand(dim, R, generator=g) * R ** -0.5,
        "out_proj_weight": torch.randn(d_model, dim, generator=g) * dim ** -0.5,
        "out_proj_bias": torch.randn(d_model, generator=g) * 0.1,
        "A": -torch.arange(1, N + 1, dtype=torch.float32).repeat(dim, 1),
        "D": torch.ones(dim),
        "delta_bias": torch.log(torch.expm1(torch.rand(dim, generator=g) * 0.099 + 0.001)),
    }
    xz = torch.randn(batch, 2 * dim, L, generator=g).to(torch.bfloat16)
    dres = torch.randn(batch, L, d_model, generator=g).to(torch.bfloat16)
    args = ("conv1d_weight", "conv1d_bias", "x_proj_weight", "delta_proj_weight", "out_proj_weight",
            "out_proj_bias", "A")

    def grads():
        gp = {k: (v.to(torch.bfloat16) if k not in ("A", "D", "delta_bias") else v).to(DEV).requires_grad_(True)
              for k, v in p.items()}
        xzg = xz.to(DEV).requires_grad_(True)
        out = mamba_inner_fn(xzg, *(gp[k] for k in args), D=gp["D"], delta_bias=gp["delta_bias"],
                             delta_softplus=True)
        out.backward(dres.to(DEV))
        torch.cuda.synchronize()
        return {"xz": xzg.grad.clone(), **{k: v.grad.clone() for k, v in gp.items()}}

    prev = torch.are_deterministic_algorithms_enabled()
    prev_warn = torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        a, b = grads(), grads()
    finally:
        torch.use_deterministic_algorithms(prev, warn_only=prev_warn)
    for k in a:
        assert torch.equal(a[k], b[k]), f"d{k} differs between runs"
