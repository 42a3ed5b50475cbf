"""GPU parity: HIP selective scan vs the fp64 oracle (outputs and gradients).

Tolerances (stated by the task for this path): fp32 rtol 1e-3 / atol 1e-3,
bf16 and fp16 rtol 2e-2 / atol 2e-2, elementwise against the float64 oracle
evaluated on the same (already rounded) inputs.
"""
import sys

import pytest
import torch

from oracle.selective_scan_ref import make_inputs
from tests._util import NAMES, assert_close, oracle_fwd_bwd

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-3, 1e-3), torch.bfloat16: (2e-2, 2e-2), torch.float16: (2e-2, 2e-2)}

# (batch, dim, dstate, seqlen, dtype, n_groups, var_B, var_C, has_z, has_D, has_bias, softplus)
CASES = [
    (2, 64, 16, 256, torch.float32, 1, True, True, True, True, True, True),     # benchmark distributions, small
    (2, 64, 16, 256, torch.float32, 1, True, True, False, True, True, True),    # reference surface (no z)
    (1, 16, 16, 1, torch.float32, 1, True, True, True, True, True, True),       # L = 1
    (1, 16, 16, 7, torch.float32, 1, True, True, True, True, True, True),       # shorter than a tile
    (2, 32, 16, 33, torch.float32, 1, True, True, True, True, True, True),      # one step past a chunk
    (1, 32, 16, 100, torch.float32, 1, True, True, False, False, False, False), # no D, no bias, no softplus
    (2, 16, 16, 129, torch.float32, 1, False, True, True, True, True, True),    # constant B
    (2, 16, 16, 129, torch.float32, 1, True, False, True, True, True, True),    # constant C
    (2, 16, 16, 64, torch.float32, 1, False, False, False, True, True, True),   # constant B and C
    (2, 64, 16, 96, torch.float32, 2, True, True, True, True, True, True),      # 2 groups, 32 ch each
    (1, 40, 16, 48, torch.float32, 4, True, True, True, True, True, True),      # 10 channels per group
    (2, 20, 16, 40, torch.float32, 1, True, True, True, True, True, True),      # dim not a multiple of 16
    (1, 16, 1, 50, torch.float32, 1, True, True, True, True, True, True),       # dstate 1
    (1, 16, 4, 50, torch.float32, 1, True, True, True, True, True, True),       # dstate 4
    (1, 16, 32, 50, torch.float32, 1, True, True, True, True, True, True),      # dstate 32 (2 state groups)
    (1, 16, 64, 40, torch.float32, 1, True, True, True, True, True, True),      # dstate 64
    (1, 16, 128, 40, torch.float32, 1, True, True, True, True, True, True),     # dstate 128
    (1, 16, 200, 37, torch.float32, 1, True, True, True, True, True, True),     # dstate 200 (partial state group)
    (2, 16, 256, 33, torch.float32, 1, True, True, True, True, True, True),     # dstate 256, the largest
    (2, 64, 16, 256, torch.bfloat16, 1, True, True, True, True, True, True),    # bf16 I/O
    (1, 32, 16, 70, torch.float16, 1, True, True, True, True, True, True),      # fp16 I/O
    # fast path: dstate 16, variable B/C, 16-channel groups
    (1, 32, 16, 128, torch.float16, 2, True, True, True, True, True, True),     # fp16, 2 groups
    (2, 48, 16, 192, torch.float32, 1, True, True, False, True, True, True),    # no z, 3 workgroups
    (1, 16, 16, 64, torch.bfloat16, 1, True, True, True, False, False, True),   # one super-tile, no D / bias
    (1, 16, 16, 320, torch.float32, 1, True, True, True, True, True, True),     # 5 super-tiles (odd count, z)
    # many channel blocks per group (more than 96): dB / dC summed through workspace slices
    (1, 3072, 16, 128, torch.float32, 1, True, True, True, True, True, True),   # 192 blocks: 2 slices
    (1, 3200, 16, 64, torch.bfloat16, 2, True, True, True, True, True, True),   # 100 blocks per group: 2 slices
    (2, 512, 16, 256, torch.float32, 1, True, True, True, True, True, True),    # 32 blocks: direct accumulation
    # ragged lengths on the fast kernels: a partial last tile of identity steps,
    # row accesses at any element alignment; dB / dC through a slice with
    # rows padded to 32 steps when seqlen is not a multiple of 32
    (2, 64, 16, 1001, torch.bfloat16, 1, True, True, True, True, True, True),   # bf16, odd seqlen
    (2, 32, 16, 2044, torch.float32, 1, True, True, True, True, True, True),    # 4-aligned rows, 60-step tail
    (2, 32, 16, 2064, torch.float32, 1, True, True, True, True, True, True),    # last chunk wholly padded
    (1, 64, 16, 4095, torch.float32, 1, True, True, True, True, True, True),    # sequence segments + tail
    (1, 32, 16, 40, torch.float32, 2, True, True, True, True, True, True),      # 2 groups, one partial tile
    (1, 16, 16, 17, torch.float16, 1, True, True, False, True, True, True),     # fp16, no z, 2 chunks
    # chunk-boundary invariance: lengths either side of 128 and 2048 steps
    (1, 16, 16, 127, torch.float32, 1, True, True, True, True, True, True),
    (1, 16, 16, 128, torch.float32, 1, True, True, True, True, True, True),
    (1, 16, 16, 129, torch.float32, 1, True, True, True, True, True, True),
    (1, 16, 16, 2047, torch.float32, 1, True, True, True, True, True, True),
    (1, 16, 16, 2048, torch.float32, 1, True, True, True, True, True, True),
    (1, 16, 16, 2049, torch.float32, 1, True, True, True, True, True, True),
]


def _ids(c):
    b, d, n, l, dt, g, vb, vc, z, hd, hb, sp = c
    return f"b{b}-d{d}-n{n}-l{l}-{str(dt).split('.')[-1]}-g{g}-{'vB' if vb else 'cB'}{'vC' if vc else 'cC'}" \
           f"{'-z' if z else ''}{'' if hd else '-noD'}{'' if hb else '-nobias'}{'' if sp else '-nosp'}"


def _run_gpu(x, dev, delta_softplus):
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    g = {k: (x[k].to(dev).requires_grad_(True) if x[k] is not None else None) for k in NAMES}
    out = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                            delta_bias=g["delta_bias"], delta_softplus=delta_softplus)
    out.backward(x["dout"].to(dev))
    torch.cuda.synchronize()
    return out.detach().cpu(), {k: g[k].grad.cpu() for k in NAMES if g[k] is not None}


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_selective_scan_fn_matches_oracle(case):
    b, d, n, l, dt, G, vb, vc, hz, hd, hb, sp = case
    print(f"\n[parity] selective_scan_fn {_ids(case)}", flush=True)
    sys.stdout.flush()
    x = make_inputs(b, d, n, l, seed=1234, dtype=dt, n_groups=G, var_B=vb, var_C=vc,
                    has_z=hz, has_D=hd, has_delta_bias=hb)
    if not sp:
        # without softplus the step size is used as given: keep it positive so
        # the recurrence is stable (a = exp(delta * A) < 1)
        x["delta"] = (x["delta"].float().abs() * 0.5).to(dt)
        if x["delta_bias"] is not None:
            x["delta_bias"] = x["delta_bias"].abs()
    out, grads = _run_gpu(x, torch.device("cuda:0"), sp)
    ref, rgrads = oracle_fwd_bwd(x, delta_softplus=sp)
    rtol, atol = TOL[dt]
    assert out.dtype == dt
    assert_close(out, ref, rtol, atol, "out")
    for k, gr in rgrads.items():
        assert_close(grads[k], gr, rtol, atol, f"d{k}")


@pytest.mark.parametrize("shape", [(2, 64, 16, 256), (1, 16, 32, 50)], ids=["fast", "general"])
def test_softplus_above_its_threshold(shape):
    # step sizes well past the softplus threshold (delta + bias > 20, where
    # softplus(x) is taken as x and its derivative as 1, forward_kernel.cu:217-221
    # and backward_kernel.cu:512-514) mixed with ordinary ones, on the fast and
    # the general kernels, against the float64 oracle
    b, d, n, l = shape
    print(f"\n[parity] softplus threshold {shape}", flush=True)
    sys.stdout.flush()
    x = make_inputs(b, d, n, l, seed=4321)
    gen = torch.Generator().manual_seed(4322)
    big = torch.rand(x["delta"].shape, generator=gen) < 0.3
    x["delta"] = torch.where(big, 20.0 + 15.0 * torch.rand(x["delta"].shape, generator=gen), x["delta"])
    assert bool((x["delta"] + x["delta_bias"][None, :, None] > 20).any())
    out, grads = _run_gpu(x, torch.device("cuda:0"), True)
    ref, rgrads = oracle_fwd_bwd(x, delta_softplus=True)
    assert_close(out, ref, 1e-3, 1e-3, "out")
    for k, gr in rgrads.items():
        assert_close(grads[k], gr, 1e-3, 1e-3, f"d{k}")


def test_reference_surface_SelectiveScanFn():
    """SelectiveScanFn.apply with the reference's 8 positional args (modules/mamba_simple.py:131-140)."""
    from mamba_amd.ops.selective_scan_interface import SelectiveScanFn
    print("\n[parity] SelectiveScanFn b2-d64-n16-l256 fp32", flush=True)
    x = make_inputs(2, 64, 16, 256, seed=7, has_z=False)
    dev = torch.device("cuda:0")
    g = {k: (x[k].to(dev).requires_grad_(True) if x[k] is not None else None) for k in NAMES}
    out = SelectiveScanFn.apply(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], g["delta_bias"], True)
    out.backward(x["dout"].to(dev))
    ref, rgrads = oracle_fwd_bwd(x, delta_softplus=True)
    assert_close(out.cpu(), ref, 1e-3, 1e-3, "out")
    for k, gr in rgrads.items():
        assert_close(g[k].grad.cpu(), gr, 1e-3, 1e-3, f"d{k}")


def test_strided_z_and_last_state():
    """z as a channel slice of a packed xz tensor (no copy) and return_last_state."""
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    from oracle.selective_scan_ref import selective_scan_ref
    print("\n[parity] strided z + last state b2-d32-n16-l80", flush=True)
    x = make_inputs(2, 32, 16, 80, seed=11)
    dev = torch.device("cuda:0")
    xz = torch.cat([x["u"], x["z"]], dim=1).to(dev)      # (2, 64, 80)
    u, z = xz[:, :32], xz[:, 32:]
    assert not z.is_contiguous()
    out, last = selective_scan_fn(u, x["delta"].to(dev), x["A"].to(dev), x["B"].to(dev), x["C"].to(dev),
                                  x["D"].to(dev), z=z, delta_bias=x["delta_bias"].to(dev),
                                  delta_softplus=True, return_last_state=True)
    ref, rlast = selective_scan_ref(*(x[k].double() for k in ("u", "delta", "A", "B", "C", "D")),
                                    z=x["z"].double(), delta_bias=x["delta_bias"].double(),
                                    delta_softplus=True, return_last_state=True, compute_dtype=torch.float64)
    assert_close(out.cpu(), ref, 1e-3, 1e-3, "out")
    assert_close(last.cpu(), rlast, 1e-3, 1e-3, "last_state")


def test_fast_path_strided_z_and_last_state():
    """Fast-path shapes with z a channel slice of a packed xz tensor."""
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    print("\n[parity] fast path strided z + last state b2-d32-n16-l128", flush=True)
    x = make_inputs(2, 32, 16, 128, seed=12)
    dev = torch.device("cuda:0")
    xz = torch.cat([x["u"], x["z"]], dim=1).to(dev)      # (2, 64, 128)
    u, z = xz[:, :32], xz[:, 32:]
    g = {k: x[k].to(dev).requires_grad_(True) for k in ("delta", "A", "B", "C", "D", "delta_bias")}
    uu = u.detach().requires_grad_(True)
    zz = z.detach().requires_grad_(True)
    out, last = selective_scan_fn(uu, g["delta"], g["A"], g["B"], g["C"], g["D"], z=zz,
                                  delta_bias=g["delta_bias"], delta_softplus=True, return_last_state=True)
    out.backward(x["dout"].to(dev))
    ref, rgrads = oracle_fwd_bwd(x, delta_softplus=True)
    from oracle.selective_scan_ref import selective_scan_ref
    _, rlast = selective_scan_ref(*(x[k].double() for k in ("u", "delta", "A", "B", "C", "D")),
                                  z=x["z"].double(), delta_bias=x["delta_bias"].double(),
                                  delta_softplus=True, return_last_state=True, compute_dtype=torch.float64)
    assert_close(out.detach().cpu(), ref, 1e-3, 1e-3, "out")
    assert_close(last.cpu(), rlast, 1e-3, 1e-3, "last_state")
    assert_close(uu.grad.cpu(), rgrads["u"], 1e-3, 1e-3, "du")
    assert_close(zz.grad.cpu(), rgrads["z"], 1e-3, 1e-3, "dz")
    for k in ("delta", "A", "B", "C", "D", "delta_bias"):
        assert_close(g[k].grad.cpu(), rgrads[k], 1e-3, 1e-3, f"d{k}")


@pytest.mark.parametrize("shape", [(2, 64, 16, 256, torch.float32), (2, 48, 16, 100, torch.bfloat16),
                                   (1, 32, 4, 70, torch.float32)],
                         ids=["fast-f32", "fast-tail-bf16", "general-n4"])
def test_forward_without_checkpoints(shape):
    """A forward that no backward follows (x, y not given) writes the same out,
    and last_state equals the last checkpoint, on the fast and general kernels."""
    from mamba_amd import selective_scan as ss
    batch, dim, N, L, dt = shape
    print(f"\n[parity] forward without checkpoints b{batch}-d{dim}-n{N}-l{L} {dt}", flush=True)
    x = make_inputs(batch, dim, N, L, seed=21, dtype=dt)
    dev = torch.device("cuda:0")
    t = {k: x[k].to(dev) for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")}
    args = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True)
    out1 = torch.empty_like(t["delta"])
    y1 = torch.empty_like(out1)
    xck = torch.empty((batch, ss.n_chunks(L), dim, N), dtype=torch.float32, device=dev)
    ss.forward_into(*args, out1, xck, z=t["z"], y=y1)
    out2 = torch.full_like(out1, float("nan"))
    last = torch.full((batch, dim, N), float("nan"), device=dev)
    ss.forward_into(*args, out2, None, z=t["z"], y=None, last_state=last)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2), "out must not depend on whether checkpoints are kept"
    assert torch.equal(last, xck[:, -1]), "last_state is the state after the last step"
    with torch.no_grad():
        from mamba_amd.ops.selective_scan_interface import selective_scan_fn
        out3, last3 = selective_scan_fn(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], z=t["z"],
                                        delta_bias=t["delta_bias"], delta_softplus=True, return_last_state=True)
    assert torch.equal(out3, out1) and torch.equal(last3, last)


# the last two: segment counts that do not divide the sequence's super-chunks
# (469 into 64 segments of 7 or 8; 79 into 16 of 4 or 5)
SEG_CASES = [(1, 64, 16, 4096, torch.float32), (2, 32, 16, 2048, torch.bfloat16),
             (1, 1536, 16, 8192, torch.bfloat16), (1, 64, 16, 4093, torch.float32),
             (1, 64, 16, 30000, torch.float32), (1, 96, 16, 5000, torch.bfloat16)]


@pytest.mark.parametrize("shape", SEG_CASES, ids=[f"b{c[0]}-d{c[1]}-l{c[3]}-{str(c[4]).split('.')[-1]}"
                                                  for c in SEG_CASES])
def test_sequence_parallel_forward(shape):
    """Small batches: segments scanned in parallel and joined give the serial
    forward's out, y, checkpoints and last state (to rounding)."""
    from mamba_amd import selective_scan as ss
    batch, dim, N, L, dt = shape
    print(f"\n[parity] sequence-parallel forward b{batch}-d{dim}-l{L} {dt}", flush=True)
    x = make_inputs(batch, dim, N, L, seed=31, dtype=dt)
    dev = torch.device("cuda:0")
    t = {k: x[k].to(dev) for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")}
    args = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True)
    res = {}
    for mode in ("serial", "segments"):
        out = torch.empty_like(t["delta"])
        y = torch.empty_like(out)
        xck = torch.empty((batch, ss.n_chunks(L), dim, N), dtype=torch.float32, device=dev)
        last = torch.empty((batch, dim, N), dtype=torch.float32, device=dev)
        ss.forward_into(*args, out, xck, z=t["z"], y=y, last_state=last,
                        workspace=None if mode == "serial" else "auto")
        res[mode] = (out.float().cpu(), y.float().cpu(), xck.cpu(), last.cpu())
    assert ss.forward_workspace_bytes(*args, out, xck, z=t["z"], y=y) > 0, "this shape should use segments"
    tol = 1e-4 if dt == torch.float32 else 2e-2
    for name, a, b in zip(("out", "y", "x", "last_state"), res["segments"], res["serial"]):
        assert_close(a, b, tol, tol * max(1.0, float(b.abs().max())), name)


def test_sequence_parallel_forward_then_backward_matches_oracle():
    """The backward reads checkpoints written by the segmented forward."""
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    print("\n[parity] sequence-parallel forward + backward vs oracle b1-d64-n16-l4096", flush=True)
    x = make_inputs(1, 64, 16, 4096, seed=32)
    dev = torch.device("cuda:0")
    g = {k: x[k].to(dev).requires_grad_(True) for k in NAMES}
    out = selective_scan_fn(g["u"], g["delta"], g["A"], g["B"], g["C"], g["D"], z=g["z"],
                            delta_bias=g["delta_bias"], delta_softplus=True)
    out.backward(x["dout"].to(dev))
    ref, rgrads = oracle_fwd_bwd(x, delta_softplus=True)
    assert_close(out.detach().cpu(), ref, 1e-3, 1e-3, "out")
    for k, gr in rgrads.items():
        scale = max(1.0, float(gr.abs().max()))
        assert_close(g[k].grad.cpu(), gr, 1e-3, 1e-3 * scale, f"d{k}")
    with torch.no_grad():
        out2, last = selective_scan_fn(*(g[k].detach() for k in ("u", "delta", "A", "B", "C", "D")),
                                       z=g["z"].detach(), delta_bias=g["delta_bias"].detach(),
                                       delta_softplus=True, return_last_state=True)
    from oracle.selective_scan_ref import selective_scan_ref
    _, rlast = selective_scan_ref(*(x[k].double() for k in ("u", "delta", "A", "B", "C", "D")),
                                  z=x["z"].double(), delta_bias=x["delta_bias"].double(),
                                  delta_softplus=True, return_last_state=True, compute_dtype=torch.float64)
    assert_close(out2.cpu(), ref, 1e-3, 1e-3, "out (forward only)")
    assert_close(last.cpu(), rlast, 1e-3, 1e-3, "last_state (forward only)")


@pytest.mark.parametrize("shape", [(1, 64, 16, 4096, torch.float32), (1, 1536, 16, 8192, torch.bfloat16),
                                   (1, 64, 16, 4093, torch.float32), (1, 64, 16, 30000, torch.float32)],
                         ids=["b1-d64-l4096-f32", "b1-d1536-l8192-bf16", "b1-d64-l4093-f32",
                              "b1-d64-l30000-f32-uneven"])
def test_sequence_parallel_backward(shape):
    """Small batches: the backward's segments (adjoint carries scanned in parallel
    and joined) give the serial backward's gradients (to rounding)."""
    from mamba_amd import selective_scan as ss
    batch, dim, N, L, dt = shape
    print(f"\n[parity] sequence-parallel backward b{batch}-d{dim}-l{L} {dt}", flush=True)
    x = make_inputs(batch, dim, N, L, seed=33, dtype=dt)
    dev = torch.device("cuda:0")
    t = {k: x[k].to(dev) for k in ("u", "delta", "A", "B", "C", "D", "z", "delta_bias", "dout")}
    out = torch.empty_like(t["delta"])
    y = torch.empty_like(out)
    xck = torch.empty((batch, ss.n_chunks(L), dim, N), dtype=torch.float32, device=dev)
    ss.forward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, out, xck,
                    z=t["z"], y=y)
    res = {}
    for mode in ("serial", "segments"):
        g = [torch.empty_like(t["u"]), torch.empty_like(t["delta"]),
             torch.empty(t["A"].shape, device=dev), torch.empty(t["B"].shape, device=dev),
             torch.empty(t["C"].shape, device=dev), torch.empty(t["D"].shape, device=dev),
             torch.empty(t["delta_bias"].shape, device=dev), torch.empty_like(t["z"])]
        args = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], t["dout"], xck, True,
                *g[:7])
        if mode == "segments":
            need = ss.workspace_bytes(*args, z=t["z"], y=y, dz=g[7])
            ws = torch.empty(need, dtype=torch.uint8, device=dev)
        else:
            ws = None
        ss.backward_into(*args, z=t["z"], y=y, dz=g[7], workspace=ws, zero_grads=True)
        res[mode] = [v.float().cpu() for v in g]
    tol = 1e-4 if dt == torch.float32 else 2e-2
    for name, a, b in zip(("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz"), res["segments"],
                          res["serial"]):
        assert_close(a, b, tol, tol * max(1.0, float(b.abs().max())), name)


# (batch, dim, seqlen, workspace bytes): 192 channel blocks (2 slices);
# ragged seqlens, whose workspace is one slice with rows padded to 32 steps
# and whose direct accumulation adds the zero sums of the steps past the
# sequence inside the row (1001: a partial chunk and one wholly past it;
# 2064: one wholly past it)
WS_CASES = [(1, 3072, 128, 2 * 2 * (1 * 16 * 128) * 4), (8, 64, 1001, None), (8, 32, 2064, None)]


@pytest.mark.parametrize("case", WS_CASES, ids=["slices", "ragged-1001", "ragged-2064"])
def test_backward_with_and_without_workspace(case):
    """The dB / dC slices (workspace) and direct accumulation give the same gradients."""
    from mamba_amd import selective_scan as ss
    batch, dim, L, ws_bytes = case
    print(f"\n[parity] workspace vs direct b{batch}-d{dim}-n16-l{L} fp32", flush=True)
    dev = torch.device("cuda:0")
    x = make_inputs(batch, dim, 16, L, seed=21)
    t = {k: x[k].to(dev) for k in NAMES}
    dout = x["dout"].to(dev)
    out, xck, y = ss.forward(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, z=t["z"])
    res = {}
    for mode in ("auto", None):
        g = [torch.empty_like(t["u"]), torch.empty_like(t["delta"])] + \
            [torch.zeros(t[k].shape, dtype=torch.float32, device=dev) for k in ("A", "B", "C", "D", "delta_bias")]
        dz = torch.empty_like(t["z"])
        args = (t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], dout, xck, True, *g)
        if mode == "auto":
            n = ss.workspace_bytes(*args, z=t["z"], y=y, dz=dz)
            assert n == ws_bytes if ws_bytes is not None else n >= 2 * batch * 16 * ((L + 31) // 32 * 32) * 4
        ss.backward_into(*args, z=t["z"], y=y, dz=dz, workspace=mode)
        torch.cuda.synchronize()
        res[mode] = [v.cpu() for v in g] + [dz.cpu()]
    # (the workspace also brings sequence segments at the small shapes, whose
    # joined carries round differently: the segment tests' tolerance)
    for a, b_, name in zip(res["auto"], res[None], ("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias", "dz")):
        assert_close(a, b_, 1e-4, 1e-4 * max(1.0, float(b_.abs().max())), name)


@pytest.mark.parametrize("mode", ["auto", None])
def test_zero_grads_clears_and_plain_call_accumulates(mode):
    """zero_grads ignores what the accumulators hold (NaN here); without it the
    call adds into them (the reference's backward zero-initialises them,
    selective_scan.cpp:274-287; this boundary lets the caller choose)."""
    from mamba_amd import selective_scan as ss
    print(f"\n[parity] zero_grads workspace={mode} b2-d512-n16-l128 fp32", flush=True)
    dev = torch.device("cuda:0")
    x = make_inputs(2, 512, 16, 128, seed=23)
    t = {k: x[k].to(dev) for k in NAMES}
    dout = x["dout"].to(dev)
    out, xck, y = ss.forward(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], True, z=t["z"])
    acc_names = ("A", "B", "C", "D", "delta_bias")

    def run(fill, zero_grads):
        g = [torch.empty_like(t["u"]), torch.empty_like(t["delta"])] + \
            [torch.full(t[k].shape, fill, dtype=torch.float32, device=dev) for k in acc_names]
        dz = torch.empty_like(t["z"])
        ss.backward_into(t["u"], t["delta"], t["A"], t["B"], t["C"], t["D"], t["delta_bias"], dout, xck, True,
                         *g, z=t["z"], y=y, dz=dz, workspace=mode, zero_grads=zero_grads)
        torch.cuda.synchronize()
        return [v.cpu() for v in g]

    ref = run(0.0, False)
    cleared = run(float("nan"), True)
    added = run(1.0, False)
    names = ("du", "ddelta", "dA", "dB", "dC", "dD", "ddelta_bias")
    for a, b_, name in zip(cleared, ref, names):
        assert torch.isfinite(a).all(), name
        assert_close(a, b_, 1e-5, 1e-5, name)
    for i, name in enumerate(names):
        want = ref[i] + 1.0 if i >= 2 else ref[i]
        assert_close(added[i], want, 1e-5, 1e-5, name)


def test_zero_grads_with_empty_batch():
    """batch 0: no scan work, but zero_grads still returns zeroed dA / dD / ddelta_bias."""
    from mamba_amd import selective_scan as ss
    print("\n[parity] zero_grads with batch 0", flush=True)
    dev = torch.device("cuda:0")
    x = make_inputs(1, 32, 16, 64, seed=24)
    t = {k: x[k].to(dev) for k in NAMES}
    e = {k: t[k][:0] for k in ("u", "delta", "z", "B", "C")}
    xck = torch.empty((0, ss.n_chunks(64), 32, 16), dtype=torch.float32, device=dev)
    y = torch.empty_like(e["u"])
    res = ss.backward(e["u"], e["delta"], t["A"], e["B"], e["C"], t["D"], t["delta_bias"], torch.empty_like(e["u"]),
                      xck, True, z=e["z"], y=y)
    torch.cuda.synchronize()
    for i, shape in ((2, (32, 16)), (5, (32,)), (6, (32,))):
        assert tuple(res[i].shape) == shape
        assert (res[i].cpu() == 0).all()
