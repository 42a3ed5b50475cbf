"""Shared helpers for the tests (input construction and closeness checks)."""
import torch

from oracle.selective_scan_ref import make_inputs, selective_scan_ref

NAMES = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")


def assert_close(got, want, rtol, atol, what):
    """|got - want| <= atol + rtol * |want| elementwise, with the worst element reported."""
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} vs {tuple(want.shape)}"
    err = (got - want).abs()
    bound = atol + rtol * want.abs()
    bad = err > bound
    if bad.any():
        i = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{err.numel()} elements out of tolerance; worst at flat index {i}: "
            f"got {got.flatten()[i].item():.6g} want {want.flatten()[i].item():.6g} "
            f"(max abs err {err.max().item():.3g}, max |want| {want.abs().max().item():.3g})")


def oracle_fwd_bwd(x, delta_softplus=True, with_grad=True):
    """fp64 oracle output and autograd gradients for the dict from make_inputs."""
    ins = {k: (x[k].detach().double().requires_grad_(with_grad) if x[k] is not None else None) for k in NAMES}
    out = selective_scan_ref(ins["u"], ins["delta"], ins["A"], ins["B"], ins["C"], ins["D"],
                             z=ins["z"], delta_bias=ins["delta_bias"], delta_softplus=delta_softplus,
                             compute_dtype=torch.float64)
    grads = {}
    if with_grad:
        out.backward(x["dout"].double())
        grads = {k: ins[k].grad for k in NAMES if ins[k] is not None}
    return out.detach(), grads
