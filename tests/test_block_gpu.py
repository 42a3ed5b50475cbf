"""GPU parity of the Mamba block around the scan, through the HIP library.

* causal conv1d (+ SiLU) forward and backward against float64 autograd of
  the conv oracle: widths 1-4, with and without bias and activation, x as a
  channel slice of a packed xz tensor, a seqlen that is not a multiple of 4
  (element path), fp32 / bf16 / fp16;
* 40 seeded random conv1d shapes (batch, channels, seqlen from 1 to 5000,
  width, dtype, bias, SiLU, padded channel rows, atomic or fixed-order
  dweight / dbias sums) against float64 autograd of the conv oracle;
* mamba_inner_fn forward and backward (all 14 differentiable inputs)
  against float64 autograd of mamba_inner_ref, also on 12 seeded random
  shapes (d_inner not a multiple of 16, ragged seqlens, dstate other than
  16, odd dt_rank, with and without biases);
* MambaSimple (both forward paths) and CausalLM against the oracle, with
  the same weights;
* a no-grad MambaSimple forward (fp32 parameters cached by version) equal bit
  for bit to one with autograd, also after an in-place parameter update;
  a block built under torch.inference_mode (no version counters) forwards
  and steps without the cache.

Tolerances: fp32 rtol / atol 1e-3, bf16 / fp16 2e-2 (relative to the
largest magnitude for the GEMM-heavy block outputs, stated per test).
"""
import sys

import pytest
import torch

from oracle.mamba_block_ref import causal_conv1d_ref, causal_lm_ref, mamba_inner_ref, mamba_simple_ref
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: (1e-3, 1e-3), torch.bfloat16: (2e-2, 2e-2), torch.float16: (2e-2, 2e-2)}


def _say(msg):
    print(f"\n[block] {msg}", flush=True)
    sys.stdout.flush()


CONV_CASES = [
    # batch, dim, seqlen, width, bias, act, dtype, strided x
    (2, 64, 256, 4, True, "silu", torch.float32, False),
    (2, 64, 256, 4, False, "silu", torch.float32, True),
    (1, 32, 1000, 3, True, None, torch.float32, False),
    (3, 16, 37, 2, True, "silu", torch.float32, False),     # element path (seqlen % 4 != 0)
    (2, 8, 5, 1, False, "silu", torch.float32, False),
    (2, 64, 2048, 4, True, "silu", torch.bfloat16, True),      # 8-element vectors
    (1, 48, 130, 4, False, "silu", torch.float16, False),      # element path (seqlen % 4 != 0)
    (2, 32, 1028, 4, True, "silu", torch.bfloat16, False),     # 16-bit 4-element vectors (seqlen % 8 == 4)
    (1, 16, 4104, 4, True, "silu", torch.bfloat16, True),      # 3 workgroup segments, the last ragged
    (1, 16, 3000, 3, True, None, torch.float32, False),        # fp32, 3 workgroup segments
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[f"b{c[0]}-d{c[1]}-l{c[2]}-w{c[3]}-{'bias' if c[4] else 'nobias'}"
                                                  f"-{c[5]}-{str(c[6]).split('.')[-1]}{'-strided' if c[7] else ''}"
                                                  for c in CONV_CASES])
def test_causal_conv1d(case):
    from mamba_amd.ops.causal_conv1d import causal_conv1d_fn
    batch, dim, L, width, has_bias, act, dt, strided = case
    _say(f"causal_conv1d {case}")
    g = torch.Generator().manual_seed(dim + L)
    xz = torch.randn(batch, 2 * dim if strided else dim, L, generator=g).to(dt)
    w = torch.randn(dim, 1, width, generator=g) * 0.5
    b = torch.randn(dim, generator=g) if has_bias else None
    dout = torch.randn(batch, dim, L, generator=g).to(dt)
    xg = xz.to(DEV).requires_grad_(True)
    x = xg[:, :dim]
    wg = w.to(DEV).requires_grad_(True)
    bg = b.to(DEV).requires_grad_(True) if b is not None else None
    out = causal_conv1d_fn(x, wg, bg, activation=act)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    xr = xz[:, :dim].double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    br = b.double().requires_grad_(True) if b is not None else None
    ref = causal_conv1d_ref(xr, wr, br, activation=act)
    ref.backward(dout.double())
    rtol, atol = TOL[dt]
    assert out.dtype == dt
    assert_close(out.cpu(), ref, rtol, atol, "out")
    assert_close(xg.grad[:, :dim].cpu(), xr.grad, rtol, atol, "dx")
    if strided:
        assert torch.all(xg.grad[:, dim:] == 0)
    scale = max(1.0, float(wr.grad.abs().max()))
    assert_close(wg.grad.cpu(), wr.grad, rtol, atol * scale, "dweight")
    if b is not None:
        assert_close(bg.grad.cpu(), br.grad, rtol, atol * max(1.0, float(br.grad.abs().max())), "dbias")


@pytest.mark.parametrize("i", range(40))
def test_causal_conv1d_random(i):
    import random
    from mamba_amd.ops.causal_conv1d import causal_conv1d_bwd, causal_conv1d_fwd
    rnd = random.Random(5000 + i)
    batch = rnd.choice([1, 2, 3, 5])
    dim = rnd.choice([1, 3, 16, 40, 64, 100])
    L = rnd.choice([1, 2, 3, 4, 5, 7, 8, 15, 16, 31, 64, 100, 255, 256, 1023, 1024, 1025, 2048, 3001, 4104,
                    rnd.randint(1, 5000)])
    width = rnd.choice([1, 2, 3, 4])
    dt = rnd.choice([torch.float32, torch.bfloat16, torch.float16])
    has_bias = rnd.random() < 0.6
    silu = rnd.random() < 0.7
    pad = rnd.choice([0, 0, 8, 3])
    det = rnd.random() < 0.5
    _say(f"conv1d random {i}: batch {batch} dim {dim} seqlen {L} width {width} {dt} bias {has_bias} "
         f"silu {silu} pad {pad} fixed-order {det}")
    g = torch.Generator().manual_seed(6000 + i)
    xz = torch.randn(batch, dim + pad, L, generator=g).to(dt)
    w = torch.randn(dim, width, generator=g) * 0.5
    b = torch.randn(dim, generator=g) if has_bias else None
    dout = torch.randn(batch, dim, L, generator=g).to(dt)
    x = xz.to(DEV)[:, :dim]
    bd = b.to(DEV) if b is not None else None
    out = causal_conv1d_fwd(x, w.to(DEV), bd, silu)
    dx, dw, db = causal_conv1d_bwd(x, w.to(DEV), bd, dout.to(DEV), silu, deterministic=det)
    torch.cuda.synchronize()
    xr = xz[:, :dim].double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    br = b.double().requires_grad_(True) if b is not None else None
    ref = causal_conv1d_ref(xr, wr, br, activation="silu" if silu else None)
    ref.backward(dout.double())
    rtol, atol = TOL[dt]
    assert_close(out.float().cpu(), ref.detach(), rtol, atol, "out")
    assert_close(dx.float().cpu(), xr.grad, rtol, atol, "dx")
    assert_close(dw.cpu(), wr.grad, rtol, atol * max(1.0, float(wr.grad.abs().max())), "dweight")
    if b is not None:
        assert_close(db.cpu(), br.grad, rtol, atol * max(1.0, float(br.grad.abs().max())), "dbias")


def _block_params(d_model, dim, R, N, width, dt, seed, out_bias=True, conv_bias=True):
    g = torch.Generator().manual_seed(seed)
    p = {
        "conv1d_weight": torch.randn(dim, 1, width, generator=g) * 0.3,
        "conv1d_bias": torch.randn(dim, generator=g) * 0.1 if conv_bias else None,
        "x_proj_weight": torch.randn(R + 2 * N, dim, generator=g) * dim ** -0.5,
        "delta_proj_weight": torch.rand(dim, R, generator=g) * R ** -0.5,
        "out_proj_weight": torch.randn(d_model, dim, generator=g) * dim ** -0.5,
        "out_proj_bias": torch.randn(d_model, generator=g) * 0.1 if out_bias else None,
        "A": -torch.arange(1, N + 1, dtype=torch.float32).repeat(dim, 1),
        "D": torch.ones(dim),
        "delta_bias": torch.log(torch.expm1(torch.rand(dim, generator=g) * 0.099 + 0.001)),
    }
    return {k: (v.to(dt) if v is not None and k not in ("A", "D", "delta_bias") else v) for k, v in p.items()}


ARGS = ("conv1d_weight", "conv1d_bias", "x_proj_weight", "delta_proj_weight", "out_proj_weight",
        "out_proj_bias", "A")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_mamba_inner_fn(dt):
    from mamba_amd.ops.selective_scan_interface import mamba_inner_fn
    batch, d_model, dim, L, R, N, width = 2, 32, 64, 128, 4, 16, 4
    _say(f"mamba_inner_fn batch {batch} dim {dim} seqlen {L} {dt}")
    p = _block_params(d_model, dim, R, N, width, dt, seed=5)
    g = torch.Generator().manual_seed(6)
    xz = torch.randn(batch, 2 * dim, L, generator=g).to(dt)
    dres = torch.randn(batch, L, d_model, generator=g).to(dt)

    gp = {k: (v.to(DEV).requires_grad_(True) if v is not None else None) for k, v in p.items()}
    xzg = xz.to(DEV).requires_grad_(True)
    out = mamba_inner_fn(xzg, *(gp[k] for k in ARGS), D=gp["D"], delta_bias=gp["delta_bias"], delta_softplus=True)
    out.backward(dres.to(DEV))
    torch.cuda.synchronize()

    rp = {k: (v.double().requires_grad_(True) if v is not None else None) for k, v in p.items()}
    xzr = xz.double().requires_grad_(True)
    ref = mamba_inner_ref(xzr, *(rp[k] for k in ARGS), D=rp["D"], delta_bias=rp["delta_bias"], delta_softplus=True)
    ref.backward(dres.double())

    rtol, atol = TOL[dt]
    assert out.shape == ref.shape and out.dtype == dt
    # GEMM chains: compare against the largest magnitude of each tensor
    def close(a, b, what):
        assert_close(a, b, rtol, atol * max(1.0, float(b.detach().abs().max())), what)
    close(out.float().cpu(), ref, "out")
    close(xzg.grad.float().cpu(), xzr.grad, "dxz")
    for k in p:
        if p[k] is not None:
            close(gp[k].grad.float().cpu(), rp[k].grad, f"d{k}")


@pytest.mark.parametrize("i", range(12))
def test_mamba_inner_fn_random(i):
    import random
    from mamba_amd.ops.selective_scan_interface import mamba_inner_fn
    rnd = random.Random(2100 + i)
    batch = rnd.choice([1, 2, 3])
    d_model = rnd.choice([8, 16, 24, 32])
    dim = rnd.choice([16, 24, 40, 64, 80])
    L = rnd.choice([1, 5, 16, 33, 64, 100, 127, 200, rnd.randint(1, 300)])
    R = rnd.choice([1, 3, 4, 8])
    N = rnd.choice([16, 16, 4, 8, 32])
    width = rnd.choice([2, 3, 4])
    dt = rnd.choice([torch.float32, torch.float32, torch.bfloat16])
    out_bias, conv_bias = rnd.random() < 0.5, rnd.random() < 0.5
    _say(f"mamba_inner_fn random {i}: batch {batch} d_model {d_model} dim {dim} seqlen {L} rank {R} dstate {N} "
         f"width {width} {dt} out_bias {out_bias} conv_bias {conv_bias}")
    p = _block_params(d_model, dim, R, N, width, dt, seed=2200 + i, out_bias=out_bias, conv_bias=conv_bias)
    g = torch.Generator().manual_seed(2300 + i)
    xz = torch.randn(batch, 2 * dim, L, generator=g).to(dt)
    dres = torch.randn(batch, L, d_model, generator=g).to(dt)
    gp = {k: (v.to(DEV).requires_grad_(True) if v is not None else None) for k, v in p.items()}
    xzg = xz.to(DEV).requires_grad_(True)
    out = mamba_inner_fn(xzg, *(gp[k] for k in ARGS), D=gp["D"], delta_bias=gp["delta_bias"], delta_softplus=True)
    out.backward(dres.to(DEV))
    torch.cuda.synchronize()
    rp = {k: (v.double().requires_grad_(True) if v is not None else None) for k, v in p.items()}
    xzr = xz.double().requires_grad_(True)
    ref = mamba_inner_ref(xzr, *(rp[k] for k in ARGS), D=rp["D"], delta_bias=rp["delta_bias"], delta_softplus=True)
    ref.backward(dres.double())
    rtol, atol = TOL[dt]

    def close(a, b, what):
        assert_close(a, b, rtol, atol * max(1.0, float(b.detach().abs().max())), what)
    close(out.detach().float().cpu(), ref.detach(), "out")
    close(xzg.grad.float().cpu(), xzr.grad, "dxz")
    for k in p:
        if p[k] is not None:
            close(gp[k].grad.float().cpu(), rp[k].grad, f"d{k}")


def test_mamba_simple_both_paths_and_causal_lm():
    from mamba_amd.models import CausalLM, CausalLMConfig
    from mamba_amd.modules import MambaSimple
    _say("MambaSimple fast / reference paths, CausalLM forward")
    torch.manual_seed(11)
    m = MambaSimple(model_dim=32, state_dim=16).to(DEV)
    sd = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
    hidden = torch.randn(2, 64, 32)
    hg = hidden.to(DEV).requires_grad_(True)
    fast = m(hg)
    fast.sum().backward()
    grads_fast = {n: q.grad.detach().cpu().clone() for n, q in m.named_parameters()}
    dh_fast = hg.grad.detach().cpu().clone()
    m.zero_grad()
    hg.grad = None
    m.use_fast_path = False
    slow = m(hg)
    slow.sum().backward()
    grads_slow = {n: q.grad.detach().cpu().clone() for n, q in m.named_parameters()}
    ref = mamba_simple_ref(sd, hidden.double())
    assert_close(fast.detach().cpu(), ref, 1e-3, 1e-3, "MambaSimple fast path")
    assert_close(slow.detach().cpu(), ref, 1e-3, 1e-3, "MambaSimple reference path")
    for n in grads_fast:
        scale = max(1.0, float(grads_slow[n].abs().max()))
        assert_close(grads_fast[n], grads_slow[n], 1e-3, 1e-3 * scale, f"grad {n}")
    assert_close(dh_fast, hg.grad.cpu(), 1e-3, 1e-3, "d hidden")

    cfg = CausalLMConfig(vocab_size=101, model_dim=32, state_dim=16, num_layers=2)
    lm = CausalLM(cfg).to(DEV).eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 64))
    with torch.no_grad():
        logits = lm(ids.to(DEV)).cpu()
    ref = causal_lm_ref({k: v.detach().double().cpu() for k, v in lm.state_dict().items()}, ids, num_layers=2)
    assert_close(logits, ref, 1e-3, 1e-3 * float(ref.abs().max()), "CausalLM logits")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_mamba_simple_no_grad_forward_matches(dt):
    from mamba_amd.modules import MambaSimple
    _say(f"MambaSimple no-grad forward with cached parameters, {dt}")
    torch.manual_seed(12)
    m = MambaSimple(model_dim=64, state_dim=16, conv_bias=True, device=DEV, dtype=dt)
    hidden = torch.randn(2, 256, 64, device=DEV).to(dt)

    def both():
        with torch.no_grad():
            a = m(hidden)
        b = m(hidden).detach()
        torch.cuda.synchronize()
        return a, b
    a, b = both()
    assert torch.equal(a, b)
    with torch.no_grad():            # in place: the cached fp32 copies must follow
        m.log_A.add_(0.25)
        m.D.mul_(0.5)
        m.delta_proj.bias.add_(0.1)
        m.short_conv.weight.mul_(-1.0)
        m.short_conv.bias.add_(0.2)
    a2, b2 = both()
    assert torch.equal(a2, b2)
    assert not torch.equal(a2, a)


def test_mamba_simple_parameters_made_in_inference_mode():
    # inference tensors carry no version counter: no-grad forwards and decode
    # steps compute the fp32 parameters on every call instead of caching them
    from mamba_amd.modules import MambaSimple
    _say("MambaSimple built under torch.inference_mode")
    torch.manual_seed(13)
    with torch.inference_mode():
        m = MambaSimple(model_dim=64, state_dim=16, conv_bias=True, device=DEV, dtype=torch.float32)
        hidden = torch.randn(2, 128, 64, device=DEV)
        out = m(hidden)
        conv_state, ssm_state = m.allocate_inference_cache(2)
        steps = [m.step(hidden[:, t], conv_state, ssm_state) for t in range(4)]
        sd0 = {k: v.clone() for k, v in m.state_dict().items()}
        m.log_A.add_(0.25)                      # in place, no version counter moves
        out2 = m(hidden)
        sd1 = {k: v.clone() for k, v in m.state_dict().items()}
    ref = MambaSimple(model_dim=64, state_dim=16, conv_bias=True, device=DEV, dtype=torch.float32)
    with torch.no_grad():
        ref.load_state_dict(sd0)
        want = ref(hidden.clone())
        ref.load_state_dict(sd1)
        want2 = ref(hidden.clone())
    torch.cuda.synchronize()
    assert torch.equal(out, want) and torch.equal(out2, want2)
    for t, y in enumerate(steps):
        assert_close(y.cpu(), want[:, t].cpu(), 1e-3, 1e-3, f"step {t}")
