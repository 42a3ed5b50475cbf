"""GPU parity of the fused RMSNorm (+ residual) kernels, through the HIP library.

* forward: out against rms_norm_ref in float64 from the same (rounded) sum
  s; s itself bit-exact against PyTorch's x + residual in the I/O dtype;
  rstd against the float64 value;
* backward: dx (= dresidual) and dweight against float64 autograd of
  rms_norm_ref, with a gradient arriving at s as well (prenorm);
* row lengths that take one register segment, several segments (rows read
  twice), and the one-element-per-lane path (lengths or strides that are
  not whole 16-byte vectors); strided rows; more rows than backward
  workgroups can take at once; no rows;
* 30 seeded random cases (rows, row length from 1 to 6000, dtypes, residual,
  row padding) through the same checks;
* dweight has the same bits on every run;
* CausalLM with the residual stream fused into the norms against the
  reference's block order (every op on the GPU), forward and gradients.

Tolerances: out / dx: fp32 1e-5, fp16 2e-3, bf16 1e-2 (rtol and atol; the
kernels compute in fp32 and round once); dweight: the same relative to its
largest magnitude.
"""
import sys

import pytest
import torch

from oracle.mamba_block_ref import add_rms_norm_ref, rms_norm_ref
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1e-2}


def _say(msg):
    print(f"\n[rmsnorm] {msg}", flush=True)
    sys.stdout.flush()


CASES = [
    # leading shape, dim, dtype, weight dtype, residual, row padding (0: contiguous rows)
    ((4, 64), 768, torch.bfloat16, torch.bfloat16, True, 0),     # one segment per row
    ((2, 33), 4096, torch.bfloat16, torch.float32, True, 0),     # several segments
    ((3, 50), 1024, torch.float32, torch.float32, False, 0),
    ((5, 7), 100, torch.float16, torch.float16, True, 0),        # one element per lane per slot
    ((2, 9), 5000, torch.float32, torch.float32, True, 0),       # fp32, 5 / 10 segments
    ((3, 11), 3001, torch.bfloat16, torch.bfloat16, True, 0),    # element path, several segments
    ((6, 40), 768, torch.bfloat16, torch.bfloat16, True, 32),    # strided rows, 16-byte aligned
    ((6, 40), 768, torch.bfloat16, torch.float32, False, 2),     # strided rows, element path
    ((5000,), 768, torch.bfloat16, torch.bfloat16, True, 0),     # several rows per backward wave
    ((1,), 1, torch.float32, torch.float32, True, 0),
]


def _ids(c):
    return (f"{'x'.join(map(str, c[0]))}-d{c[1]}-{str(c[2]).split('.')[-1]}-w{str(c[3]).split('.')[-1]}"
            f"{'-res' if c[4] else ''}{f'-pad{c[5]}' if c[5] else ''}")


def _rows_tensor(shape, dim, dtype, pad, gen):
    """A (shape..., dim) tensor whose rows are `dim + pad` apart in memory."""
    full = torch.randn(*shape, dim + pad, generator=gen).to(dtype).to(DEV)
    return full[..., :dim] if pad else full


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_rms_norm_fwd_bwd(case):
    from mamba_amd.ops.rms_norm import rms_norm_fn
    shape, dim, dt, wdt, with_res, pad = case
    _say(f"case {_ids(case)}")
    gen = torch.Generator().manual_seed(100 + dim)
    x = _rows_tensor(shape, dim, dt, pad, gen)
    r = _rows_tensor(shape, dim, dt, 0, gen) if with_res else None
    w = (0.5 * torch.randn(dim, generator=gen)).to(wdt).to(DEV)
    dout = torch.randn(*shape, dim, generator=gen).to(dt).to(DEV)
    dres = torch.randn(*shape, dim, generator=gen).to(dt).to(DEV) if with_res else None

    xg = x.detach().requires_grad_(True)
    wg = w.detach().requires_grad_(True)
    rg = r.detach().requires_grad_(True) if with_res else None
    if with_res:
        out, s = rms_norm_fn(xg, wg, rg, eps=1e-6, prenorm=True)
        torch.autograd.backward([out, s], [dout, dres])
    else:
        out = rms_norm_fn(xg, wg, None, eps=1e-6)
        out.backward(dout)
        s = x

    # oracle: s in the I/O dtype, the norm and its gradients in float64 from s
    want_out, want_s = add_rms_norm_ref(x.cpu(), r.cpu() if with_res else None, w.cpu())
    assert torch.equal(s.detach().cpu(), want_s), "s = x + residual must be the dtype's sum"
    sd = want_s.double().requires_grad_(True)
    wd = w.cpu().double().requires_grad_(True)
    od = rms_norm_ref(sd, wd)
    od.backward(dout.cpu().double())
    ds_want = sd.grad + (dres.cpu().double() if with_res else 0.0)
    tol = TOL[dt]
    assert_close(out.detach().cpu(), od.detach(), tol, tol, "out")
    assert_close(xg.grad.cpu(), ds_want, tol, tol * max(1.0, float(ds_want.abs().max())), "dx")
    if with_res:
        assert torch.equal(rg.grad, xg.grad), "dresidual must equal dx"
    dw_want = wd.grad
    wtol = max(tol, TOL[wdt])
    assert_close(wg.grad.cpu(), dw_want, wtol, wtol * float(dw_want.abs().max()), "dweight")


def _random_case(i):
    import random
    rnd = random.Random(4000 + i)
    dt = rnd.choice([torch.float32, torch.bfloat16, torch.float16])
    dim = rnd.choice([1, 7, 8, 64, 100, 512, 768, 1000, 1024, 2048, 2049, 4096, rnd.randint(1, 6000)])
    rows = rnd.choice([1, 2, 17, 64, 300, rnd.randint(1, 3000)])
    return ((rows,), dim, dt, rnd.choice([dt, torch.float32]), rnd.random() < 0.6, rnd.choice([0, 0, 8, 3]))


@pytest.mark.parametrize("i", range(30))
def test_rms_norm_random(i):
    test_rms_norm_fwd_bwd(_random_case(i))


def test_rstd_and_deterministic_dweight():
    from mamba_amd.ops.rms_norm import rms_norm_bwd, rms_norm_fwd
    _say("rstd, deterministic dweight")
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(6000, 768, generator=gen).bfloat16().to(DEV)
    r = torch.randn(6000, 768, generator=gen).bfloat16().to(DEV)
    w = (0.5 * torch.randn(768, generator=gen)).bfloat16().to(DEV)
    out, s, rstd = rms_norm_fwd(x, w, r, eps=1e-6, want_rstd=True)
    sd = s.cpu().double()
    rstd_want = torch.rsqrt(sd.pow(2).mean(-1) + 1e-6)
    assert_close(rstd.cpu(), rstd_want, 1e-5, 0.0, "rstd")
    dout = torch.randn(6000, 768, generator=gen).bfloat16().to(DEV)
    dx1, dw1 = rms_norm_bwd(s, w, rstd, dout)
    dx2, dw2 = rms_norm_bwd(s, w, rstd, dout)
    torch.cuda.synchronize()
    assert torch.equal(dx1, dx2)
    assert torch.equal(dw1, dw2), "dweight must not depend on scheduling"


@pytest.mark.parametrize("case", [(6000, 768, torch.bfloat16), (3000, 768, torch.float32), (700, 8192, torch.bfloat16)],
                         ids=["resident-bf16", "segments-fp32", "long-rows-2-waves"])
def test_dweight_same_bits_every_run(case):
    # fp32 weight (dweight fp32, so no rounding to the weight dtype can hide
    # a different summation order): three backward runs give the same bits, on
    # the one-segment path, the multi-segment path and rows long enough that
    # a workgroup has 2 waves; dweight against the float64 sum
    from mamba_amd.ops.rms_norm import rms_norm_bwd, rms_norm_fwd
    rows, dim, dt = case
    _say(f"dweight reproducible {case}")
    gen = torch.Generator().manual_seed(11 + dim)
    x = torch.randn(rows, dim, generator=gen).to(dt).to(DEV)
    w = (0.5 * torch.randn(dim, generator=gen)).to(DEV)                   # fp32
    out, _, rstd = rms_norm_fwd(x, w, None, eps=1e-6, want_rstd=True, want_s=False)
    dout = torch.randn(rows, dim, generator=gen).to(dt).to(DEV)
    runs = [rms_norm_bwd(x, w, rstd, dout) for _ in range(3)]
    torch.cuda.synchronize()
    for dx, dw in runs[1:]:
        assert torch.equal(dx, runs[0][0])
        assert torch.equal(dw, runs[0][1]), "dweight must not depend on scheduling"
    xd, dd = x.double().cpu(), dout.double().cpu()
    want = (dd * xd * rstd.double().cpu()[:, None]).sum(0)
    assert_close(runs[0][1].cpu(), want, 1e-4, 1e-4 * float(want.abs().max()), "dweight")


def test_empty_rows():
    from mamba_amd.ops.rms_norm import rms_norm_bwd, rms_norm_fwd
    _say("no rows")
    x = torch.empty(0, 768, dtype=torch.bfloat16, device=DEV)
    w = torch.randn(768, device=DEV).bfloat16()
    out, s, rstd = rms_norm_fwd(x, w, x, want_rstd=True)
    assert out.shape == (0, 768) and s.shape == (0, 768) and rstd.shape == (0,)
    dx, dw = rms_norm_bwd(x, w, rstd, x)
    torch.cuda.synchronize()
    assert dx.shape == (0, 768)
    assert torch.equal(dw.cpu(), torch.zeros(768, dtype=torch.bfloat16)), "no rows: dweight is zero"


def test_causal_lm_fused_residual_matches_reference_order():
    from mamba_amd.models import CausalLM, CausalLMConfig
    _say("CausalLM fused residual stream vs the reference's block order")
    torch.manual_seed(12)
    cfg = CausalLMConfig(vocab_size=97, model_dim=64, state_dim=16, num_layers=3, dropout_rate=0.0)
    lm = CausalLM(cfg).to(DEV)
    with torch.no_grad():
        for layer in lm.layers:
            layer.norm.weight.uniform_(-0.3, 0.3)
        lm.norm.weight.uniform_(-0.3, 0.3)
    ids = torch.randint(0, cfg.vocab_size, (2, 128), device=DEV)

    def run(fast):
        for layer in lm.layers:
            layer.norm.use_fast_path = fast
        lm.norm.use_fast_path = fast
        lm.zero_grad()
        logits = lm(ids)
        (logits.float() * torch.linspace(-1, 1, logits.shape[-1], device=DEV)).sum().backward()
        return logits.detach().cpu(), {n: p.grad.detach().cpu().clone() for n, p in lm.named_parameters()}

    fused, gf = run(True)
    assert lm._fused_residual(torch.empty(1, device=DEV))
    ref, gr = run(False)
    scale = float(ref.abs().max())
    assert_close(fused, ref, 1e-4, 1e-4 * scale, "logits")
    for n in gr:
        s = max(1e-6, float(gr[n].abs().max()))
        assert_close(gf[n], gr[n], 1e-3, 1e-3 * s, f"grad {n}")
