"""GPU parity of single-token decode, through the HIP library.

* ss_state_update against the float64 step oracle: dstate 16 (16-byte state
  path) and 5 (element path), a strided state, strided B / C, 1 and 2
  groups, with and without D / z / bias, fp32 / bf16 / fp16 I/O; delta as
  the low-rank pair (dt_low, dt_weight) summed in the kernel (vector and
  element loads);
* ss_conv1d_update against the step oracle: widths 1-4, with and without
  bias and SiLU; the shifted state is bit-exact;
* token-by-token state updates from a zero state reproduce
  selective_scan_fn over the sequence on the GPU (outputs and last state);
* MambaSimple and CausalLM: prefill of a prompt (filling the decode cache
  from the parallel forward) followed by step() on the remaining tokens
  gives the logits of forward() over the whole sequence; greedy generate()
  agrees with forward() on its own output;
* GraphedStep (the step captured into a HIP graph): six replays, with eager
  work and synchronisations between them, bit-identical to the eager step
  (logits and cache);
* decode_linear (ss_decode_linear): fixed and 24 seeded random shapes
  against the fp32 product and the unsplit kernel, the K split (tile
  counters back at zero, the same bits on a second call, graph replays)
  and the fused conv step (the bits of decode_linear followed by
  causal_conv1d_update); the fused RMSNorm (the bits of rms_norm_fn
  followed by decode_linear, output, residual stream and conv state).

Tolerances: fp32 1e-4 (outputs of a step, relative to the largest
magnitude where stated), bf16 / fp16 2e-2.
"""
import sys

import pytest
import torch

from oracle.decode_ref import causal_conv1d_update_ref, selective_state_update_ref
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def _say(msg):
    print(f"\n[decode] {msg}", flush=True)
    sys.stdout.flush()


SU_CASES = [
    # batch, dim, dstate, groups, dtype, z, D, bias, strided state
    (3, 48, 16, 1, torch.float32, True, True, True, False),
    (2, 64, 16, 2, torch.bfloat16, True, True, True, False),
    (4, 32, 5, 1, torch.float16, False, True, False, False),
    (1, 16, 16, 1, torch.float32, False, False, True, True),
    (16, 1536, 16, 1, torch.bfloat16, True, True, True, False),
]


@pytest.mark.parametrize("case", SU_CASES, ids=[f"b{c[0]}-d{c[1]}-n{c[2]}-g{c[3]}-{str(c[4]).split('.')[-1]}"
                                                f"{'-z' if c[5] else ''}{'-D' if c[6] else ''}"
                                                f"{'-bias' if c[7] else ''}{'-strided' if c[8] else ''}"
                                                for c in SU_CASES])
def test_state_update_matches_oracle(case):
    from mamba_amd.ops.selective_state_update import selective_state_update
    batch, dim, N, G, dt_, with_z, with_D, with_bias, strided = case
    _say(f"state update {case}")
    gen = torch.Generator().manual_seed(200 + dim + N)
    r = lambda *s: torch.randn(*s, generator=gen)
    x, dt, z = r(batch, dim).to(dt_), r(batch, dim).to(dt_), r(batch, dim).to(dt_)
    A = -torch.rand(dim, N, generator=gen) * 3
    B, C = r(batch, G, N).to(dt_), r(batch, G, N).to(dt_)
    D = r(dim)
    bias = r(dim) * 0.5
    state0 = r(batch, dim, N)
    if strided:   # every other dstate element of a wider buffer
        big = torch.zeros(batch, dim, 2 * N, device=DEV)
        big[..., ::2] = state0.to(DEV)
        st = big[..., ::2]
    else:
        st = state0.to(DEV).clone()
    out = selective_state_update(st, x.to(DEV), dt.to(DEV), A.to(DEV), B.to(DEV), C.to(DEV),
                                 D.to(DEV) if with_D else None, z=z.to(DEV) if with_z else None,
                                 dt_bias=bias.to(DEV) if with_bias else None, dt_softplus=True)
    want_out, want_st = selective_state_update_ref(state0, x, dt, A, B, C, D if with_D else None,
                                                   z=z if with_z else None, dt_bias=bias if with_bias else None,
                                                   dt_softplus=True)
    tol = TOL[dt_]
    assert_close(st.cpu(), want_st, 1e-5, 1e-5, "state")
    assert_close(out.cpu(), want_out.double(), tol, tol, "out")


@pytest.mark.parametrize("dt_", [torch.float32, torch.bfloat16])
def test_state_update_strided_B_C(dt_):
    """dstate 16 with a contiguous state (the path that loads state, A, B and C
    before the delta) but B and C as views with a dstate stride of 2 (element
    loads instead of 16-byte ones) against the oracle, and against the same
    call with contiguous copies of B and C (the same bits)."""
    from mamba_amd.ops.selective_state_update import selective_state_update
    _say(f"state update, strided B / C, {dt_}")
    gen = torch.Generator().manual_seed(321)
    r = lambda *s: torch.randn(*s, generator=gen)
    batch, dim, N = 3, 128, 16
    x, dt, z = r(batch, dim).to(dt_), r(batch, dim).to(dt_), r(batch, dim).to(dt_)
    A = -torch.rand(dim, N, generator=gen) * 3
    Bw, Cw = r(batch, 1, 2 * N).to(dt_), r(batch, 1, 2 * N).to(dt_)
    D, bias = r(dim), r(dim) * 0.5
    state0 = r(batch, dim, N)
    outs = []
    for strided in (True, False):
        Bd, Cd = Bw.to(DEV)[..., ::2], Cw.to(DEV)[..., ::2]
        if not strided:
            Bd, Cd = Bd.contiguous(), Cd.contiguous()
        st = state0.to(DEV).clone()
        out = selective_state_update(st, x.to(DEV), dt.to(DEV), A.to(DEV), Bd, Cd, D.to(DEV), z=z.to(DEV),
                                     dt_bias=bias.to(DEV), dt_softplus=True)
        outs.append((out, st))
    want_out, want_st = selective_state_update_ref(state0, x, dt, A, Bw[..., ::2], Cw[..., ::2], D, z=z,
                                                   dt_bias=bias, dt_softplus=True)
    tol = TOL[dt_]
    assert_close(outs[0][1].cpu(), want_st, 1e-5, 1e-5, "state")
    assert_close(outs[0][0].cpu(), want_out.double(), tol, tol, "out")
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1]), "strided vs contiguous B / C"


@pytest.mark.parametrize("dt_,rank", [(torch.float32, 48), (torch.bfloat16, 48), (torch.float16, 7)])
def test_state_update_low_rank_delta(dt_, rank):
    """dt given as (dt_low, dt_weight): the delta projection summed inside the
    kernel equals the oracle fed dt = dt_low @ dt_weight.T in float64, rounded
    to the input type as a dt tensor of that type is (the kernel rounds its
    fp32 sum the same way); dt_low is a column slice of a wider row.  Rank 48
    takes the 16-byte vector loads, rank 7 the element loads with an unpaired
    last term."""
    from mamba_amd.ops.selective_state_update import selective_state_update
    _say(f"state update, low-rank delta, rank {rank} {dt_}")
    gen = torch.Generator().manual_seed(500 + rank)
    r = lambda *s: torch.randn(*s, generator=gen)
    batch, dim, N = 5, 96, 16
    x, z = r(batch, dim).to(dt_), r(batch, dim).to(dt_)
    xdb = (0.3 * r(batch, rank + 2 * N)).to(dt_)          # x_proj output: [dt_low | B | C]
    w = (r(dim, rank) / rank ** 0.5).to(dt_)
    A = -torch.rand(dim, N, generator=gen) * 3
    B, C = r(batch, 1, N).to(dt_), r(batch, 1, N).to(dt_)
    D, bias = r(dim), r(dim) * 0.5
    state0 = r(batch, dim, N)
    st = state0.to(DEV).clone()
    xdb_d = xdb.to(DEV)
    out = selective_state_update(st, x.to(DEV), (xdb_d[:, :rank], w.to(DEV)), A.to(DEV), B.to(DEV), C.to(DEV),
                                 D.to(DEV), z=z.to(DEV), dt_bias=bias.to(DEV), dt_softplus=True)
    dt64 = (xdb[:, :rank].double() @ w.double().t()).to(dt_).double()
    want_out, want_st = selective_state_update_ref(state0.double(), x.double(), dt64, A.double(), B.double(),
                                                   C.double(), D.double(), z=z.double(), dt_bias=bias.double(),
                                                   dt_softplus=True)
    tol = TOL[dt_]
    assert_close(st.cpu().double(), want_st, 1e-4, 1e-4, "state")
    assert_close(out.cpu().double(), want_out.double(), tol, tol, "out")


@pytest.mark.parametrize("i", range(30))
def test_state_update_random(i):
    """Seeded random state updates: batch, dim, dstate (1 to 200), groups, dtype,
    z / D / bias, dt full or as the low-rank pair (any rank), B / C as column
    slices of the x-projection output, a strided state; against the float64
    oracle (a low-rank dt rounded to the input type first, as the kernel does).
    The kernel rounds its fp32 sum of the low-rank product, the oracle its
    float64 sum: where the two fall on either side of a rounding boundary of a
    16-bit type, dt differs by one unit in its last place (2^-8 relative for
    bf16) and the state by as much, so the state is then held to the input
    type's tolerance."""
    import random
    from mamba_amd.ops.selective_state_update import selective_state_update
    rnd = random.Random(3000 + i)
    batch = rnd.choice([1, 2, 5, 16, 33])
    N = rnd.choice([1, 4, 8, 16, 16, 16, 32, 64, 200])
    G = rnd.choice([1, 1, 2])
    dim = G * rnd.choice([1, 7, 16, 48, 96, 200])
    dt_ = rnd.choice([torch.float32, torch.bfloat16, torch.float16])
    with_z, with_D, with_bias = rnd.random() < 0.7, rnd.random() < 0.7, rnd.random() < 0.7
    rank = rnd.choice([0, 0, 1, 7, 16, 48, 64])
    strided = rnd.random() < 0.3
    _say(f"state update random {i}: batch {batch} dim {dim} dstate {N} groups {G} {dt_} z {with_z} D {with_D} "
         f"bias {with_bias} rank {rank} strided {strided}")
    gen = torch.Generator().manual_seed(3500 + i)
    r = lambda *s: torch.randn(*s, generator=gen)
    x, z = r(batch, dim).to(dt_), r(batch, dim).to(dt_)
    xdb = (0.3 * r(batch, rank + 2 * G * N)).to(dt_)       # [dt_low | B | C], B and C as column slices
    B = xdb[:, rank:rank + G * N].reshape(batch, G, N)
    C = xdb[:, rank + G * N:].reshape(batch, G, N)
    A = -torch.rand(dim, N, generator=gen) * 3
    D, bias = r(dim), r(dim) * 0.5
    state0 = r(batch, dim, N)
    if rank:
        w = (r(dim, rank) / rank ** 0.5).to(dt_)
        dt64 = (xdb[:, :rank].double() @ w.double().t()).to(dt_).double()
    else:
        dtv = r(batch, dim).to(dt_)
        dt64 = dtv.double()
    if strided:
        big = torch.zeros(batch, dim, 2 * N, device=DEV)
        big[..., ::2] = state0.to(DEV)
        st = big[..., ::2]
    else:
        st = state0.to(DEV).clone()
    xdb_d = xdb.to(DEV)
    Bd = xdb_d[:, rank:rank + G * N].view(batch, G, N)
    Cd = xdb_d[:, rank + G * N:].view(batch, G, N)
    dt_arg = (xdb_d[:, :rank], w.to(DEV)) if rank else dtv.to(DEV)
    out = selective_state_update(st, x.to(DEV), dt_arg, A.to(DEV), Bd, Cd, D.to(DEV) if with_D else None,
                                 z=z.to(DEV) if with_z else None, dt_bias=bias.to(DEV) if with_bias else None,
                                 dt_softplus=True)
    want_out, want_st = selective_state_update_ref(state0.double(), x.double(), dt64, A.double(), B.double(),
                                                   C.double(), D.double() if with_D else None,
                                                   z=z.double() if with_z else None,
                                                   dt_bias=bias.double() if with_bias else None, dt_softplus=True)
    tol = TOL[dt_]
    stol = 1e-4 if rank == 0 or dt_ == torch.float32 else tol
    assert_close(st.cpu().double(), want_st, stol, stol, "state")
    assert_close(out.cpu().double(), want_out.double(), tol, tol, "out")


@pytest.mark.parametrize("width,bias,act,dt_", [(4, True, "silu", torch.float32), (3, False, None, torch.float32),
                                                (1, True, "silu", torch.bfloat16), (2, True, "silu", torch.float16),
                                                (4, False, "silu", torch.bfloat16)])
def test_conv_update_matches_oracle(width, bias, act, dt_):
    from mamba_amd.ops.causal_conv1d import causal_conv1d_update
    _say(f"conv update width {width} bias {bias} act {act} {dt_}")
    gen = torch.Generator().manual_seed(300 + width)
    batch, dim = 3, 40
    x = torch.randn(batch, dim, generator=gen).to(dt_)
    st0 = torch.randn(batch, dim, width, generator=gen).to(dt_)
    w = torch.randn(dim, 1, width, generator=gen)
    b = torch.randn(dim, generator=gen) if bias else None
    st = st0.to(DEV).clone()
    out = causal_conv1d_update(x.to(DEV), st, w.to(DEV), b.to(DEV) if bias else None, act)
    want_out, want_st = causal_conv1d_update_ref(x.double(), st0.double(), w.double(),
                                                 b.double() if bias else None, act)
    assert torch.equal(st.cpu(), want_st.to(dt_)), "the conv state is shifted, not recomputed"
    tol = TOL[dt_]
    assert_close(out.cpu(), want_out, tol, tol, "out")


def test_state_updates_replay_the_scan():
    from mamba_amd.ops.selective_scan_interface import selective_scan_fn
    from mamba_amd.ops.selective_state_update import selective_state_update
    _say("token-by-token updates vs selective_scan_fn")
    torch.manual_seed(9)
    batch, dim, N, L = 2, 64, 16, 40
    u, delta, z = (torch.randn(batch, dim, L, device=DEV) for _ in range(3))
    A = -torch.rand(dim, N, device=DEV) * 3
    B, C = torch.randn(batch, 1, N, L, device=DEV), torch.randn(batch, 1, N, L, device=DEV)
    D, bias = torch.randn(dim, device=DEV), 0.3 * torch.randn(dim, device=DEV)
    want, last = selective_scan_fn(u, delta, A, B, C, D, z=z, delta_bias=bias, delta_softplus=True,
                                   return_last_state=True)
    st = torch.zeros(batch, dim, N, device=DEV)
    outs = [selective_state_update(st, u[..., t], delta[..., t], A, B[..., t], C[..., t], D, z=z[..., t],
                                   dt_bias=bias, dt_softplus=True) for t in range(L)]
    got = torch.stack(outs, -1)
    scale = float(want.abs().max())
    assert_close(got.cpu(), want.cpu(), 1e-4, 1e-4 * scale, "outputs")
    assert_close(st.cpu(), last.cpu(), 1e-4, 1e-4 * float(last.abs().max()), "last state")


@pytest.mark.parametrize("dt_", [torch.float32, torch.bfloat16])
def test_causal_lm_prefill_and_step_match_forward(dt_):
    from mamba_amd.models import CausalLM, CausalLMConfig
    _say(f"CausalLM prefill + step vs forward, {dt_}")
    torch.manual_seed(13)
    cfg = CausalLMConfig(vocab_size=101, model_dim=64, state_dim=16, num_layers=2, dropout_rate=0.0)
    lm = CausalLM(cfg).to(DEV).to(dt_).eval()
    with torch.no_grad():
        for layer in lm.layers:
            layer.norm.weight.uniform_(-0.3, 0.3)
    ids = torch.randint(0, cfg.vocab_size, (3, 50), device=DEV)
    P = 37                                              # prompt length (not a multiple of 16 or of the conv width)
    with torch.no_grad():
        full = lm(ids).float()
        cache = lm.allocate_inference_cache(3)
        pre = lm(ids[:, :P], inference_cache=cache).float()
        steps = [lm.step(ids[:, t], cache).float() for t in range(P, ids.shape[1])]
    scale = float(full.abs().max())
    tol = TOL[dt_]
    assert_close(pre.cpu(), full[:, :P].cpu(), tol, tol * scale, "prefill logits")
    assert_close(torch.stack(steps, 1).cpu(), full[:, P:].cpu(), tol, tol * scale, "step logits")


def test_generate_greedy_agrees_with_forward():
    from mamba_amd.models import CausalLM, CausalLMConfig
    _say("greedy generate vs forward")
    torch.manual_seed(14)
    cfg = CausalLMConfig(vocab_size=97, model_dim=64, state_dim=16, num_layers=2, dropout_rate=0.0)
    lm = CausalLM(cfg).to(DEV).eval()
    prompt = torch.randint(0, cfg.vocab_size, (2, 20), device=DEV)
    out = lm.generate(prompt, max_new_tokens=12, temperature=0)
    assert out.shape == (2, 32) and torch.equal(out[:, :20], prompt)
    with torch.no_grad():
        logits = lm(out).float()
    top2 = logits[:, 19:31].topk(2, dim=-1).values
    clear = (top2[..., 0] - top2[..., 1]) > 1e-3        # positions without a near tie
    assert torch.equal(logits[:, 19:31].argmax(-1)[clear], out[:, 20:32][clear])
    assert clear.float().mean() > 0.8
    # sampling: the right shape, tokens in range
    g = torch.Generator(device=DEV).manual_seed(0)
    s = lm.generate(prompt, max_new_tokens=5, temperature=0.8, generator=g)
    assert s.shape == (2, 25) and int(s.max()) < cfg.vocab_size and int(s.min()) >= 0


def test_graphed_step_replays_match_eager():
    # several replays, with eager work and synchronisations between them, each
    # checked against the eager step on an identical cache
    from mamba_amd.models import CausalLM, CausalLMConfig, GraphedStep
    _say("graph-captured step vs eager step")
    torch.manual_seed(15)
    cfg = CausalLMConfig(vocab_size=89, model_dim=64, state_dim=16, num_layers=2, dropout_rate=0.0)
    lm = CausalLM(cfg).to(DEV).eval()
    prompt = torch.randint(0, cfg.vocab_size, (4, 24), device=DEV)
    cache_g = lm.allocate_inference_cache(4)
    cache_e = lm.allocate_inference_cache(4)
    with torch.no_grad():
        lm(prompt, inference_cache=cache_g)
        lm(prompt, inference_cache=cache_e)
    step = GraphedStep(lm, cache_g, 4)
    for t in range(6):
        ids = torch.randint(0, cfg.vocab_size, (4,), device=DEV)
        got = step(ids).float().clone()
        torch.cuda.synchronize()
        with torch.no_grad():
            want = lm.step(ids, cache_e).float()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {t} differs from the eager step"
        for (c1, s1), (c2, s2) in zip(cache_g, cache_e):
            assert torch.equal(c1, c2) and torch.equal(s1, s2), f"cache after replay {t}"


LIN_CASES = [
    # batch, k_in, n_out, dtype, bias dtype (None: no bias), x as a column slice of a wider tensor
    (16, 768, 3072, torch.bfloat16, None, False),
    (16, 1536, 80, torch.bfloat16, None, False),
    (16, 48, 1536, torch.bfloat16, None, True),
    (5, 64, 37, torch.bfloat16, torch.float32, False),
    (33, 128, 100, torch.float16, torch.float16, False),
    (64, 1024, 50, torch.bfloat16, torch.bfloat16, True),
]


@pytest.mark.parametrize("case", LIN_CASES, ids=[f"b{c[0]}-k{c[1]}-n{c[2]}-{str(c[3]).split('.')[-1]}"
                                                  f"{'-bias' if c[4] is not None else ''}{'-slice' if c[5] else ''}"
                                                  for c in LIN_CASES])
def test_decode_linear_matches_fp32_product(case):
    # the matrix-core kernel (operand layouts, K split over waves, tails in n and batch)
    # against the same product in fp32
    from mamba_amd.ops.decode_linear import _fits, decode_linear
    batch, k, n, dt, bdt, sliced = case
    _say(f"decode linear {case}")
    gen = torch.Generator().manual_seed(400 + k + n)
    if sliced:
        wide = torch.randn(batch, k + 32, generator=gen).to(dt).to(DEV)
        x = wide[:, 16:16 + k]
    else:
        x = torch.randn(batch, k, generator=gen).to(dt).to(DEV)
    w = (torch.randn(n, k, generator=gen) / k ** 0.5).to(dt).to(DEV)
    b = torch.randn(n, generator=gen).to(bdt).to(DEV) if bdt is not None else None
    assert _fits(x, w, b), "this case must take the HIP kernel"
    y = decode_linear(x, w, b)
    want = x.float() @ w.float().t() + (b.float() if b is not None else 0.0)
    assert y.dtype == dt and y.shape == (batch, n)
    scale = float(want.abs().max())
    assert_close(y.float().cpu(), want.cpu(), 1e-2, 1e-2 * scale, "y")


SPLIT_CASES = [
    # batch, k_in, n_out, conv channels (0: none), bias dtype (None: no bias), dtype
    (16, 768, 3072, 1536, torch.bfloat16, torch.bfloat16),   # the block's input projection + conv (192 tiles: no split)
    (16, 1536, 80, 0, None, torch.bfloat16),                 # x-projection: 5 tiles, 4 slices
    (16, 1536, 768, 0, torch.bfloat16, torch.bfloat16),      # output projection: 48 tiles, 4 slices
    (16, 768, 1008, 256, torch.float32, torch.bfloat16),     # 63 tiles (the largest split shape), conv
    (5, 80, 37, 20, torch.float32, torch.float16),           # ragged tiles, 16-element K steps, 2 slices
    (33, 256, 64, 64, None, torch.bfloat16),                 # 3 batch tiles, 4 slices, the conv on every output
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[f"b{c[0]}-k{c[1]}-n{c[2]}-conv{c[3]}" for c in SPLIT_CASES])
def test_decode_linear_split_and_fused_conv(case):
    # K split over workgroups (last-arriving workgroup sums the partial tiles)
    # against the fp32 product and the unsplit kernel; the workspace counters
    # are back at zero after each call and a second call gives the same bits;
    # the fused conv step equals decode_linear followed by causal_conv1d_update
    # on the same product (outputs and conv state bit for bit)
    from mamba_amd.ops import decode_linear as dlm
    from mamba_amd.ops.causal_conv1d import causal_conv1d_update
    batch, k, n, cdim, bdt, dt = case
    _say(f"decode linear split {case}")
    gen = torch.Generator().manual_seed(500 + k + n)
    x = torch.randn(batch, k, generator=gen).to(dt).to(DEV)
    w = (torch.randn(n, k, generator=gen) / k ** 0.5).to(dt).to(DEV)
    b = torch.randn(n, generator=gen).to(bdt).to(DEV) if bdt is not None else None
    assert dlm._fits(x, w, b)
    want = x.float() @ w.float().t() + (b.float() if b is not None else 0.0)
    scale = float(want.abs().max())
    y1 = dlm.decode_linear(x, w, b)
    y0 = dlm.decode_linear(x, w, b, split=False)
    torch.cuda.synchronize()
    ws = dlm._workspaces[(DEV.index if DEV.index is not None else 0, torch.cuda.current_stream(DEV).cuda_stream)]
    tiles = ((n + 15) // 16) * ((batch + 15) // 16)
    assert int(ws[:tiles * 4].view(torch.int32).abs().sum()) == 0, "tile counters not reset"
    assert_close(y1.float().cpu(), want.cpu(), 1e-2, 1e-2 * scale, "split")
    assert_close(y0.float().cpu(), want.cpu(), 1e-2, 1e-2 * scale, "unsplit")
    assert torch.equal(dlm.decode_linear(x, w, b), y1), "split result differs between calls"
    if cdim:
        st0 = torch.randn(batch, cdim, 4, generator=gen).to(dt).to(DEV)
        cw = torch.randn(cdim, 4, generator=gen).to(DEV)
        cb = torch.randn(cdim, generator=gen).to(DEV)
        for split, ylin in ((True, y1), (False, y0)):
            st_f, st_r = st0.clone(), st0.clone()
            yf = dlm.decode_linear(x, w, b, conv=(st_f, cw, cb, "silu"), split=split)
            xr = causal_conv1d_update(ylin[:, :cdim].contiguous(), st_r, cw, cb, "silu")
            torch.cuda.synchronize()
            assert torch.equal(yf[:, :cdim], xr), f"fused conv output (split {split})"
            assert torch.equal(yf[:, cdim:], ylin[:, cdim:]), f"outputs past the conv channels (split {split})"
            assert torch.equal(st_f, st_r), f"conv state (split {split})"


def test_decode_linear_split_replays_in_a_graph():
    # the split kernel captured in a HIP graph (its workspace made before the
    # capture, on the capture stream): replays, with eager work between them,
    # give the eager bits
    from mamba_amd.ops import decode_linear as dlm
    _say("decode linear split in a graph")
    gen = torch.Generator().manual_seed(77)
    x = torch.randn(16, 1536, generator=gen).bfloat16().to(DEV)
    w = (torch.randn(400, 1536, generator=gen) / 40).bfloat16().to(DEV)     # 25 tiles, 4 slices
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = dlm.decode_linear(x, w)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = dlm.decode_linear(x, w)
    for rep in range(4):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {rep}"
        _ = (x.float() * 2).sum().item()


@pytest.mark.parametrize("i", range(24))
def test_decode_linear_random_shapes(i):
    # seeded random shapes through decode_linear (split or not, as the library
    # decides; the 16- and 8-byte load paths; ragged output and batch tiles;
    # with and without the fused conv step) against the fp32 product, the
    # unsplit kernel, and decode_linear followed by causal_conv1d_update (the
    # same bits)
    import random
    from mamba_amd.ops import decode_linear as dlm
    from mamba_amd.ops.causal_conv1d import causal_conv1d_update
    rnd = random.Random(700 + i)
    batch = rnd.choice([1, 2, 5, 16, 17, 33, 64])
    k = 16 * rnd.choice([1, 2, 3, 5, 8, 24, 48, 96, 128])
    n = rnd.choice([1, 7, 16, 37, 80, 200, 500, 1008, 1024])
    dt = rnd.choice([torch.bfloat16, torch.float16])
    bdt = rnd.choice([None, dt, torch.float32])
    cdim = rnd.choice([0, 0, n, max(1, n // 2)])
    width = rnd.choice([2, 3, 4])
    _say(f"decode linear random {i}: batch {batch} k {k} n {n} {dt} bias {bdt} conv {cdim} width {width}")
    gen = torch.Generator().manual_seed(800 + i)
    x = torch.randn(batch, k, generator=gen).to(dt).to(DEV)
    w = (torch.randn(n, k, generator=gen) / k ** 0.5).to(dt).to(DEV)
    b = torch.randn(n, generator=gen).to(bdt).to(DEV) if bdt is not None else None
    assert dlm._fits(x, w, b)
    want = x.float() @ w.float().t() + (b.float() if b is not None else 0.0)
    scale = max(1.0, float(want.abs().max()))
    y1 = dlm.decode_linear(x, w, b)
    y0 = dlm.decode_linear(x, w, b, split=False)
    assert_close(y1.float().cpu(), want.cpu(), 1e-2, 1e-2 * scale, "split")
    assert_close(y0.float().cpu(), want.cpu(), 1e-2, 1e-2 * scale, "unsplit")
    if cdim:
        st0 = torch.randn(batch, cdim, width, generator=gen).to(dt).to(DEV)
        cw = torch.randn(cdim, width, generator=gen).to(DEV)
        cb = torch.randn(cdim, generator=gen).to(DEV)
        st_f, st_r = st0.clone(), st0.clone()
        yf = dlm.decode_linear(x, w, b, conv=(st_f, cw, cb, "silu"))
        xr = causal_conv1d_update(y1[:, :cdim].contiguous(), st_r, cw, cb, "silu")
        torch.cuda.synchronize()
        assert torch.equal(yf[:, :cdim], xr), "fused conv output"
        assert torch.equal(yf[:, cdim:], y1[:, cdim:]), "outputs past the conv channels"
        assert torch.equal(st_f, st_r), "conv state"


NORM_CASES = [
    # batch, k_in, n_out, residual, norm weight dtype (None: the row dtype), conv channels, dtype
    (16, 768, 3072, True, None, 1536, torch.bfloat16),       # the LM block's norm + input projection + conv
    (16, 768, 3072, False, None, 1536, torch.bfloat16),      # the first block: no residual yet
    (5, 1024, 200, True, torch.float32, 0, torch.bfloat16),  # fp32 weight, ragged tiles, the largest fused k_in
    (33, 256, 64, True, None, 32, torch.float16),            # 3 batch tiles
    (16, 1536, 128, True, None, 0, torch.bfloat16),          # k_in above 1024: the RMSNorm kernel first
]


@pytest.mark.parametrize("case", NORM_CASES, ids=[f"b{c[0]}-k{c[1]}-n{c[2]}{'-res' if c[3] else ''}"
                                                  f"{'-w32' if c[4] else ''}-conv{c[5]}" for c in NORM_CASES])
def test_decode_linear_fused_norm(case):
    # the RMSNorm inside the product's launch against rms_norm_fn (prenorm)
    # followed by decode_linear: the same bits for the output, the residual
    # stream and the conv state
    from mamba_amd.ops import decode_linear as dlm
    from mamba_amd.ops.rms_norm import rms_norm_fn
    batch, k, n, with_res, wdt, cdim, dt = case
    _say(f"decode linear with fused norm {case}")
    gen = torch.Generator().manual_seed(900 + k + n + batch)
    x = torch.randn(batch, k, generator=gen).to(dt).to(DEV)
    res = torch.randn(batch, k, generator=gen).to(dt).to(DEV) if with_res else None
    nw = (0.1 * torch.randn(k, generator=gen)).to(wdt or dt).to(DEV)
    w = (torch.randn(n, k, generator=gen) / k ** 0.5).to(dt).to(DEV)
    b = torch.randn(n, generator=gen).to(dt).to(DEV)
    conv = None
    if cdim:
        st0 = torch.randn(batch, cdim, 4, generator=gen).to(dt).to(DEV)
        cw, cb = torch.randn(cdim, 4, generator=gen).to(DEV), torch.randn(cdim, generator=gen).to(DEV)
    st_f = st0.clone() if cdim else None
    y, s = dlm.decode_linear(x, w, b, conv=(st_f, cw, cb, "silu") if cdim else None, norm=(res, nw, 1e-5))
    normed, s_r = rms_norm_fn(x, nw, res, 1e-5, prenorm=True)
    st_r = st0.clone() if cdim else None
    # the fused launch (k_in up to 1024) does not split K, so the reference runs
    # unsplit; above that the op runs the RMSNorm kernel, then decode_linear as
    # usual (split where the library splits), and so does the reference
    fused = k <= 1024
    y_r = dlm.decode_linear(normed, w, b, conv=(st_r, cw, cb, "silu") if cdim else None, split=not fused)
    torch.cuda.synchronize()
    assert torch.equal(s, s_r), "residual stream"
    assert torch.equal(y, y_r), "output"
    if cdim:
        assert torch.equal(st_f, st_r), "conv state"
    want = normed.float() @ w.float().t() + b.float()
    assert_close(y[:, cdim:].float().cpu(), want[:, cdim:].cpu(), 1e-2, 1e-2 * float(want.abs().max()), "vs fp32")


@pytest.mark.parametrize("i", range(20))
def test_decode_linear_fused_norm_random(i):
    # seeded random shapes through the same bit-for-bit checks: batch 1 to 64,
    # k_in a multiple of 16 up to 1024 (and above, where the RMSNorm kernel runs
    # first), ragged output tiles, fp32 or row-dtype norm weight, with and
    # without residual and conv channels
    import random
    rnd = random.Random(1700 + i)
    batch = rnd.choice([1, 2, 5, 16, 17, 33, 64])
    k = 16 * rnd.choice([1, 3, 8, 24, 48, 64, 80])
    n = rnd.choice([16, 37, 80, 200, 512, 1008])
    cdim = rnd.choice([0, 0, n, max(1, n // 2)])
    case = (batch, k, n, rnd.random() < 0.7, rnd.choice([None, torch.float32]), cdim,
            rnd.choice([torch.bfloat16, torch.float16]))
    test_decode_linear_fused_norm(case)
