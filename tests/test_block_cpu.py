"""CPU checks of the Mamba-block oracle and the module mirrors (no GPU).

* causal_conv1d_ref against torch's conv1d configured as the reference
  configures it (nn.Conv1d(dim, dim, width, groups=dim, padding=width - 1),
  output cut to seqlen: modules/mamba_simple.py:40-47,100);
* mamba_simple_ref (the oracle of the whole block, from a parameter dict)
  against the reference's own op sequence (modules/mamba_simple.py:95-149)
  run on real nn.Linear / nn.Conv1d modules with the scan oracle in place of
  SelectiveScanFn;
* causal_lm_ref against the same op sequence stacked as models/causal_lm.py
  stacks it;
* the module mirrors carry the reference's state_dict keys and shapes.
"""
import pytest
import torch
import torch.nn.functional as F

from mamba_amd.models import CausalLM, CausalLMConfig
from mamba_amd.modules import MambaSimple, RMSNorm
from oracle.mamba_block_ref import causal_conv1d_ref, causal_lm_ref, mamba_inner_ref, mamba_simple_ref, rms_norm_ref
from oracle.selective_scan_ref import selective_scan_ref

F64 = torch.float64


@pytest.mark.parametrize("width", [1, 2, 3, 4])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("act", [None, "silu"])
def test_conv_oracle_matches_torch_conv1d(width, bias, act):
    g = torch.Generator().manual_seed(width)
    dim, L = 6, 23
    x = torch.randn(3, dim, L, generator=g, dtype=F64)
    conv = torch.nn.Conv1d(dim, dim, width, padding=width - 1, groups=dim, bias=bias).double()
    want = conv(x)[..., :L]
    if act:
        want = F.silu(want)
    got = causal_conv1d_ref(x, conv.weight, conv.bias, activation=act)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


def _reference_forward(m, hidden):
    """modules/mamba_simple.py:95-149 on module m, scan oracle for SelectiveScanFn."""
    batch_size, seq_len, _ = hidden.shape
    state_inputs, gate_logits = torch.chunk(m.input_proj(hidden).permute(0, 2, 1).contiguous(), chunks=2, dim=1)
    state_inputs = m.act(m.short_conv(state_inputs)[..., :seq_len])
    ssm_params = m.ssm_param_proj(state_inputs.permute(0, 2, 1).contiguous().view(batch_size * seq_len, m.inner_dim))
    delta, B, C = torch.split(ssm_params, [m.delta_rank, m.state_dim, m.state_dim], dim=-1)
    delta = m.delta_proj.weight @ delta.t()
    delta = delta.view(m.inner_dim, batch_size, seq_len).permute(1, 0, 2).contiguous()
    B = B.view(batch_size, seq_len, m.state_dim).permute(0, 2, 1).contiguous().unsqueeze(1)
    C = C.view(batch_size, seq_len, m.state_dim).permute(0, 2, 1).contiguous().unsqueeze(1)
    A = -torch.exp(m.log_A.double())
    y = selective_scan_ref(state_inputs, delta, A, B, C, m.D.double(), delta_bias=m.delta_proj.bias.double(),
                           delta_softplus=True, compute_dtype=F64)
    h = y.permute(0, 2, 1).contiguous() * m.act(gate_logits.permute(0, 2, 1).contiguous())
    return m.output_proj(h)


@pytest.mark.parametrize("bias,conv_bias", [(False, False), (True, True)])
def test_block_oracle_matches_reference_op_sequence(bias, conv_bias):
    torch.manual_seed(0)
    m = MambaSimple(model_dim=16, state_dim=4, conv_kernel=4, expansion_factor=2, bias=bias,
                    conv_bias=conv_bias).double()
    hidden = torch.randn(2, 11, 16, dtype=F64)
    want = _reference_forward(m, hidden)
    got = mamba_simple_ref({k: v for k, v in m.state_dict().items()}, hidden, state_dim=4)
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-12)


def test_causal_lm_oracle_matches_reference_structure():
    torch.manual_seed(1)
    cfg = CausalLMConfig(vocab_size=37, model_dim=16, state_dim=4, num_layers=2)
    model = CausalLM(cfg).double().eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 9))
    with torch.no_grad():
        h = model.embedding(ids)
        for blk in model.layers:
            h = h + _reference_forward(blk.mamba, rms_norm_ref(h, blk.norm.weight))
        want = model.lm_head(rms_norm_ref(h, model.norm.weight))
        got = causal_lm_ref(model.state_dict(), ids, num_layers=2, state_dim=4)
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-12)


def test_rms_norm_module_matches_oracle():
    torch.manual_seed(2)
    n = RMSNorm(24)
    with torch.no_grad():
        n.weight.uniform_(-0.5, 0.5)
    x = torch.randn(3, 5, 24)
    assert torch.allclose(n(x), rms_norm_ref(x, n.weight), rtol=1e-6, atol=1e-6)
    # closed form: a constant row c normalises to sign(c) * (1 + w) when eps is negligible
    x = torch.full((1, 1, 24), -3.0)
    assert torch.allclose(n(x)[0, 0], -(1 + n.weight.detach()), rtol=1e-5, atol=1e-5)


def test_rms_norm_oracle_matches_torch_rms_norm():
    # a library routine: F.rms_norm(x, (dim,), weight, eps) = x * rsqrt(mean(x^2) + eps) * weight
    from oracle.mamba_block_ref import add_rms_norm_ref
    torch.manual_seed(3)
    w = torch.empty(48).uniform_(-0.5, 0.5)
    x = torch.randn(7, 48) * 3
    want = torch.nn.functional.rms_norm(x, (48,), weight=1 + w, eps=1e-6)
    assert torch.allclose(rms_norm_ref(x, w), want, rtol=1e-6, atol=1e-6)
    # scale invariance (eps negligible) and unit mean square with weight 0
    assert torch.allclose(rms_norm_ref(x * 37.0, w), rms_norm_ref(x, w), rtol=1e-5, atol=1e-5)
    assert torch.allclose(rms_norm_ref(x, torch.zeros(48)).pow(2).mean(-1), torch.ones(7), rtol=1e-5)
    # bf16: normalised in fp32 and rounded once (not a bf16 computation)
    xb = x.bfloat16()
    want_b = torch.nn.functional.rms_norm(xb.float(), (48,), weight=1 + w, eps=1e-6).bfloat16()
    assert torch.equal(rms_norm_ref(xb, w), want_b)
    # residual add: s is the dtype's sum (rounded once), the norm is of s
    r = torch.randn(7, 48).bfloat16()
    out, s = add_rms_norm_ref(xb, r, w)
    assert torch.equal(s, (xb.float() + r.float()).bfloat16())
    assert torch.equal(out, rms_norm_ref(s, w))
    out0, s0 = add_rms_norm_ref(xb, None, w)
    assert s0 is xb and torch.equal(out0, rms_norm_ref(xb, w))


def test_rms_norm_oracle_gradient_matches_finite_differences():
    # the GPU backward is checked against autograd of rms_norm_ref in float64;
    # gradcheck pins that autograd against central differences
    from oracle.mamba_block_ref import add_rms_norm_ref
    torch.manual_seed(4)
    x = torch.randn(3, 10, dtype=torch.float64, requires_grad=True)
    r = torch.randn(3, 10, dtype=torch.float64, requires_grad=True)
    w = (0.3 * torch.randn(10, dtype=torch.float64)).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b, c: add_rms_norm_ref(a, b, c), (x, r, w))


@pytest.mark.parametrize("groups,with_z,with_D", [(1, True, True), (2, False, True), (1, True, False)])
def test_state_update_oracle_replays_the_scan(groups, with_z, with_D):
    # a step applied token after token from a zero state is the scan: every output and
    # the last state of selective_scan_ref (a different formulation: exp of the whole
    # (L, N) grid, then a sequential sum)
    from oracle.decode_ref import selective_state_update_ref
    from oracle.selective_scan_ref import selective_scan_ref
    torch.manual_seed(5)
    batch, dim, N, L = 2, 8, 4, 13
    u = torch.randn(batch, dim, L, dtype=torch.float64)
    delta = torch.randn(batch, dim, L, dtype=torch.float64)
    z = torch.randn(batch, dim, L, dtype=torch.float64) if with_z else None
    A = -torch.rand(dim, N, dtype=torch.float64) * 2
    B = torch.randn(batch, groups, N, L, dtype=torch.float64)
    C = torch.randn(batch, groups, N, L, dtype=torch.float64)
    D = torch.randn(dim, dtype=torch.float64) if with_D else None
    bias = torch.randn(dim, dtype=torch.float64) * 0.3
    want, last = selective_scan_ref(u, delta, A, B, C, D, z=z, delta_bias=bias, delta_softplus=True,
                                    return_last_state=True, compute_dtype=torch.float64)
    h = torch.zeros(batch, dim, N, dtype=torch.float64)
    outs = []
    for t in range(L):
        y, h = selective_state_update_ref(h, u[..., t], delta[..., t], A, B[..., t], C[..., t], D,
                                          z=z[..., t] if with_z else None, dt_bias=bias, dt_softplus=True)
        outs.append(y)
    assert torch.allclose(torch.stack(outs, -1), want, rtol=1e-12, atol=1e-12)
    assert torch.allclose(h, last, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("width", [1, 2, 4])
def test_conv_update_oracle_replays_the_conv(width):
    from oracle.decode_ref import causal_conv1d_update_ref
    torch.manual_seed(6)
    x = torch.randn(2, 5, 9, dtype=torch.float64)
    w = torch.randn(5, width, dtype=torch.float64)
    b = torch.randn(5, dtype=torch.float64)
    want = causal_conv1d_ref(x, w, b, activation="silu")
    st = torch.zeros(2, 5, width, dtype=torch.float64)
    outs = []
    for t in range(x.shape[-1]):
        y, st = causal_conv1d_update_ref(x[..., t], st, w, b, "silu")
        outs.append(y)
    assert torch.allclose(torch.stack(outs, -1), want, rtol=1e-12, atol=1e-12)
    assert torch.equal(st, x[..., -width:])                 # the state is the last width inputs


def test_state_dict_keys_are_the_references():
    # parameter names and shapes of models/causal_lm.py:21-51 and modules/mamba_simple.py:35-85
    cfg = CausalLMConfig(vocab_size=50, model_dim=24, state_dim=16, conv_kernel=4, num_layers=2)
    sd = CausalLM(cfg).state_dict()
    inner, rank = 48, 2          # expansion 2; delta rank ceil(24 / 16)
    want = {"embedding.weight": (50, 24), "norm.weight": (24,), "lm_head.weight": (50, 24)}
    for i in range(2):
        p = f"layers.{i}."
        want.update({
            p + "norm.weight": (24,),
            p + "mamba.input_proj.weight": (2 * inner, 24),
            p + "mamba.short_conv.weight": (inner, 1, 4),
            p + "mamba.ssm_param_proj.weight": (rank + 32, inner),
            p + "mamba.delta_proj.weight": (inner, rank),
            p + "mamba.delta_proj.bias": (inner,),
            p + "mamba.log_A": (inner, 16),
            p + "mamba.D": (inner,),
            p + "mamba.output_proj.weight": (24, inner),
        })
    assert {k: tuple(v.shape) for k, v in sd.items()} == want
    m = CausalLM(cfg)
    assert m.lm_head.weight is m.embedding.weight


def test_initialisation_matches_reference_rules():
    torch.manual_seed(3)
    m = MambaSimple(model_dim=32, state_dim=16)
    A = torch.exp(m.log_A.detach())
    assert torch.allclose(A, torch.arange(1, 17, dtype=torch.float32).expand(64, 16))
    assert torch.all(m.D.detach() == 1)
    dt = F.softplus(m.delta_proj.bias.detach())          # inverse softplus of dt in [1e-3, 1e-1]
    assert float(dt.min()) >= 1e-3 * 0.999 and float(dt.max()) <= 1e-1 * 1.001
    bound = m.delta_rank ** -0.5
    assert float(m.delta_proj.weight.detach().abs().max()) <= bound


def test_c_scan_autograd_matches_scan_oracle():
    """c_oracle.scan (the float64 C restatement as an autograd function, used by
    the block and model oracles on long sequences) gives selective_scan_ref's
    output and, through autograd, its gradients; a Mamba block differentiated
    through either scan agrees too."""
    from oracle import c_oracle
    from oracle.selective_scan_ref import make_inputs, selective_scan_ref
    x = make_inputs(2, 24, 8, 40, seed=31)
    names = ("u", "delta", "A", "B", "C", "D", "z", "delta_bias")
    a = {k: x[k].double().requires_grad_(True) for k in names}
    b = {k: x[k].double().requires_grad_(True) for k in names}
    oa = selective_scan_ref(*(a[k] for k in names[:6]), z=a["z"], delta_bias=a["delta_bias"],
                            delta_softplus=True, compute_dtype=torch.float64)
    ob = c_oracle.scan(*(b[k] for k in names[:6]), z=b["z"], delta_bias=b["delta_bias"], delta_softplus=True)
    assert torch.allclose(oa, ob, rtol=1e-10, atol=1e-10)
    dout = x["dout"].double()
    oa.backward(dout)
    ob.backward(dout)
    for k in names:
        assert torch.allclose(a[k].grad, b[k].grad, rtol=1e-9, atol=1e-9), k

    torch.manual_seed(3)
    batch, d_model, dim, L, R, N = 2, 16, 32, 24, 4, 8
    xz = torch.randn(batch, 2 * dim, L, dtype=torch.float64)
    w = [torch.randn(dim, 1, 4, dtype=torch.float64) * 0.3, torch.randn(dim, dtype=torch.float64) * 0.1,
         torch.randn(R + 2 * N, dim, dtype=torch.float64) * dim ** -0.5,
         torch.rand(dim, R, dtype=torch.float64) * R ** -0.5, torch.randn(d_model, dim, dtype=torch.float64) * 0.2,
         None, -torch.arange(1, N + 1, dtype=torch.float64).repeat(dim, 1)]
    grads = []
    for scan in (None, c_oracle.scan):
        xg = xz.clone().requires_grad_(True)
        ws = [t.clone().requires_grad_(True) if t is not None else None for t in w]
        out = mamba_inner_ref(xg, *ws, D=torch.ones(dim, dtype=torch.float64),
                              delta_bias=torch.full((dim,), -2.0, dtype=torch.float64), scan=scan)
        out.pow(2).sum().backward()
        grads.append([xg.grad] + [t.grad for t in ws if t is not None])
    for ga, gb in zip(*grads):
        assert torch.allclose(ga, gb, rtol=1e-9, atol=1e-9)
