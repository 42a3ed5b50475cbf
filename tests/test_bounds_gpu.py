"""Every scan output stays inside its array.

Each output of the forward and backward (out, y, x, du, ddelta, dz, dB, dC,
dA, dD, ddelta_bias) and every sequence input is placed inside a larger
buffer between two guard regions filled with a sentinel value; the sequence
tensors also get padded rows (a row stride larger than seqlen, the padding
filled with the sentinel too).  After a forward + backward through the C
ABI (``forward_into`` / ``backward_into``) every guard and every row
padding still holds the sentinel, and the results equal those of a run on
plain contiguous tensors (the same bits for everything but the atomic
sums).  Cases: the fast kernels at an aligned and a ragged seqlen, bf16
with two workspace slices, sequence segments, and a ragged fp16 call
without workspace (dB / dC added straight into their rows).
"""
import sys

import pytest
import torch

from oracle.selective_scan_ref import make_inputs
from tests._util import assert_close

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GUARD = 4096          # elements before and after each array
SENT = -7777.0        # exact in fp32, bf16 and fp16


class Guarded:
    """A tensor view of `shape` inside a sentinel-filled buffer; sequence
    tensors (3-d, last dim seqlen) get rows of seqlen + pad elements."""

    def __init__(self, shape, dtype, pad=0):
        shape = tuple(shape)
        if len(shape) == 3 and pad:
            b, d, L = shape
            n = b * d * (L + pad)
            self.buf = torch.full((2 * GUARD + n,), SENT, dtype=dtype, device=DEV)
            self.view = self.buf[GUARD:GUARD + n].view(b, d, L + pad)[..., :L]
        else:
            n = 1
            for s in shape:
                n *= s
            self.buf = torch.full((2 * GUARD + n,), SENT, dtype=dtype, device=DEV)
            self.view = self.buf[GUARD:GUARD + n].view(shape)
        self.used = torch.zeros(self.buf.shape, dtype=torch.bool, device=DEV)
        flat = self.used[GUARD:GUARD + n]
        if len(shape) == 3 and pad:
            flat.view(b, d, L + pad)[..., :L] = True
        else:
            flat[:] = True

    def untouched(self):
        """True when every element outside the view still holds SENT."""
        rest = self.buf[~self.used]
        return bool((rest == SENT).all())


def _say(msg):
    print(f"\n[bounds] {msg}", flush=True)
    sys.stdout.flush()


def _run(x, dtype, guarded, pad, workspace):
    from mamba_amd import selective_scan as ss
    batch, dim, L = x["u"].shape
    dstate = x["A"].shape[1]
    g = {}

    def mk(name, shape, dt, init=None, seq=False):
        if guarded:
            t = Guarded(shape, dt, pad if seq else 0)
            g[name] = t
            v = t.view
        else:
            v = torch.empty(shape, dtype=dt, device=DEV)
        if init is not None:
            v.copy_(init)
        return v

    seq = {k: mk(k, x[k].shape, x[k].dtype, x[k], seq=True) for k in ("u", "delta", "z")}
    dout = mk("dout", x["dout"].shape, x["dout"].dtype, x["dout"], seq=True)
    A, B, C, D, bias = (x[k].to(DEV) for k in ("A", "B", "C", "D", "delta_bias"))
    out = mk("out", (batch, dim, L), dtype, seq=True)
    y = mk("y", (batch, dim, L), dtype, seq=True)
    xck = mk("x", (batch, ss.n_chunks(L), dim, dstate), torch.float32)
    ss.forward_into(seq["u"], seq["delta"], A, B, C, D, bias, True, out, xck, z=seq["z"], y=y,
                    workspace=workspace)
    du = mk("du", (batch, dim, L), dtype, seq=True)
    dd = mk("ddelta", (batch, dim, L), dtype, seq=True)
    dz = mk("dz", (batch, dim, L), dtype, seq=True)
    grads = {k: mk("d" + k, x[k].shape, torch.float32) for k in ("A", "B", "C", "D", "delta_bias")}
    ss.backward_into(seq["u"], seq["delta"], A, B, C, D, bias, dout, xck, True, du, dd,
                     grads["A"], grads["B"], grads["C"], grads["D"], grads["delta_bias"],
                     z=seq["z"], y=y, dz=dz, workspace=workspace, zero_grads=True)
    torch.cuda.synchronize()
    res = {"out": out, "y": y, "x": xck, "du": du, "ddelta": dd, "dz": dz}
    res.update({"d" + k: v for k, v in grads.items()})
    return {k: v.clone() for k, v in res.items()}, g


# (batch, dim, seqlen, dtype, workspace): aligned fast kernels; ragged seqlen
# (partial and padded chunks, a padded dB / dC slice); bf16 with two workspace
# slices (192 channel blocks); one long sequence (sequence segments); ragged
# fp16 without workspace
CASES = [(2, 64, 256, torch.float32, "auto"), (2, 64, 1001, torch.float32, "auto"),
         (1, 3072, 130, torch.bfloat16, "auto"), (1, 32, 4096, torch.float32, "auto"),
         (2, 48, 333, torch.float16, None)]


@pytest.mark.parametrize("case", CASES, ids=["fast", "ragged", "bf16-slices", "segments", "fp16-no-ws"])
def test_outputs_stay_in_their_arrays(case):
    batch, dim, L, dtype, ws = case
    _say(f"batch {batch} dim {dim} seqlen {L} {dtype} workspace {ws}")
    x = make_inputs(batch, dim, 16, L, seed=700 + L, dtype=dtype)
    x = {k: v.to(DEV) for k, v in x.items()}
    want, _ = _run(x, dtype, guarded=False, pad=0, workspace=ws)
    got, g = _run(x, dtype, guarded=True, pad=5, workspace=ws)
    for name, t in g.items():
        assert t.untouched(), f"{name}: an element outside the array changed"
    for k in ("out", "y", "x", "du", "ddelta", "dz"):
        assert torch.equal(got[k], want[k]), k
    for k in ("dA", "dB", "dC", "dD", "ddelta_bias"):      # atomic sums: the order may differ
        w = want[k].float()
        assert_close(got[k].float().cpu(), w.cpu(), 1e-5, 1e-5 * max(1.0, float(w.abs().max())), k)


def test_ragged_tail_sums_stay_in_their_state_rows():
    # seqlen 333 (333 % 32 = 13) without workspace: dB / dC rows of seqlen
    # floats, a partial last chunk (steps 320..332) and a chunk wholly past
    # the sequence (336..351), whose sums go onto steps of the row.  An
    # infinite u at the last step makes the state infinite there, so the
    # identity steps past the sequence produce 0 * inf = NaN partial sums;
    # they must stay on the row's last step and never reach the first steps
    # of the next state row.
    from mamba_amd import selective_scan as ss
    batch, dim, L = 1, 16, 333
    _say(f"batch {batch} dim {dim} seqlen {L} float32 workspace None, inf at the last step")
    x = make_inputs(batch, dim, 16, L, seed=333)
    x = {k: v.to(DEV) for k, v in x.items()}
    x["u"][:, :, L - 1] = float("inf")
    out, y = torch.empty_like(x["u"]), torch.empty_like(x["u"])
    xck = torch.empty((batch, ss.n_chunks(L), dim, 16), device=DEV)
    ss.forward_into(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["delta_bias"], True, out, xck,
                    z=x["z"], y=y, workspace=None)
    du, dd, dz = torch.empty_like(out), torch.empty_like(out), torch.empty_like(out)
    dA = torch.empty(x["A"].shape, device=DEV)
    dB, dC = torch.empty(x["B"].shape, device=DEV), torch.empty(x["C"].shape, device=DEV)
    dD, db = torch.empty(dim, device=DEV), torch.empty(dim, device=DEV)
    ss.backward_into(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["delta_bias"], x["dout"], xck, True,
                     du, dd, dA, dB, dC, dD, db, z=x["z"], y=y, dz=dz, workspace=None, zero_grads=True,
                     deterministic=False)
    torch.cuda.synchronize()
    assert not torch.isfinite(xck[0, -1]).all(), "the state at the end should be infinite"
    for name, t in (("dB", dB), ("dC", dC)):
        assert torch.isfinite(t[..., :L - 1]).all(), f"{name}: a non-finite sum landed before the last step"
