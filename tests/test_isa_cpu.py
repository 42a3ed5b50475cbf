"""The built library's gfx950 code keeps the DPP / transcendental / wide-store
wait states its inline asm and buffer stores rely on and has no packed fp32
VALU ops (CPU only: disassembles the library, runs nothing)."""
import os
import tempfile

import pytest

from tests import isa_check

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "mamba_amd", "_lib",
                   "libmamba_ss.so")

pytestmark = pytest.mark.skipif(not (os.path.exists(LIB) and isa_check.tools_available()),
                                reason="library not built or ROCm LLVM tools missing")


@pytest.fixture(scope="module")
def funcs():
    return isa_check.functions(isa_check.disassemble(LIB, tempfile.mkdtemp()))


def test_every_scan_kernel_is_present(funcs):
    names = " ".join(funcs)
    for k in ("ss_fwd_fast", "ss_bwd_fast", "ss_fwd_kernel", "ss_bwd_kernel", "ss_zero_segs", "ss_ws_reduce"):
        assert k in names, k


def test_inline_asm_dpp_is_used(funcs):
    """The fused v_fmac_f32_dpp only comes from the inline asm: its presence
    shows the check below looks at the code it is meant for."""
    bwd = [f for f in funcs if "ss_bwd_fast" in f]
    assert bwd and all(any(i.startswith("v_fmac_f32_dpp") for i in funcs[f]) for f in bwd)


def test_no_hazards_and_no_packed_fp32(funcs):
    problems = []
    for name, insns in funcs.items():
        problems += isa_check.check_function(name, insns)
    assert not problems, "\n".join(f"{k}: {m}" for k, m in problems[:20])


@pytest.fixture(scope="module")
def code():
    return isa_check.function_code(isa_check.disassemble(LIB, tempfile.mkdtemp()))


def test_no_waterfall_loop_in_the_scan_main_loops(code):
    """The fast scan kernels keep every buffer resource and uniform offset of
    their per-chunk loop in SGPRs (no waterfall loop inside the main loop)."""
    fast = [f for f in code if "ss_fwd_fast" in f or "ss_bwd_fast" in f]
    assert len(fast) >= 4
    bad = {f: isa_check.waterfalls_in_main_loop(code[f]) for f in fast}
    assert not any(bad.values()), {f: v for f, v in bad.items() if v}


def test_waterfall_check_finds_a_planted_one():
    """A waterfall loop planted inside a main loop is found; the same loop
    after the main loop is not counted."""
    def asm(lines, start=0x1000):
        out = [f"{start:016x} <k>:"]
        for i, t in enumerate(lines):
            a = start + 4 * i
            tgt = ""
            if t.startswith(("s_branch", "s_cbranch")):
                tgt = f" <k+0x{4 * int(t.split('@')[1]):x}>"
                t = t.split("@")[0]
            out.append(f"\t{t}   // {a:012X}: 00000000{tgt}")
        return "\n".join(out)
    wf = ["v_readfirstlane_b32 s4, v0", "v_cmp_eq_u32_e32 vcc, s4, v0", "s_and_saveexec_b64 s[2:3], vcc",
          "buffer_store_dword v1, v2, s[4:7], 0 offen", "s_xor_b64 exec, exec, s[2:3]"]
    inside = ["v_mul_f32_e32 v1, v1, v3"] + wf + ["s_cbranch_execnz @1", "v_add_f32_e32 v1, v1, v3",
                                                   "s_cbranch_scc1 @0", "s_endpgm"]
    code_in = isa_check.function_code(asm(inside))["k"]
    assert len(isa_check.waterfalls_in_main_loop(code_in)) == 1
    after = ["v_mul_f32_e32 v1, v1, v3", "v_add_f32_e32 v1, v1, v3", "s_cbranch_scc1 @0"] + wf + \
            ["s_cbranch_execnz @3", "s_endpgm"]
    code_after = isa_check.function_code(asm(after))["k"]
    assert len(isa_check.waterfall_loops(code_after)) == 1
    assert isa_check.waterfalls_in_main_loop(code_after) == []


def test_isa_check_catches_planted_hazards():
    """isa_check itself flags a DPP read 1 wait state after the write, a
    transcendental result read at once, and a packed fp32 op."""
    bad = ["v_mul_f32_e32 v1, 0x40400000, v1",
           "s_waitcnt vmcnt(2)",
           "v_mul_f32_dpp v2, v1, v2 row_newbcast:3 row_mask:0xf bank_mask:0xf",
           "v_exp_f32_e32 v5, v2",
           "v_add_f32_e32 v6, v5, v6",
           "v_pk_fma_f32 v[8:9], v[8:9], v[10:11], v[12:13]"]
    kinds = sorted(k for k, _ in isa_check.check_function("planted", bad))
    assert kinds == ["dpp", "packed-fp32", "trans"]
    store = ["buffer_store_dwordx4 v[58:61], v66, s[20:23], s2 offen",
             "v_mul_f32_e32 v58, v122, v58"]
    assert [k for k, _ in isa_check.check_function("store", store)] == ["store-data"]
    store_ok = ["buffer_store_dwordx4 v[58:61], v66, s[20:23], 0 offen",
                "v_mul_f32_e32 v123, 0xbfb8aa3b, v119",
                "v_exp_f32_e32 v123, v123",
                "v_mul_f32_e32 v58, v122, v58"]
    assert isa_check.check_function("store_ok", store_ok) == []
    good = ["v_mul_f32_e32 v1, 0x40400000, v1",
            "s_nop 1",
            "v_mul_f32_dpp v2, v1, v2 row_newbcast:3 row_mask:0xf bank_mask:0xf",
            "v_exp_f32_e32 v5, v2",
            "s_nop 0",
            "v_add_f32_e32 v6, v5, v6"]
    assert isa_check.check_function("clean", good) == []
