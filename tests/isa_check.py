"""Static checks over the gfx950 disassembly of libmamba_ss.so.

The scan kernels issue some DPP row broadcasts as inline asm (bmul / bfmac
in ss_device.hpp), where the compiler's hazard recognizer does not look.
These checks re-derive, from the disassembled code object, the rules such
asm must keep:

* DPP source wait states: a VALU write of a VGPR followed by a DPP
  instruction that reads it as src0 needs at least 2 wait states between
  them (each issued instruction counts as one, s_nop N as N + 1);
* transcendental forwarding: the result of v_exp / v_log / v_rcp / v_rsq /
  v_sqrt / v_sin / v_cos read by a non-transcendental VALU needs at least
  1 wait state;
* wide store data: a store of more than 8 bytes (dwordx3 / dwordx4) reads
  its data VGPRs after issue, so a VALU write to one of them needs at least
  2 wait states after the store.  The compiler skips this for buffer stores
  whose uniform offset is a register, so the kernels avoid that form; the
  check covers every wide store;
* no packed fp32 VALU ops (v_pk_fma_f32, v_pk_mul_f32, v_pk_add_f32): the
  library is built with them disabled;
* no waterfall loop inside a scan kernel's main loop: a buffer resource or
  uniform offset the compiler holds in VGPRs makes every access through it a
  loop of v_readfirstlane / v_cmp / s_and_saveexec / s_cbranch_execnz, which
  in the per-chunk loop costs dozens of issue slots per chunk.

The scan is linear over each function's instruction stream, the order the
compiler laid out; a branch instruction counts as one wait state like any
other.  Only the library's own build is disassembled.
"""
import os
import re
import shutil
import subprocess

LLVM_BIN = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
TRANS = re.compile(r"^v_(exp|log|rcp|rsq|sqrt|sin|cos)_")
WIDE_STORE = re.compile(r"^(buffer|global|flat|scratch)_store_dwordx[34]$")
PACKED_F32 = re.compile(r"^v_pk_(fma|mul|add)_f32")


def tools_available():
    return all(os.path.exists(os.path.join(LLVM_BIN, t))
               for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"))


MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def disassemble(lib_path, workdir):
    """gfx950 disassembly (text) of the device code embedded in lib_path:
    the .hip_fatbin section holds one offload bundle per source file."""
    fat = os.path.join(workdir, "fatbin.bin")
    subprocess.run([os.path.join(LLVM_BIN, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", lib_path,
                    os.path.join(workdir, "stripped.so")], check=True, capture_output=True)
    data = open(fat, "rb").read()
    starts, i = [], data.find(MAGIC)
    while i >= 0:
        starts.append(i)
        i = data.find(MAGIC, i + len(MAGIC))
    texts = []
    for k, st in enumerate(starts):
        end = starts[k + 1] if k + 1 < len(starts) else len(data)
        part = os.path.join(workdir, f"bundle{k}.bin")
        co = os.path.join(workdir, f"co{k}.o")
        with open(part, "wb") as f:
            f.write(data[st:end])
        subprocess.run([os.path.join(LLVM_BIN, "clang-offload-bundler"), "--unbundle", "--type=o",
                        f"--input={part}", f"--targets={TARGET}", f"--output={co}"], check=True,
                       capture_output=True)
        res = subprocess.run([os.path.join(LLVM_BIN, "llvm-objdump"), "-d", "--mcpu=gfx950", co],
                             check=True, capture_output=True, text=True)
        texts.append(res.stdout)
    shutil.rmtree(workdir, ignore_errors=True)
    return "\n".join(texts)


def _vregs(tok):
    tok = tok.strip()
    m = re.match(r"^v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"^v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def functions(disasm):
    """{name: [instruction text, ...]} from llvm-objdump output."""
    out, cur = {}, None
    for line in disasm.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            cur = out.setdefault(m.group(1), [])
            continue
        if cur is None:
            continue
        text = line.split("//")[0].strip()
        if text and not text.endswith(":"):
            cur.append(text)
    return out


def function_code(disasm):
    """{name: [(address, instruction text), ...]} from llvm-objdump output;
    branch instructions keep their target as "<name+0xoff>"."""
    out, cur, start = {}, None, 0
    for line in disasm.splitlines():
        m = re.match(r"^([0-9a-f]+) <(\S+)>:", line)
        if m:
            start = int(m.group(1), 16)
            cur = out.setdefault(m.group(2), [])
            continue
        if cur is None:
            continue
        parts = line.split("//", 1)
        text = parts[0].strip()
        if not text or text.endswith(":") or len(parts) < 2:
            continue
        m = re.match(r"\s*([0-9A-Fa-f]+):", parts[1])
        if not m:
            continue
        t = re.search(r"<\S+\+0x([0-9a-f]+)>", parts[1])
        cur.append((int(m.group(1), 16), text + (f" <{start + int(t.group(1), 16)}>" if t else "")))
    return out


def _target(text):
    m = re.search(r"<(\d+)>$", text)
    return int(m.group(1)) if m else None


def loops(code):
    """(start, end) address ranges closed by a backward branch.  Blocks the
    compiler places after s_endpgm jump back into the body without forming
    a loop; branches from there are left out."""
    out = []
    for addr, text in code:
        if text.startswith("s_endpgm"):
            break
        if text.startswith(("s_branch", "s_cbranch")):
            t = _target(text)
            if t is not None and t <= addr:
                out.append((t, addr))
    return out


def waterfall_loops(code):
    """Backward s_cbranch_execnz loops whose body reads a lane into an SGPR
    (v_readfirstlane) and narrows exec (s_and_saveexec): the compiler's
    waterfall loops around a VGPR-held resource or offset."""
    out = []
    for t, end in loops(code):
        body = [text for addr, text in code if t <= addr <= end]
        if body and body[-1].startswith("s_cbranch_execnz") and \
                any(x.startswith("v_readfirstlane") for x in body) and any("saveexec" in x for x in body):
            out.append((t, end))
    return out


def waterfalls_in_main_loop(code):
    """Waterfall loops inside the function's largest loop."""
    ls = loops(code)
    if not ls:
        return []
    s0, e0 = max(ls, key=lambda r: r[1] - r[0])
    return [(s, e) for s, e in waterfall_loops(code) if s0 <= s and e <= e0 and (s, e) != (s0, e0)]


def _split(text):
    parts = text.split(None, 1)
    op = parts[0]
    rest = parts[1] if len(parts) > 1 else ""
    # operands end where the modifiers (row_*, quad_perm, *_mask, bound_ctrl, offset...) begin
    ops = []
    for tok in rest.split(","):
        tok = tok.strip()
        head = tok.split()[0] if tok else ""
        ops.append(head)
    return op, ops


def check_function(name, insns):
    """List of (kind, message) problems found in one function."""
    problems = []
    hist = []           # (op, vgprs written, wait states it provides)
    stores = []         # (wide store op or None, its data vgprs, wait states it provides)
    for text in insns:
        op, ops = _split(text)
        if op == "s_nop":
            hist.append((op, set(), int(ops[0], 0) + 1))
            stores.append((None, set(), int(ops[0], 0) + 1))
            continue
        if PACKED_F32.match(op):
            problems.append(("packed-fp32", f"{name}: {text}"))
        srcs = [_vregs(o) for o in ops[1:]]
        is_dpp = op.startswith("v_") and ("row_" in text or "quad_perm" in text or "_dpp" in op)
        if is_dpp and srcs:
            ws = 0
            for hop, hdst, hw in reversed(hist):
                if ws >= 2:
                    break
                if hdst & srcs[0] and hop.startswith("v_"):
                    problems.append(("dpp", f"{name}: '{text}' reads v{sorted(hdst & srcs[0])} "
                                            f"written by {hop} {ws} wait state(s) before"))
                    break
                ws += hw
        if op.startswith("v_") and not TRANS.match(op):
            used = set().union(*srcs) if srcs else set()
            if op.startswith(("v_fmac", "v_mac")) and ops:
                used |= _vregs(ops[0])
            if hist:
                hop, hdst, _ = hist[-1]
                if TRANS.match(hop) and hdst & used:
                    problems.append(("trans", f"{name}: '{text}' reads v{sorted(hdst & used)} "
                                              f"straight after {hop}"))
        writes_vgpr = op.startswith("v_") and not op.startswith(("v_cmp", "v_readlane", "v_readfirstlane"))
        dst = _vregs(ops[0]) if (writes_vgpr and ops) else set()
        if dst:
            ws = 0
            for hop, hdata, hw in reversed(stores):
                if ws >= 2:
                    break
                if hop is not None and hdata & dst:
                    problems.append(("store-data", f"{name}: '{text}' overwrites v{sorted(hdata & dst)} "
                                                   f"{ws} wait state(s) after {hop}"))
                    break
                ws += hw
        if WIDE_STORE.match(op) and ops:
            data = _vregs(ops[0] if op.startswith("buffer_") else ops[1])
            stores.append((op, data, 1))
        else:
            stores.append((None, set(), int(ops[0], 0) + 1 if op == "s_nop" else 1))
        del stores[:-8]
        hist.append((op, dst, 1))
        del hist[:-8]
    return problems
