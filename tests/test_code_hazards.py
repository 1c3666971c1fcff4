"""The built gfx950 code object against the wait states an MFMA needs after a VALU write of its sources (no GPU).

A VALU instruction that writes a VGPR must be followed by at least two wait states (instructions, or s_nop N counting
N + 1) before an MFMA reads that VGPR as its A, B or C operand. The compiler inserts them for instructions it
emits itself; an inline-asm block's outputs are invisible to its hazard recognizer, so a kernel whose asm output
feeds an MFMA directly can read a stale register, and whether it does depends on how the waves interleave. The
kernels keep the last VALU step before an MFMA operand out of the asm (the decode's fp16 fma), and this test holds
both libraries to the rule: it unbundles each one's gfx950 code object, disassembles it, and walks back from
every MFMA within its straight-line code.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBS = [os.path.join(ROOT, "radiance-exl3_amd", n) for n in ("libexl3c4.so", "libexl3c4_calib.so")]
LLVM = "/opt/rocm/llvm/bin"
NEED = 2          # wait states from a VALU write of a VGPR to an MFMA that reads it


def _vregs(tok):
    tok = tok.strip()
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _operands(line):
    op, _, rest = line.partition(" ")
    return op, [t.strip() for t in rest.split(",")]


def violations(lines):
    """(function, valu line, mfma line, wait states) for each MFMA source written by a VALU fewer than NEED wait
    states before it; the walk stops at a function start or an unconditional branch / s_endpgm (no straight-line
    predecessor)."""
    out, func, block = [], None, []
    for raw in lines:
        if raw.endswith(">:"):
            func, block = raw, []
            continue
        ins = raw.split("//")[0].strip()
        if not ins or not re.match(r"[sv]_|buffer_|global_|ds_|flat_|scratch_", ins):
            continue
        op, args = _operands(ins)
        if op.startswith("v_mfma"):
            srcs = set().union(*(_vregs(a.split()[0]) for a in args[1:4] if a))
            ws = 0
            for prev in reversed(block):
                pop, pargs = _operands(prev)
                if pop.startswith("v_") and not pop.startswith("v_mfma") and _vregs(pargs[0]) & srcs and ws < NEED:
                    out.append((func, prev, ins, ws))
                    break
                ws += int(pargs[0], 0) + 1 if pop == "s_nop" else 1
                if ws >= NEED:
                    break
        block.append(ins)
        if len(block) > 16:
            del block[:8]
        if op in ("s_branch", "s_endpgm", "s_setpc_b64"):
            block = []
    return out


def _disassemble(tmp_path, lib):
    if not os.path.exists(lib):
        pytest.skip(f"{os.path.basename(lib)} is not built")
    tools = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")]
    if not all(shutil.which(t) for t in tools):
        pytest.skip("the ROCm LLVM tools are not installed")
    fat, co = str(tmp_path / "fat.bin"), str(tmp_path / "co.o")
    subprocess.run([tools[0], f"--dump-section=.hip_fatbin={fat}", lib, str(tmp_path / "lib.so")], check=True)
    subprocess.run([tools[1], "--unbundle", "--type=o", f"--input={fat}", f"--output={co}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950"], check=True)
    dis = subprocess.run([tools[2], "-d", "--mcpu=gfx950", co], check=True, capture_output=True, text=True).stdout
    return dis.splitlines()


def test_the_rule_is_seen_on_a_planted_sequence():
    """The walk itself: a VALU write read by the next MFMA, one instruction apart, behind an s_nop 0 (enough), and
    a write the MFMA does not read."""
    f = "0000 <k>:"
    bad = [f, "\tv_pk_fma_f16 v51, v12, s16, v39", "\ts_waitcnt lgkmcnt(0)",
           "\tv_mfma_f32_16x16x32_f16 v[10:13], v[44:47], v[48:51], v[14:17]"]
    ok = [f, "\tv_pk_fma_f16 v51, v12, s16, v39", "\ts_waitcnt lgkmcnt(0)", "\ts_nop 0",
          "\tv_mfma_f32_16x16x32_f16 v[10:13], v[44:47], v[48:51], v[14:17]"]
    other = [f, "\tv_pk_fma_f16 v52, v12, s16, v39",
             "\tv_mfma_f32_16x16x32_f16 v[10:13], v[44:47], v[48:51], v[14:17]"]
    acc = [f, "\tv_add_f32_e32 v15, v1, v2", "\tv_mfma_f32_16x16x32_f16 v[10:13], v[44:47], v[48:51], v[14:17]"]
    assert [v[3] for v in violations(bad)] == [1]
    assert violations(ok) == [] and violations(other) == []
    assert [v[3] for v in violations(acc)] == [0]


@pytest.mark.parametrize("lib", LIBS, ids=[os.path.basename(p) for p in LIBS])
def test_no_mfma_reads_a_fresh_valu_result(tmp_path, lib):
    lines = _disassemble(tmp_path, lib)
    n_mfma = sum(1 for l in lines if l.strip().startswith("v_mfma"))
    assert n_mfma > (1000 if lib.endswith("libexl3c4.so") else 0)   # the decode and prefill kernels are there
    bad = violations(lines)
    for func, prev, ins, ws in bad[:10]:
        print(func, "|", prev, "|", ins, "| wait states", ws)
    assert not bad, f"{len(bad)} MFMAs read a VGPR a VALU wrote fewer than {NEED} wait states before"
