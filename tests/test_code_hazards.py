"""The built gfx950 code object against the wait states an MFMA needs around VALU writes of its sources (no GPU).

Two rules, in wait states (each instruction one, s_nop N counting N + 1), both of which the compiler's hazard
recognizer enforces for the instructions it emits itself and for no inline-asm block's outputs:
  RAW: a VALU write of a VGPR, then an MFMA that reads it as A, B or C: two wait states between them.
  WAR: an MFMA that reads a VGPR as C (accumulating into other registers), then a VALU write of that VGPR: three
       wait states between them (v_mfma_f32_16x16x32_f16 on gfx950; the compiler's own writes keep this spacing).
A kernel whose asm writes break either can feed an MFMA a stale or a clobbered register, and whether it does depends
on how the waves interleave. The decode keeps every asm write on a register the compiler itself defined just before
(its own VALU write kept the spacing) and out of MFMA operands; this test holds both libraries to the two rules: it
unbundles each one's gfx950 code object, disassembles it, and walks from every MFMA within its straight-line code.
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
NEED_WAR = 3      # wait states from an MFMA that reads a VGPR as C (not its destination) to a VALU write of it


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


def _instructions(lines):
    """(function, instruction) in order; None marks a point with no straight-line predecessor (a function start,
    after an unconditional branch or s_endpgm)."""
    func = None
    for raw in lines:
        if raw.endswith(">:"):
            func = raw
            yield func, None
            continue
        ins = raw.split("//")[0].strip()
        if ins and re.match(r"[sv]_|buffer_|global_|ds_|flat_|scratch_", ins):
            yield func, ins
            if ins.split()[0] in ("s_branch", "s_endpgm", "s_setpc_b64"):
                yield func, None


def _wait_states(ins):
    op, args = _operands(ins)
    return int(args[0], 0) + 1 if op == "s_nop" else 1


def _valu_dst(ins):
    op, args = _operands(ins)
    return _vregs(args[0]) if op.startswith("v_") and not op.startswith("v_mfma") else set()


def violations(lines):
    """RAW: (function, valu line, mfma line, wait states) for each MFMA source written by a VALU fewer than NEED
    wait states before it."""
    out, block = [], []
    for func, ins in _instructions(lines):
        if ins is None:
            block = []
            continue
        op, args = _operands(ins)
        if op.startswith("v_mfma"):
            srcs = set().union(*(_vregs(a.split()[0]) for a in args[1:4] if a))
            ws = 0
            for prev in reversed(block):
                if _valu_dst(prev) & srcs:
                    out.append((func, prev, ins, ws))
                    break
                ws += _wait_states(prev)
                if ws >= NEED:
                    break
        block.append(ins)
        if len(block) > 16:
            del block[:8]
    return out


def war_violations(lines):
    """WAR: (function, mfma line, valu line, wait states) for each VALU write of a VGPR that an MFMA read as C into
    other registers, fewer than NEED_WAR wait states after the MFMA."""
    out, open_reads = [], []            # [mfma line, its C registers, wait states since]
    for func, ins in _instructions(lines):
        if ins is None:
            open_reads = []
            continue
        op, args = _operands(ins)
        d = _valu_dst(ins)
        for m in open_reads:
            if d & m[1]:
                out.append((func, m[0], ins, m[2]))
        if op.startswith("v_mfma"):
            for m in open_reads:
                m[2] += 1
            c, dst = _vregs(args[3].split()[0]), _vregs(args[0])
            if c != dst:
                open_reads.append([ins, c - dst, 0])
        else:
            for m in open_reads:
                m[2] += _wait_states(ins)
        open_reads = [m for m in open_reads if m[2] < NEED_WAR]
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


def test_the_rules_are_seen_on_planted_sequences():
    """The walks themselves: a VALU write read by the next MFMA, one wait state apart (too few) and behind an s_nop 0
    (enough), a write the MFMA does not read, an accumulator input written right before; a write of an MFMA's C
    right after it (too soon), three instructions after (enough), and a write of an in-place accumulator's
    registers (the MFMA's own destination: not this rule)."""
    f = "0000 <k>:"
    mf = "\tv_mfma_f32_16x16x32_f16 v[10:13], v[44:47], v[48:51], v[14:17]"
    bad = [f, "\tv_pk_fma_f16 v51, v12, s16, v39", "\ts_waitcnt lgkmcnt(0)", mf]
    ok = [f, "\tv_pk_fma_f16 v51, v12, s16, v39", "\ts_waitcnt lgkmcnt(0)", "\ts_nop 0", mf]
    other = [f, "\tv_pk_fma_f16 v52, v12, s16, v39", mf]
    acc = [f, "\tv_add_f32_e32 v15, v1, v2", mf]
    assert [v[3] for v in violations(bad)] == [1]
    assert violations(ok) == [] and violations(other) == []
    assert [v[3] for v in violations(acc)] == [0]
    war = [f, mf, "\tv_alignbit_b32 v20, v1, v2, 4", "\tv_mad_u32_u16 v16, v4, s13, v16 op_sel:[1,0,0,0]"]
    war_ok = [f, mf, "\tv_alignbit_b32 v20, v1, v2, 4", "\ts_nop 1", "\tv_pk_mul_lo_u16 v16, v4, s12 op_sel:[1,0]"]
    in_place = [f, "\tv_mfma_f32_16x16x32_f16 v[14:17], v[44:47], v[48:51], v[14:17]", "\tv_mov_b32_e32 v20, 0"]
    assert [v[3] for v in war_violations(war)] == [1]
    assert war_violations(war_ok) == [] and war_violations(in_place) == []
    assert war_violations([f, mf, "\ts_branch 0", "\tv_mov_b32_e32 v14, 0"]) == []


@pytest.mark.parametrize("lib", LIBS, ids=[os.path.basename(p) for p in LIBS])
def test_no_mfma_operand_races_a_valu_write(tmp_path, lib):
    lines = _disassemble(tmp_path, lib)
    n_mfma = sum(1 for l in lines if l.strip().startswith("v_mfma"))
    assert n_mfma > (1000 if lib.endswith("libexl3c4.so") else 0)   # the decode and prefill kernels are there
    raw, war = violations(lines), war_violations(lines)
    for v in (raw[:5] + war[:5]):
        print(" | ".join(map(str, v)))
    assert not raw, f"{len(raw)} MFMAs read a VGPR a VALU wrote fewer than {NEED} wait states before"
    assert not war, f"{len(war)} VALU writes of an MFMA's source C fewer than {NEED_WAR} wait states after it"
