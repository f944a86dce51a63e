"""The wait-state check of the built library's machine code (lfm2.5-vl-optimization_amd/csrc/hazard_lint.py).

The direct-to-LDS loads are inline asm, and the compiler inserts no wait states in front of an inline-asm statement.
The check must find the two gfx9 hazards on their scalar operands -- an SGPR written by a VALU instruction fewer
than 5 wait states before a vector memory instruction reads it, and M0 written by an SALU instruction right before
a direct-to-LDS load -- and, in kernels with direct-to-LDS loads, an LDS read that may still be outstanding at an
s_barrier, along every control-flow path, and the library as built must have none. The planted cases are
disassembly text in llvm-objdump's format.
"""

import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
CSRC = ROOT / "lfm2.5-vl-optimization_amd" / "csrc"
LIB = ROOT / "lfm2.5-vl-optimization_amd" / "lib" / "liblfm2q.so"
sys.path.insert(0, str(CSRC))

import hazard_lint  # noqa: E402


def dis(body, name="k"):
    """llvm-objdump-style text of one function from (mnemonic + operands) lines; addresses 4 bytes apart."""
    lines, addr = [f"0000000000001000 <{name}>:"], 0x1000
    for ins in body:
        if ins.endswith(":"):  # a label: the next instruction's address, for branches to refer to
            continue
        lines.append(f"\t{ins:<58}// {addr:012X}: 00000000")
        addr += 4
    return lines


def violations(body):
    funcs = hazard_lint.parse(dis(body))
    return [v for insts in funcs.values() for v in hazard_lint.check_function(insts)]


LOAD = "buffer_load_dword v1, s[44:47], 0 offen lds"


def test_valu_sgpr_write_right_before_the_load():
    v = violations(["s_mov_b32 m0, s4", "s_nop 0", "v_readlane_b32 s47, v178, 3", LOAD])
    assert len(v) == 1 and v[0][2] == "VALU writes SGPR" and v[0][4] == 0


def test_five_wait_states_clear_it():
    assert violations(["s_mov_b32 m0, s4", "v_readlane_b32 s47, v178, 3", "s_nop 4", LOAD]) == []
    # four are not enough
    assert len(violations(["s_mov_b32 m0, s4", "v_readlane_b32 s46, v178, 3", "s_nop 3", LOAD])) == 1


def test_other_sgprs_and_vgpr_writes_do_not_count():
    assert violations(["v_readlane_b32 s48, v178, 3", "v_add_u32_e32 v1, s44, v2", "s_mov_b32 m0, s4", "s_nop 0",
                       LOAD]) == []


def test_m0_written_by_salu_right_before_the_load():
    v = violations(["s_add_i32 m0, s15, s40", LOAD])
    assert len(v) == 1 and v[0][2] == "SALU writes M0"
    assert violations(["s_add_i32 m0, s15, s40", "s_nop 0", LOAD]) == []


def test_compare_into_an_sgpr_pair_and_readfirstlane():
    assert len(violations(["v_cmp_gt_u32_e64 s[46:47], v1, v2", "s_mov_b32 m0, s4", "s_nop 0", LOAD])) == 1
    assert len(violations(["v_readfirstlane_b32 s44, v4", "s_mov_b32 m0, s4", "s_nop 1", LOAD])) == 1


def test_hazard_through_a_branch():
    """The write sits in a block that branches to the load; the load's fall-through predecessor is clean."""
    lines = dis(["v_readlane_b32 s47, v1, 0", "s_mov_b32 m0, s4", "s_nop 0", "s_branch 3", "s_nop 7",
                 "s_mov_b32 m0, s4", "s_nop 0", LOAD])
    lines[4] += " <k+0x1c>"  # llvm-objdump prints the target after the encoding: s_branch -> the load at 0x101c
    funcs = hazard_lint.parse(lines)
    v = [x for insts in funcs.values() for x in hazard_lint.check_function(insts)]
    assert len(v) == 1 and v[0][2] == "VALU writes SGPR" and v[0][4] == 3, v
    # without the branch edge the same code is clean
    lines[4] = lines[4].replace(" <k+0x1c>", "")
    funcs = hazard_lint.parse(lines)
    assert [x for insts in funcs.values() for x in hazard_lint.check_function(insts)] == []


def barrier_violations(lines):
    funcs = hazard_lint.parse(lines)
    return [v for insts in funcs.values() for v in hazard_lint.check_barriers(insts)]


READ = "ds_read_b32 v61, v17 offset:24576"
REFILL = "buffer_load_dword v34, s[12:15], 0 offen lds"


def test_lds_read_outstanding_at_a_barrier():
    """The grouped GEMM's race: a stage's scale read issued, its wait sunk below the next barrier, after which the
    ring slot it reads is refilled by a direct-to-LDS load."""
    body = [READ, "v_mfma_i32_32x32x32_i8 v[18:33], v[34:37], v[38:41], v[18:33]", "s_waitcnt vmcnt(3)",
            "s_barrier", "s_mov_b32 m0, s35", "s_nop 4", REFILL, "s_waitcnt lgkmcnt(0)",
            "v_fmac_f32_e32 v2, v18, v61"]
    v = barrier_violations(dis(body))
    assert len(v) == 1 and v[0][1].startswith("ds_read_b32"), v
    # a full LDS wait before the barrier clears it; a partial one does not
    fixed = body[:3] + ["s_waitcnt lgkmcnt(0)"] + body[3:]
    assert barrier_violations(dis(fixed)) == []
    assert barrier_violations(dis(["s_waitcnt vmcnt(3) lgkmcnt(0)" if x == "s_waitcnt vmcnt(3)" else x
                                   for x in body])) == []
    assert len(barrier_violations(dis(body[:3] + ["s_waitcnt lgkmcnt(1)"] + body[3:]))) == 1
    # a function without direct-to-LDS loads has no asynchronous LDS writer, so the rule does not apply
    assert barrier_violations(dis([x for x in body if x != REFILL])) == []


def test_lds_read_outstanding_through_a_branch():
    """The read sits in a block that branches to the barrier; the fall-through path waits."""
    lines = dis([READ, "s_branch 3", "s_nop 0", "ds_read_b32 v62, v17", "s_waitcnt lgkmcnt(0)", "s_barrier", REFILL])
    lines[2] += " <k+0x14>"  # s_branch -> the barrier at 0x1014
    v = barrier_violations(lines)
    assert len(v) == 1 and v[0][2] == 0x1000, v
    lines[2] = lines[2].replace(" <k+0x14>", "")
    assert barrier_violations(lines) == []


@pytest.mark.skipif(not LIB.exists(), reason="liblfm2q.so is not built")
def test_built_library_is_clean():
    viol, nf, nv = hazard_lint.lint(str(LIB))
    assert nf > 100 and nv > 1000, (nf, nv)  # every object's code object was read
    assert viol == [], viol[:5]
