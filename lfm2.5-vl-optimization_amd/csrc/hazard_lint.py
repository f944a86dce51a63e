"""Wait-state check of the gfx950 machine code in liblfm2q.so (a build step: the Makefile runs it on the library).

The kernels issue their direct-to-LDS loads (`buffer_load_dword[x4] ... lds`) as inline asm, so that the compiler
does not drain every load in flight before each LDS read or barrier. The compiler's hazard recognizer inserts the
wait states an instruction needs only for the instructions it generates itself; an inline-asm statement is opaque to
it, so two gfx9 hazards on the asm's scalar operands are left to the source:

  * a VALU instruction that writes an SGPR (v_readlane_b32 -- an SGPR spill reloaded from VGPR lanes --,
    v_readfirstlane_b32, a compare or carry-out into an SGPR pair) needs 5 wait states before a vector memory
    instruction reads that SGPR (its buffer resource or scalar offset). Closer, the load can use the SGPR's old
    value: a stale resource means a stale base address, and the load faults;
  * an SALU write of M0 needs 1 wait state before a direct-to-LDS load reads it as the LDS address.

The compiler does honour both for its own instructions (a buffer load from the builtin after v_readfirstlane gets an
`s_nop 3` in front of it on gfx950), so every violation found here is in inline asm.

A third rule covers the LDS rings those loads fill: in a kernel with direct-to-LDS loads, no LDS read may still be
outstanding at an s_barrier (an s_waitcnt lgkmcnt(0) between them on every path). After the barrier another
wavefront may refill the slot the read targets, and the asynchronous LDS write of a direct-to-LDS load is not
ordered after an LDS read issued before it. The barriers are inline asm too (a bare s_barrier, so that the loads in
flight are not drained), and the compiler moves a read's consumers, and with them its wait, across them.

This tool extracts the gfx950 code object from the library, disassembles it (llvm-objdump), builds each kernel's
control-flow graph (branch targets and fall-through edges) and, for every vector memory instruction, walks back
along every path counting wait states (one per instruction, N + 1 for s_nop N) until the hazard's window is
covered, and for every s_barrier walks back to an LDS-count wait or an LDS read. It prints each violation and exits
1 if there is any.

Usage: python3 hazard_lint.py path/to/liblfm2q.so   (or a .o / .co / a disassembly text file)
"""

import os
import re
import subprocess
import sys
import tempfile

LLVM = "/opt/rocm/llvm/bin"
VMEM_PREFIX = ("buffer_", "global_", "flat_", "scratch_")
VALU_SGPR_WAIT = 5  # VALU writes SGPR -> VMEM reads it
M0_LDS_WAIT = 1     # SALU writes M0 -> direct-to-LDS load reads it

_INST = re.compile(r"^\s+([a-z_0-9]+)(?:\s+([^/]*?))?\s*//\s*([0-9A-Fa-f]+):")
_FUNC = re.compile(r"^([0-9a-f]+) <(.+)>:$")
_TARGET = re.compile(r"<(.+)\+0x([0-9a-f]+)>\s*$")
_SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b|\b(vcc|vcc_lo|vcc_hi|m0|exec|exec_lo|exec_hi)\b")
_NAMED = {"vcc": (106, 107), "vcc_lo": (106,), "vcc_hi": (107,), "m0": ("m0",), "exec": (126, 127),
          "exec_lo": (126,), "exec_hi": (127,)}


def sregs(text):
    """Scalar registers named in an operand string (numbers, or 'm0')."""
    out = set()
    for a, b, one, named in _SREG.findall(text or ""):
        if a:
            out.update(range(int(a), int(b) + 1))
        elif one:
            out.add(int(one))
        else:
            out.update(_NAMED[named])
    return out


def split_ops(text):
    return [o.strip() for o in (text or "").split(",")] if text else []


def valu_sgpr_defs(mn, ops):
    """SGPRs a VALU instruction writes (explicit destinations and the implicit VCC of VOPC / carry e32 forms)."""
    if not mn.startswith("v_"):
        return set()
    o = split_ops(ops)
    if mn.startswith(("v_readlane_b32", "v_readfirstlane_b32")):
        return sregs(o[0]) if o else set()
    if mn.startswith(("v_cmp_", "v_cmpx_", "v_cmps_", "v_cmpsx_")):
        if mn.endswith("_e32") or (o and o[0] in ("vcc",)):
            return set(_NAMED["vcc"])
        return sregs(o[0]) if o else set()
    if re.match(r"v_(add|sub|subrev|addc|subb|subbrev)_co_u32|v_div_scale_f(32|64)|v_mad_(u64_u32|i64_i32)", mn):
        if mn.endswith("_e32"):
            return set(_NAMED["vcc"])
        return sregs(o[1]) if len(o) > 1 else set()
    return set()


def salu_defs(mn, ops):
    """Registers an SALU instruction writes (its first operand), for the M0 rule."""
    if not mn.startswith("s_") or mn.startswith(("s_nop", "s_waitcnt", "s_barrier", "s_branch", "s_cbranch",
                                                 "s_endpgm", "s_sendmsg", "s_setprio", "s_sleep", "s_trap",
                                                 "s_cmp", "s_bitcmp", "s_set_gpr", "s_setreg", "s_load",
                                                 "s_buffer_load")):
        return set()
    o = split_ops(ops)
    return sregs(o[0]) if o else set()


def wait_states(mn, ops):
    if mn == "s_nop":
        try:
            return int(ops.strip(), 0) + 1
        except ValueError:
            return 1
    return 1


def parse(dis_lines):
    """{function: [(addr, mnemonic, operands, branch_target_addr_or_None)]}"""
    funcs, cur, base = {}, None, 0
    for line in dis_lines:
        m = _FUNC.match(line.strip())
        if m:
            base, cur = int(m.group(1), 16), m.group(2)
            funcs[cur] = []
            continue
        if cur is None:
            continue
        m = _INST.match(line)
        if not m:
            continue
        mn, ops, addr = m.group(1), m.group(2) or "", int(m.group(3), 16)
        tgt = None
        if mn.startswith(("s_branch", "s_cbranch")):
            t = _TARGET.search(line)
            if t and t.group(1) == cur:
                tgt = base + int(t.group(2), 16)
        funcs[cur].append((addr, mn, ops, tgt))
    return funcs


def check_function(insts):
    """Violations in one function: (addr, vmem text, writer text, wait states between)."""
    idx = {a: i for i, (a, _, _, _) in enumerate(insts)}
    preds = [[] for _ in insts]
    for i, (a, mn, ops, tgt) in enumerate(insts):
        if tgt is not None and tgt in idx:
            preds[idx[tgt]].append(i)
        ends = mn in ("s_branch", "s_endpgm", "s_setpc_b64")
        if not ends and i + 1 < len(insts):
            preds[i + 1].append(i)
    found = []

    def walk(i, regs, window, writer_fn):
        """Earliest (fewest wait states) write of `regs` by writer_fn on any path ending just before i."""
        best = None
        stack = [(p, 0) for p in preds[i]]
        seen = {}
        while stack:
            j, ws = stack.pop()
            if ws >= window or seen.get(j, window + 1) <= ws:
                continue
            seen[j] = ws
            _, mn, ops, _ = insts[j]
            if writer_fn(mn, ops) & regs:
                if best is None or ws < best[0]:
                    best = (ws, j)
                continue
            w = wait_states(mn, ops)
            for p in preds[j]:
                stack.append((p, ws + w))
        return best

    for i, (a, mn, ops, _) in enumerate(insts):
        if not mn.startswith(VMEM_PREFIX):
            continue
        o = split_ops(ops)
        scalar = set()
        for op in o[1:]:
            scalar |= {r for r in sregs(op) if r != "m0"}
        if scalar:
            hit = walk(i, scalar, VALU_SGPR_WAIT, valu_sgpr_defs)
            if hit:
                found.append((a, f"{mn} {ops}", "VALU writes SGPR", f"{insts[hit[1]][1]} {insts[hit[1]][2]}", hit[0]))
        if re.search(r"\blds\b", ops):
            hit = walk(i, {"m0"}, M0_LDS_WAIT, salu_defs)
            if hit:
                found.append((a, f"{mn} {ops}", "SALU writes M0", f"{insts[hit[1]][1]} {insts[hit[1]][2]}", hit[0]))
    return found


def _clears_lgkm(mn, ops):
    return mn == "s_waitcnt" and (re.search(r"lgkmcnt\(0\)", ops) is not None or ops.strip() == "0")


def check_barriers(insts):
    """LDS reads that may still be outstanding at an s_barrier, in a function with direct-to-LDS loads: (barrier
    addr, read text, read addr). After the barrier another wavefront may refill the slot the read targets, and a
    direct-to-LDS write is not ordered after an LDS read issued before it; only an s_waitcnt lgkmcnt(0) between the
    read and the barrier (on every path) makes the read complete first."""
    if not any(mn.startswith(VMEM_PREFIX) and re.search(r"\blds\b", ops) for _, mn, ops, _ in insts):
        return []
    idx = {a: i for i, (a, _, _, _) in enumerate(insts)}
    preds = [[] for _ in insts]
    for i, (a, mn, ops, tgt) in enumerate(insts):
        if tgt is not None and tgt in idx:
            preds[idx[tgt]].append(i)
        if mn not in ("s_branch", "s_endpgm", "s_setpc_b64") and i + 1 < len(insts):
            preds[i + 1].append(i)
    found = []
    for i, (a, mn, _, _) in enumerate(insts):
        if mn != "s_barrier":
            continue
        stack, seen = list(preds[i]), set()
        while stack:
            j = stack.pop()
            if j in seen:
                continue
            seen.add(j)
            _, mnj, opsj, _ = insts[j]
            if _clears_lgkm(mnj, opsj):
                continue
            if mnj.startswith("ds_read"):
                found.append((a, f"{mnj} {opsj}", insts[j][0]))
                break
            stack.extend(preds[j])
    return found


def disassemble(path):
    if path.endswith((".s", ".txt", ".dis")):
        with open(path) as f:
            return f.read().splitlines()
    with tempfile.TemporaryDirectory() as td:
        cos = [path]
        if not path.endswith(".co"):
            # a linked library's .hip_fatbin holds one offload bundle per object file, back to back
            fat = os.path.join(td, "fatbin")
            subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", path,
                            os.path.join(td, "discard")], check=True)
            with open(fat, "rb") as f:
                blob = f.read()
            magic = b"__CLANG_OFFLOAD_BUNDLE__"
            starts = [m.start() for m in re.finditer(re.escape(magic), blob)]
            cos = []
            for n, s in enumerate(starts):
                part, co = os.path.join(td, f"b{n}"), os.path.join(td, f"b{n}.co")
                with open(part, "wb") as f:
                    f.write(blob[s:starts[n + 1] if n + 1 < len(starts) else len(blob)])
                subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={part}",
                                "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
                cos.append(co)
        lines = []
        for co in cos:
            lines += subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], check=True,
                                    capture_output=True, text=True).stdout.splitlines()
    return lines


def lint(path):
    """(violations, functions checked, vector memory instructions checked)"""
    funcs = parse(disassemble(path))
    viol, nvmem = [], 0
    for name, insts in funcs.items():
        nvmem += sum(1 for _, mn, _, _ in insts if mn.startswith(VMEM_PREFIX))
        for v in check_function(insts):
            viol.append((name,) + v)
        for b, rd, ra in check_barriers(insts):
            viol.append((name, b, "s_barrier", "LDS read outstanding at a barrier", f"{rd} at 0x{ra:x}", 0))
    return viol, len(funcs), nvmem


def main(argv):
    if len(argv) != 2:
        print(__doc__)
        return 2
    viol, nf, nv = lint(argv[1])
    for name, a, vm, kind, wr, ws in viol:
        print(f"hazard: {kind} {ws} wait state(s) before {vm!r} at 0x{a:x} ({wr!r}) in {name}")
    print(f"hazard_lint: {nf} functions, {nv} vector memory instructions, {len(viol)} violation(s)")
    return 1 if viol else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
