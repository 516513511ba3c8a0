#!/usr/bin/env python3
"""Build check: no VMEM instruction reads an SGPR that a VALU instruction wrote fewer than 5
wait states before it.

gfx9 (gfx950 included) requires 5 wait states between a VALU write of an SGPR (v_readlane_b32
reloading a spilled SGPR, v_readfirstlane_b32, v_cmp_*_e64, carry-outs) and a VMEM instruction
reading that SGPR. The compiler inserts them for the instructions it generates, but not for
the operands of inline asm: the LDS DMAs of gg_kernel.hip are inline asm. This scans the
device assembly the build writes (-save-temps) and fails on any such pair, following
fall-through and branch edges (two passes for loops).

usage: check_vmem_sgpr_hazard.py DEVICE.s
"""
import re
import sys

WAIT = 5
VMEM = re.compile(r"^(buffer_|global_|flat_|scratch_)")
SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b|\b(vcc)\b")
BRANCH = re.compile(r"^s_(cbranch_\w+|branch)\s+(\S+)")
CARRY = re.compile(r"^v_(add_co|sub_co|subrev_co|addc_co|subb_co|subbrev_co|div_scale|mad_u64_u32|mad_i64_i32)")


def regs(text):
    out = set()
    for m in SREG.finditer(text):
        if m.group(4):
            out |= {"vcc_lo", "vcc_hi"}
        elif m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def valu_sgpr_dsts(ins):
    """SGPRs a VALU instruction writes (empty for VGPR-only results)."""
    op, _, rest = ins.partition(" ")
    if not op.startswith("v_"):
        return set()
    operands = [o.strip() for o in rest.split(",")]
    dsts = operands[:2] if CARRY.match(op) else operands[:1]
    out = set()
    for d in dsts:
        if d.startswith("s") or d.startswith("vcc"):
            out |= regs(d)
    return out


def scan(lines, entry):
    """One pass. entry: label -> recent writes at its start. Returns (hazards, branch states)."""
    hazards, at_branch, recent, kernel = [], {}, [], None
    for no, raw in enumerate(lines, 1):
        line = raw.split(";")[0].strip()
        if line.endswith(":"):
            label = line[:-1]
            if not label.startswith(".L"):
                kernel, recent = label, []
            recent = recent + entry.get(label, [])
            continue
        if not line or line.startswith("."):
            continue
        if line.startswith("s_nop"):
            n = int(line.split()[1], 0) + 1 if len(line.split()) > 1 else 1
            recent = [(d + n, r) for d, r in recent if d + n < WAIT]
            continue
        if VMEM.match(line):
            used = regs(line.partition(" ")[2])
            for d, r in recent:
                if d < WAIT and r & used:
                    hazards.append((kernel, no, line))
                    break
        b = BRANCH.match(line)
        if b:
            at_branch.setdefault(b.group(2), []).extend(recent)
        recent = [(d + 1, r) for d, r in recent if d + 1 < WAIT]
        w = valu_sgpr_dsts(line)
        if w:
            recent.append((0, w))
        if line.startswith("s_branch") or line.startswith("s_endpgm") or line.startswith("s_setpc"):
            recent = []
    return hazards, at_branch


def main(argv):
    if len(argv) != 2:
        print(__doc__)
        return 2
    lines = open(argv[1]).read().split("\n")
    _, entry = scan(lines, {})
    hazards, _ = scan(lines, entry)
    for kernel, no, line in hazards:
        print(f"{argv[1]}:{no}: VALU-written SGPR read by VMEM within {WAIT} wait states in {kernel}: {line}")
    if hazards:
        return 1
    print(f"check_vmem_sgpr_hazard: {argv[1]}: no VALU SGPR -> VMEM hazards")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
