"""Build check: no VALU / VMEM read of an accumulator register too soon after the MFMA that writes it.

The kernel issues its MFMAs from inline asm, so the compiler's hazard recognizer does not see
their latency. Whenever the register allocator keeps an accumulator outside the AGPR the MFMA
writes (for example homed in VGPRs and copied with v_accvgpr_read / v_accvgpr_write around every
MFMA), the copy can read the MFMA's result one wait state after issue and get the old value: the
outputs of that accumulator block are then silently wrong. gfx950 needs up to 19 wait states
between an XDL write and a VALU or VMEM read of the result (16-pass MFMAs; fewer for shorter
ones). This scan of the gfx950 assembly (-save-temps) counts the wait states between an MFMA and
a later instruction that reads one of its destination AGPRs: one per instruction, N + 1 per
s_nop N, 4 per intervening MFMA (at least its issue cycles). MFMAs still within 19 wait states
at the end of a basic block are carried into its fall-through successor and into the target of
every branch in it (two passes, so that loop back edges are followed too). It fails when a read
comes with fewer than 19 wait states. Exit status 1 with the offending lines.

It also fails when a basic block with at least LOOP_MFMAS MFMAs (the unrolled K loop of six
steps) holds v_readlane_b32 / v_writelane_b32: SGPR spill traffic inside the K loop.

Usage: check_mfma_acc_hazard.py FILE.s [...]
"""
import re
import sys

NEED = 19
LOOP_MFMAS = 192
BRANCH = re.compile(r"^s_(cbranch_\w+|branch)\s+(\.LBB\w+)")


def aregs(spec):
    m = re.fullmatch(r"a\[(\d+):(\d+)\]", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"a(\d+)", spec)
    return {int(m.group(1))} if m else set()


def split_blocks(lines):
    """[(label or None, [instruction text])] of one function's body, in order."""
    blocks = [(None, [])]
    for line in lines:
        t = line.split(";")[0].strip()
        m = re.match(r"^(\.LBB\w+):", t)
        if m:
            blocks.append((m.group(1), []))
        elif t and not t.startswith("."):
            blocks[-1][1].append(t)
    return blocks


def merge(a, b):
    """Pending MFMAs of two paths: the fewest wait states of each."""
    out = {p[2]: list(p) for p in a}
    for p in b:
        if p[2] not in out or p[1] < out[p[2]][1]:
            out[p[2]] = list(p)
    return list(out.values())


def run_block(instrs, pending, where, bad):
    """Scan one block from the pending MFMAs at its entry; returns (pending at its end,
    [(branch target, pending at the branch)])."""
    pending = [list(p) for p in pending]
    edges = []
    for t in instrs:
        op = t.split()[0]
        if op.startswith("v_mfma"):
            # (an MFMA reading the accumulator of an earlier one is interlocked by the hardware)
            operands = t[len(op):].split(",")
            for p in pending:
                p[1] += 4
            pending.append([aregs(operands[0].strip()), 0, t])
            continue
        used = set()
        if op.startswith(("v_", "buffer_", "global_", "ds_")):
            parts = t[len(op):].split(",")
            stores = op.startswith(("buffer_store", "global_store", "ds_write"))
            reads = parts[1:] if len(parts) > 1 and not stores else parts
            for sp in re.findall(r"a\[\d+:\d+\]|a\d+\b", ",".join(reads)):
                used |= aregs(sp)
        for regs, waits, mf in pending:
            if used & regs and waits < NEED:
                bad.add(f"{where}: '{t}' reads a result of '{mf}' after {waits} wait states")
        step = int(t.split()[1], 0) + 1 if op == "s_nop" else 1
        for p in pending:
            p[1] += step
        pending = [p for p in pending if p[1] < NEED]
        m = BRANCH.match(t)
        if m:
            edges.append((m.group(2), [list(p) for p in pending]))
            if op == "s_branch":
                pending = []  # no fall-through
    return pending, edges


def scan_function(name, lines, bad, spills):
    blocks = split_blocks(lines)
    entry = {}
    for _ in range(2):  # the second pass sees the pending MFMAs of back edges
        carry = []
        for label, instrs in blocks:
            pending = merge(carry, entry.get(label, [])) if label else carry
            carry, edges = run_block(instrs, pending, f"{name[:80]} {label or 'entry'}", bad)
            for target, p in edges:
                entry[target] = merge(entry.get(target, []), p)
    for label, instrs in blocks:
        mfmas = sum(1 for t in instrs if t.startswith("v_mfma"))
        lanes = [t for t in instrs if t.startswith(("v_readlane_b32", "v_writelane_b32"))]
        if mfmas >= LOOP_MFMAS and lanes:
            spills.append(f"{name[:80]} {label}: {len(lanes)} SGPR spill lane operations in a block of "
                          f"{mfmas} MFMAs, e.g. '{lanes[0]}'")


def scan_text(text):
    """(early accumulator reads, spill operations in K-loop blocks) of an assembly file's text."""
    bad, spills = set(), []
    for km in re.finditer(r"\n(_Z\w+):", text):
        end = text.find(".Lfunc_end", km.end())
        scan_function(km.group(1), text[km.end():end].split("\n"), bad, spills)
    return sorted(bad), spills


def main():
    bad, spills = [], []
    for path in sys.argv[1:]:
        b, s = scan_text(open(path).read())
        bad += [f"{path}: {x}" for x in b]
        spills += [f"{path}: {x}" for x in s]
    for b in (bad + spills)[:20]:
        print(b)
    if bad or spills:
        print(f"check_mfma_acc_hazard: {len(bad)} accumulator reads too close to their MFMA, "
              f"{len(spills)} K-loop blocks with SGPR spill traffic")
        sys.exit(1)
    print(f"check_mfma_acc_hazard: {' '.join(sys.argv[1:])}: no early accumulator reads, no spill "
          f"traffic in the K loop")


if __name__ == "__main__":
    main()
