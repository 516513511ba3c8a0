"""Build check: no VALU / VMEM read of an accumulator register too soon after the MFMA that writes it.

The kernel issues its MFMAs from inline asm, so the compiler's hazard recognizer does not see
their latency. Whenever the register allocator keeps an accumulator outside the AGPR the MFMA
writes (for example homed in VGPRs and copied with v_accvgpr_read / v_accvgpr_write around every
MFMA), the copy can read the MFMA's result one wait state after issue and get the old value: the
outputs of that accumulator block are then silently wrong. gfx950 needs up to 19 wait states
between an XDL write and a VALU or VMEM read of the result (16-pass MFMAs; fewer for shorter
ones). This scan of the gfx950 assembly (-save-temps) counts, within a basic block, the wait states
between an MFMA and a later instruction that reads one of its destination AGPRs: one per
instruction, N + 1 per s_nop N, 4 per intervening MFMA (at least its issue cycles), and fails when
there are fewer than 19. Exit status 1 with the offending lines.

Usage: check_mfma_acc_hazard.py FILE.s [...]
"""
import re
import sys

NEED = 19


def aregs(spec):
    m = re.fullmatch(r"a\[(\d+):(\d+)\]", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"a(\d+)", spec)
    return {int(m.group(1))} if m else set()


def scan(path):
    text = open(path).read()
    bad = []
    for km in re.finditer(r"\n(_Z\w+):", text):
        name = km.group(1)
        end = text.find(".Lfunc_end", km.end())
        pending = []  # [destination registers, wait states since issue, mfma text]
        for line in text[km.end():end].split("\n"):
            t = line.split(";")[0].strip()
            if re.match(r"^\.LBB\w+:", t):
                pending = []  # the scan is per basic block (branches add wait states anyway)
                continue
            if not t or t.startswith("."):
                continue
            op = t.split()[0]
            if op.startswith("v_mfma"):
                # (an MFMA reading the accumulator of an earlier one is interlocked by the hardware)
                operands = t[len(op):].split(",")
                for p in pending:
                    p[1] += 4
                pending.append([aregs(operands[0].strip()), 0, t])
                continue
            used = set()
            if op.startswith("v_") or op.startswith("buffer_") or op.startswith("global_") or op.startswith("ds_"):
                parts = t[len(op):].split(",")
                reads = parts[1:] if len(parts) > 1 and not op.startswith(("buffer_store", "global_store", "ds_write")) else parts
                for sp in re.findall(r"a\[\d+:\d+\]|a\d+\b", ",".join(reads)):
                    used |= aregs(sp)
            for regs, waits, mf in pending:
                if used & regs and waits < NEED:
                    bad.append(f"{path}: {name[:80]}: '{t}' reads a result of '{mf}' after {waits} wait states")
            step = int(t.split()[1], 0) + 1 if op == "s_nop" else 1
            for p in pending:
                p[1] += step
            pending = [p for p in pending if p[1] < NEED]
    return bad


def main():
    bad = []
    for path in sys.argv[1:]:
        bad += scan(path)
    for b in bad[:20]:
        print(b)
    if bad:
        print(f"check_mfma_acc_hazard: {len(bad)} accumulator reads too close to their MFMA")
        sys.exit(1)
    print(f"check_mfma_acc_hazard: {' '.join(sys.argv[1:])}: no early accumulator reads")


if __name__ == "__main__":
    main()
