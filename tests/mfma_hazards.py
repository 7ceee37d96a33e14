"""Hazard scan of the product kernels' MFMA code (gfx950 assembly of gemm.hip).

The products issue their MFMAs from inline asm, which the compiler's hazard recognizer
does not look into: any register copy the compiler places next to those MFMAs gets no wait
states. This scan walks each kernel's instruction stream and reports

* an MFMA result (its destination registers) read or overwritten by a VALU instruction
  (`v_accvgpr_read/write/mov` and any other `v_` op) fewer than W wait states after the
  MFMA: W = 11 for v_mfma_f32_16x16x32_bf16 (8 passes) and 19 for
  v_mfma_f32_32x32x16_bf16 (16 passes), the XDL write -> VALU read/write requirements;
* a register written by a VALU instruction and read by an MFMA (any operand) fewer than 3
  wait states later.

The wait counts are conservative: one pass class above what the compiler itself inserts
after the same MFMAs when they come from builtins (short.hip's, at 13-16 wait states for
32 x 32 x 16). The scan is meant for kernels whose MFMAs are inline asm (gemm.hip); for
builtin MFMAs the compiler's own hazard recognizer places the waits.

Every instruction between the two counts as one wait state, `s_nop N` as N + 1. The scan
follows the control flow: a basic block starts from the union of what reaches its label by
falling through from the previous block (unless that ends in `s_branch`, `s_setpc` or
`s_endpgm`) and by every branch to it, forward or backward (loop back-edges), iterated until
no block's entry state changes. Usage:
    python mfma_hazards.py kernel.s [name-substring ...]
Exit status 1 if any hazard is found. tests/test_mfma_hazards.py runs it on a fresh
compile of gemm.hip."""
import re
import sys

MFMA_WAIT = {"v_mfma_f32_16x16x32_bf16": 11, "v_mfma_f32_32x32x16_bf16": 19}
VALU_TO_MFMA = 3
REG = re.compile(r"\b([av])(?:\[(\d+):(\d+)\]|(\d+)(?!\w))")


def regs(text):
    out = set()
    for kind, lo, hi, one in REG.findall(text):
        if one:
            out.add((kind, int(one)))
        else:
            out.update((kind, r) for r in range(int(lo), int(hi) + 1))
    return out


def operands(ins):
    parts = ins.split(None, 1)
    if len(parts) < 2:
        return []
    return [p.strip() for p in parts[1].split(",")]


def wait_states(ins):
    m = re.match(r"s_nop\s+(\d+)", ins)
    return int(m.group(1)) + 1 if m else 1


def _parse(lines):
    """Instructions and labels of a kernel: [(kind, text)] with kind "label" or "ins"."""
    out = []
    for raw in lines:
        ins = raw.split(";")[0].strip()
        if not ins:
            continue
        if ins.endswith(":") and re.match(r"^[A-Za-z_.$][\w.$]*:$", ins):
            out.append(("label", ins[:-1]))
        elif not ins.startswith("."):
            out.append(("ins", ins))
    return out


def _merge(a, b):
    """Union of two states (pending MFMA results, recent VALU writes), keeping for each
    entry the more constraining count."""
    if a is None:
        return b
    if b is None:
        return a
    pend = {}
    for regs_, left, text in a[0] + b[0]:
        key = (frozenset(regs_), text)
        pend[key] = max(pend.get(key, 0), left)
    rec = dict(a[1])
    for r, (age, text) in b[1].items():
        if r not in rec or age < rec[r][0]:
            rec[r] = (age, text)
    return ([(set(k[0]), v, k[1]) for k, v in pend.items()], rec)


def _step(state, ins, issues):
    """Advance the state over one instruction, appending the hazards it shows."""
    pending, recent = state
    op = ins.split()[0]
    ops = operands(ins)
    if op.startswith("v_mfma"):
        srcs = set().union(*(regs(o) for o in ops[1:])) if len(ops) > 1 else set()
        for r in srcs:
            if r in recent and recent[r][0] < VALU_TO_MFMA:
                issues.add(("VALU write -> MFMA read", recent[r][0], recent[r][1], ins))
        dst = regs(ops[0]) if ops else set()
        # a later MFMA accumulating into the same registers is ordered by the hardware
        pending = [p for p in pending if not (p[0] & dst)]
        pending.append((dst, MFMA_WAIT.get(op, 19), ins))
    elif op.startswith("v_"):
        touched = set().union(*(regs(o) for o in ops)) if ops else set()
        for p in pending:
            if p[0] & touched and p[1] > 0:
                issues.add(("MFMA result -> VALU", MFMA_WAIT.get(p[2].split()[0], 19) - p[1],
                            p[2], ins))
        dst = regs(ops[0]) if ops else set()
        recent = dict(recent)
        for r in dst:
            recent[r] = (0, ins)
    w = wait_states(ins)
    pending = [(p[0], p[1] - w, p[2]) for p in pending if p[1] - w > 0]
    recent = {r: (v[0] + w, v[1]) for r, v in recent.items() if v[0] + w < VALU_TO_MFMA}
    return (pending, recent)


def _canon(state):
    if state is None:
        return None
    return (sorted((tuple(sorted(p[0])), p[1], p[2]) for p in state[0]),
            sorted((r, v[0], v[1]) for r, v in state[1].items()))


def scan(lines):
    """Hazards of one kernel: [(kind, wait states, first instruction, second)]."""
    prog = _parse(lines)
    at_label = {}          # label -> entry state from branches
    issues = set()
    for _ in range(64):    # until the entry states stop changing
        changed = False
        state = ([], {})
        found = set()
        for kind, text in prog:
            if kind == "label":
                merged = _merge(state, at_label.get(text))
                state = merged if merged is not None else ([], {})
                continue
            state = _step(state, text, found)
            op = text.split()[0]
            if op.startswith("s_cbranch") or op == "s_branch":
                target = text.split()[-1]
                new = _merge(at_label.get(target), state)
                if _canon(new) != _canon(at_label.get(target)):
                    at_label[target] = new
                    changed = True
            if op in ("s_branch", "s_setpc_b64", "s_endpgm"):
                state = None  # no fallthrough into the next label
        issues = found
        if not changed:
            break
    return sorted(issues)


def kernels(path):
    """(name, lines) of every kernel function in an assembly file."""
    out, cur, name = [], None, None
    for line in open(path):
        m = re.match(r"^([A-Za-z_][\w.$]*):\s*(;.*)?$", line)
        if m and not m.group(1).startswith(".L"):
            name, cur = m.group(1), []
            out.append((name, cur))
            continue
        if cur is not None:
            cur.append(line)
            if line.strip().startswith("s_endpgm"):
                cur = None
    return out


def main(argv):
    path, wanted = argv[1], argv[2:]
    bad = 0
    for name, lines in kernels(path):
        if wanted and not any(w in name for w in wanted):
            continue
        if not any("v_mfma" in l for l in lines):
            continue
        issues = scan(lines)
        print(f"{name}: {len(issues)} hazard(s)")
        for kind, ws, a, b in issues[:8]:
            print(f"  {kind} after {ws} wait states: {a.strip()} / {b.strip()}")
        bad += len(issues)
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
