"""Build check: DPP read-after-VALU-write distance in the generated gfx950 code.

On gfx9, a DPP instruction must not read a VGPR that a VALU instruction wrote
fewer than two wait states earlier (an intervening instruction counts one,
`s_nop N` counts N + 1). The compiler's hazard recognizer does not look inside
inline asm, and the kernels issue their DPP multiply-adds as inline asm, so
this script checks the final assembly of every kernel: for each DPP
instruction it walks back along every control-flow path (fall-through and
branches into a label) until two wait states have passed, and reports any VALU
write of one of the instruction's VGPR operands in that window. Following the
compiler's own conservative rule, every VGPR operand of the DPP instruction
counts, not only the broadcast source.

Usage: python check_dpp_hazards.py file.s [...]   (exit status 1 on a finding)
"""
import re
import sys

_VREG = re.compile(r"\bv(\d+)\b|\bv\[(\d+):(\d+)\]")
_DPP_MARK = ("row_newbcast", "quad_perm", "row_mirror", "row_half_mirror", "row_shl", "row_shr",
             "row_ror", "row_bcast", "wave_shl", "wave_shr", "wave_rol", "wave_ror")
_NO_VGPR_DEF = ("v_readlane", "v_readfirstlane", "v_cmp", "v_cmpx", "v_accvgpr_write")


def vregs(text):
    out = set()
    for m in _VREG.finditer(text):
        if m.group(1) is not None:
            out.add(int(m.group(1)))
        else:
            out.update(range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def split_operands(rest):
    # operands up to the first modifier keyword (dpp controls and the like)
    return [o.strip() for o in rest.split(",")]


class Inst:
    __slots__ = ("op", "text", "defs", "uses", "dpp", "wait", "target", "uncond", "line")

    def __init__(self, op, rest, line):
        self.op = op
        self.text = rest
        self.line = line
        ops = split_operands(rest) if rest else []
        first = ops[0] if ops else ""
        self.dpp = op.endswith("_dpp") or any(k in rest for k in _DPP_MARK)
        self.defs = set()
        if op.startswith("v_") and not op.startswith(_NO_VGPR_DEF):
            self.defs = vregs(first)
        if self.dpp:
            # v_fmac/v_mac read their destination; every other operand is a use
            self.uses = vregs(rest) if ("fmac" in op or "_mac_" in op) else vregs(",".join(ops[1:]))
        else:
            self.uses = set()
        self.wait = 1
        if op == "s_nop":
            self.wait = int(first, 0) + 1
        self.target = None
        self.uncond = op in ("s_branch", "s_endpgm", "s_setpc_b64")
        if op.startswith("s_cbranch") or op == "s_branch":
            self.target = first


def parse_functions(path):
    funcs = {}
    cur = None
    for ln, raw in enumerate(open(path), 1):
        line = raw.split(";", 1)[0].rstrip()
        if not line.strip():
            continue
        s = line.strip()
        if not raw[0].isspace() and s.endswith(":") and not s.startswith("."):
            name = s[:-1]
            if cur is None or not name.startswith(".L"):
                cur = funcs.setdefault(name, [])
                continue
        if cur is None:
            continue
        if s.endswith(":"):
            cur.append(("label", s[:-1], ln))
            continue
        if s.startswith("."):
            continue
        parts = s.split(None, 1)
        cur.append(Inst(parts[0], parts[1] if len(parts) > 1 else "", ln))
    return funcs


def check_function(name, items):
    # predecessors of each label: fall-through position and branch sites
    label_pos = {}
    for i, it in enumerate(items):
        if isinstance(it, tuple):
            label_pos[it[1]] = i
    branch_sites = {}
    for i, it in enumerate(items):
        if isinstance(it, Inst) and it.target is not None:
            branch_sites.setdefault(it.target, []).append(i)

    findings = []

    def walk(i, regs, budget, seen):
        # examine items before index i (exclusive) with `budget` wait states left
        j = i - 1
        while j >= 0:
            it = items[j]
            if isinstance(it, tuple):
                for b in branch_sites.get(it[1], []):
                    key = (b, budget)
                    if key not in seen:
                        seen.add(key)
                        r = walk_from_inst(b, regs, budget, seen)
                        if r:
                            return r
                prev = j - 1
                while prev >= 0 and isinstance(items[prev], tuple):
                    prev -= 1
                if prev >= 0 and items[prev].uncond:
                    return None
                j -= 1
                continue
            return walk_from_inst(j, regs, budget, seen)
        return None

    def walk_from_inst(j, regs, budget, seen):
        it = items[j]
        if it.defs & regs:
            return it
        budget -= it.wait
        if budget <= 0:
            return None
        return walk(j, regs, budget, seen)

    for i, it in enumerate(items):
        if isinstance(it, Inst) and it.dpp and it.uses:
            hit = walk(i, it.uses, 2, set())
            if hit is not None:
                findings.append((name, it, hit))
    return findings


def main(paths):
    bad = []
    n_dpp = 0
    for p in paths:
        for name, items in parse_functions(p).items():
            n_dpp += sum(1 for it in items if isinstance(it, Inst) and it.dpp)
            bad += check_function(name, items)
    for name, it, hit in bad:
        print(f"{name}: line {it.line}: {it.op} {it.text}\n    reads a VGPR written by line "
              f"{hit.line}: {hit.op} {hit.text} (fewer than 2 wait states)")
    print(f"checked {n_dpp} DPP instructions: {len(bad)} hazard(s)")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
