"""Lane schedule of prod_bwd_contr5 (csrc/products.hip): the left and right
contraction's backward on 5 high bits (n = 9, and the two halves of n = 10
with a null top generator). Writes csrc/contr5_schedule.h; tests/
test_kernel_model.py rebuilds the header from this module and checks that it
is the committed one, that the schedule covers every block pair once and that
the CPU model of the kernel on it equals the oracle.

One problem has 32 output blocks h and 16 steps per lane. Lane h's "sub"
pairs (partner p inside h: 2^|h| of them) give one output and its "sup"
pairs (p containing h: 2^(5-|h|)) the other (for lc: gb and ga). A lane's
16 steps are three pieces, steps 0-7, 8-11 and 12-15, each summed in its
own accumulator, so every lane starts a fresh accumulator at the same steps:
  |h| = 2: sup (8) | sub (4) | helper item      |h| = 3: sub (8) | sup (4) | item
  |h| = 1: its 16 sup pairs; its 2 sub pairs are a helper item
  |h| = 4: its 16 sub pairs; its 2 sup pairs are a helper item
  h = 0:  the first 16 of its 32 sup pairs; the rest are 4 helper chunks of 4;
          its one sub pair is a helper item
  h = 31: the same with sub and sup exchanged.
The 20 lanes with |h| = 2, 3 take the 20 helper items (steps 12-15, idle
steps read a zero block). Which lane takes which item, the order of the pairs
inside each piece, which lane slot holds which h and the per-block LDS slot
swizzle are free; the values below were searched (simulated annealing, on
the CPU) to minimise LDS bank conflicts of the partner and gc block reads of
each quarter-wave (16 lanes: slots 0-15, 16-31)."""
from __future__ import annotations

NB, FULL, T = 32, 31, 16
PIECES = ((0, 8), (8, 12), (12, 16))


def popc(x):
    return bin(x).count("1")


def subsets(m):
    out, S = [], 0
    for _ in range(1 << popc(m)):
        out.append(S)
        S = (S - m) & m
    return out


def sup_list(h):
    return [h | S for S in subsets(FULL & ~h)]


def sub_list(h):
    return subsets(h)


def helper_items():
    items = [("C0", k) for k in range(4)] + [("C31", k) for k in range(4)]
    items += [("S1", 1 << b) for b in range(5)] + [("P4", FULL ^ (1 << b)) for b in range(5)]
    return items + [("S0", 0), ("P31", FULL)]


HELPERS = [h for h in range(NB) if popc(h) in (2, 3)]


def item_step(item, j):
    kind, x = item
    if kind == "C0":
        return (0, 16 + 4 * x + j, False)
    if kind == "C31":
        return (FULL, 16 + 4 * x + j, True)
    if kind == "S1":
        return (x, sub_list(x)[j], True) if j < 2 else None
    if kind == "P4":
        return (x, sup_list(x)[j], False) if j < 2 else None
    if kind == "S0":
        return (0, 0, True) if j == 0 else None
    return (FULL, FULL, False) if j == 0 else None


def natural_steps(h, assign):
    m = popc(h)
    if m == 0:
        st = [(0, p, False) for p in sup_list(0)[:16]]
    elif m == 5:
        st = [(FULL, p, True) for p in sub_list(FULL)[:16]]
    elif m == 1:
        st = [(h, p, False) for p in sup_list(h)]
    elif m == 4:
        st = [(h, p, True) for p in sub_list(h)]
    elif m == 2:
        st = [(h, p, False) for p in sup_list(h)] + [(h, p, True) for p in sub_list(h)]
    else:
        st = [(h, p, True) for p in sub_list(h)] + [(h, p, False) for p in sup_list(h)]
    if m in (2, 3):
        st += [item_step(assign[h], j) for j in range(4)]
    assert len(st) == T
    return st


# ---- searched layout (see the module docstring) ----
PERM = list(range(32))                        # lane slot -> h
ASSIGN = dict(zip(HELPERS, helper_items()))   # helper lane h -> item
ORDER = {h: list(range(16)) for h in range(NB)}   # step -> index into the lane's natural steps (within pieces)
SWZ = [((b >> 1) ^ (b >> 3)) & 3 for b in range(32)]  # LDS slot swizzle of block b


def steps_by_slot(perm=None, assign=None, order=None):
    perm, assign, order = perm or PERM, assign or ASSIGN, order or ORDER
    out = []
    for slot in range(NB):
        h = perm[slot]
        nat = natural_steps(h, assign)
        out.append([nat[order[h][t]] for t in range(T)])
    return out


def outputs_by_slot(perm=None, assign=None):
    """Per slot: U (own main output), V (second own output), W (helper item):
    each (block, sub, how) or None; how for U: 'y1' or 'sum3' (+ 'chunks' for
    h = 0 and 31), V: 'y2', W: 'y3' or ('chunk', k) (k: 0-3 output 0, 4-7
    output 31)."""
    perm, assign = perm or PERM, assign or ASSIGN
    res = []
    for slot in range(NB):
        h = perm[slot]
        m = popc(h)
        U = V = W = None
        if m == 0:
            U = (0, False, "sum3+chunks")
        elif m == 5:
            U = (FULL, True, "sum3+chunks")
        elif m == 1:
            U = (h, False, "sum3")
        elif m == 4:
            U = (h, True, "sum3")
        elif m == 2:
            U, V = (h, False, "y1"), (h, True, "y2")
        else:
            U, V = (h, True, "y1"), (h, False, "y2")
        if m in (2, 3):
            kind, x = assign[h]
            if kind == "C0":
                W = (0, False, ("chunk", x))
            elif kind == "C31":
                W = (FULL, True, ("chunk", 4 + x))
            else:
                W = {"S1": (x, True, "y3"), "P4": (x, False, "y3"), "S0": (0, True, "y3"),
                     "P31": (FULL, False, "y3")}[kind]
        res.append((U, V, W))
    return res


def lds_conflicts(steps=None, swz=None):
    """Extra LDS cycles of one problem's block reads: per step, quarter-wave
    and operand (partner, gc), the largest number of distinct blocks that
    share a bank group, minus one (ds_read_b128: 16 lanes per cycle, 16-byte
    bank groups; the same address read by several lanes costs nothing)."""
    steps, swz = steps or steps_by_slot(), swz or SWZ
    total = 0
    for t in range(T):
        for qw in range(2):
            for kind in (0, 1):
                groups = {}
                for slot in range(16 * qw, 16 * qw + 16):
                    s = steps[slot][t]
                    if s is None:
                        addr, bank = ("zero",), (0, 0)
                    else:
                        o, p, sub = s
                        blk = p if kind == 0 else o ^ p
                        rev = 3 if (kind == 0 and sub) else 0
                        region = ("a" if sub else "b") if kind == 0 else "g"
                        addr, bank = (region, blk), (blk & 3, swz[blk] ^ rev)
                    groups.setdefault(bank, set()).add(addr)
                total += max(len(v) for v in groups.values()) - 1
    return total


def header_text():
    steps = steps_by_slot()
    outs = outputs_by_slot()
    lines = ["// Generated by gen_contr5_schedule.py (lane schedule of prod_bwd_contr5); do not edit.",
             "#pragma once", "", "namespace clf {", "",
             "// kContr5Steps[slot][t]: output block | partner block << 5 | sub << 10 | idle << 11",
             "__constant__ unsigned short kContr5Steps[32][16] = {"]
    for slot in range(NB):
        row = []
        for t in range(T):
            s = steps[slot][t]
            row.append(1 << 11 if s is None else s[0] | (s[1] << 5) | (int(s[2]) << 10))
        lines.append("    {" + ", ".join(str(v) for v in row) + "},")
    lines.append("};")
    lines.append("")
    lines.append("// kContr5Out[slot][k] (k = U, V, W): block | sub << 5 | how << 6; how: 0 none, 1 y1 (U) / y2 (V) /")
    lines.append("// y3 (W), 2 y1 + y2 + y3 (U), 3 y1 + y2 + y3 + the 4 chunks of the block (U), 4 + c chunk slot c (W)")
    lines.append("__constant__ unsigned short kContr5Out[32][3] = {")
    for slot in range(NB):
        enc = []
        for k, d in enumerate(outs[slot]):
            if d is None:
                enc.append(0)
                continue
            blk, sub, how = d
            if isinstance(how, tuple):
                code = 4 + how[1]
            else:
                code = {"y1": 1, "y2": 1, "y3": 1, "sum3": 2, "sum3+chunks": 3}[how]
            enc.append(blk | (int(sub) << 5) | (code << 6))
        lines.append("    {" + ", ".join(str(v) for v in enc) + "},")
    lines.append("};")
    lines.append("")
    swz = 0
    for b in range(NB):
        swz |= SWZ[b] << (2 * b)
    lines.append(f"// LDS float4-slot swizzle of block b: (kContr5Swz >> 2b) & 3")
    lines.append(f"constexpr unsigned long long kContr5Swz = 0x{swz:016x}ull;")
    lines.append("")
    lines.append("}  // namespace clf")
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "contr5_schedule.h")
    with open(path, "w") as f:
        f.write(header_text())
    print("conflict cycles per problem-row:", lds_conflicts())


# ---- forward (prod_fwd_contr5) ------------------------------------------------
# Output block o of a problem takes the pairs (a[S], b[S | o]) for S inside ~o
# (lc; rc: (a[S | o], b[S])): 2^(5-|o|) of them. 8 steps per lane in two pieces
# (0-3, 4-7); lane h owns output h:
#   |h| = 2: its 8 pairs; |h| = 3, 4, 5: its 4, 2, 1 pairs in piece 0 and a
#   helper chunk in piece 1; |h| = 1: its first 8 pairs, two chunks of 4 by
#   helpers; h = 0: its first 8 of 32, six chunks by helpers.
FT = 8
FPIECES = ((0, 4), (4, 8))
FHELPERS = [h for h in range(NB) if popc(h) >= 3]


def fwd_chunks():
    return [(0, k) for k in range(6)] + [(1 << b, k) for b in range(5) for k in range(2)]


def fwd_list(o):
    return subsets(FULL & ~o)


FASSIGN = dict(zip(FHELPERS, fwd_chunks()))        # helper lane h -> (owner output, chunk index)
FORDER = {h: list(range(FT)) for h in range(NB)}
FPERM = list(range(32))
FSWZ = [((b >> 1) ^ (b >> 3)) & 3 for b in range(32)]


def fwd_natural_steps(h, fassign):
    m = popc(h)
    own = [(h, S) for S in fwd_list(h)]
    if m <= 2:
        st = own[:8]
    else:
        st = own + [None] * (4 - len(own))
        owner, k = fassign[h]
        st += [(owner, S) for S in fwd_list(owner)[8 + 4 * k:12 + 4 * k]]
    assert len(st) == FT
    return st


def fwd_steps_by_slot(perm=None, fassign=None, order=None):
    perm, fassign, order = perm or FPERM, fassign or FASSIGN, order or FORDER
    return [[fwd_natural_steps(perm[s], fassign)[order[perm[s]][t]] for t in range(FT)] for s in range(NB)]


def fwd_chunk_slot(owner, k):
    return k if owner == 0 else 6 + 2 * (owner.bit_length() - 1) + k


def fwd_outputs_by_slot(perm=None, fassign=None):
    """Per slot: (own block h, 'y1' | 'y1+y2' | ('y1+y2+chunks', first slot, count), chunk slot of piece 1 or None)."""
    perm, fassign = perm or FPERM, fassign or FASSIGN
    res = []
    for s in range(NB):
        h = perm[s]
        m = popc(h)
        if m == 2:
            res.append((h, "y1+y2", None))
        elif m >= 3:
            owner, k = fassign[h]
            res.append((h, "y1", fwd_chunk_slot(owner, k)))
        elif m == 1:
            res.append((h, ("y1+y2+chunks", fwd_chunk_slot(h, 0), 2), None))
        else:
            res.append((h, ("y1+y2+chunks", 0, 6), None))
    return res


def fwd_lds_conflicts(steps=None, swz=None, lc=True):
    steps, swz = steps or fwd_steps_by_slot(), swz or FSWZ
    total = 0
    for t in range(FT):
        for qw in range(2):
            for kind in (0, 1):
                groups = {}
                for slot in range(16 * qw, 16 * qw + 16):
                    s = steps[slot][t]
                    if s is None:
                        addr, bank = ("zero",), (0, 0)
                    else:
                        o, S = s
                        blk = (S if lc else S | o) if kind == 0 else (S | o if lc else S)
                        addr, bank = ("ab"[kind], blk), (blk & 3, swz[blk])
                    groups.setdefault(bank, set()).add(addr)
                total += max(len(v) for v in groups.values()) - 1
    return total
