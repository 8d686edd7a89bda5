"""Lane schedules of prod_bwd_contr5 and prod_fwd_contr5 (csrc/products.hip):
the left and right contraction on 5 high bits (n = 9, and the two halves of
n = 10 with a null top generator). Writes csrc/contr5_schedule.h; tests/
test_kernel_model.py rebuilds the header from this module and checks that it
is the committed one, that every schedule covers every block pair once and
that the CPU model of the kernels on them equals the oracle.

Backward. One problem has 32 output blocks o and 16 steps per lane: steps
0-7 compute ga pairs only and steps 8-15 gb pairs only, so the sign pattern
of a step is fixed at compile time for every lane (no per-lane mode). For lc,
ga[o] takes the partners p containing o (2^(5-|o|) pairs), gb[o] those inside
o (2^|o|); for rc the other way round. Each phase is 32 lane roles of two
4-step pieces: a full 8-pair output (F), half of a 16-pair output (H, two
lanes), a quarter of the 32-pair output (Q, four lanes), or two outputs of at
most four pairs (D, idle steps read a zero block). H and Q outputs are summed
through LDS by one of their lanes (the owner) after the last step.

Forward. 8 steps in two 4-step pieces; lane h owns output h (its
2^(5-|h|) pairs: lc (a[S], b[S | h]), rc (a[S | h], b[S]), S inside ~h):
|h| = 2 lanes walk their 8 pairs, |h| = 3, 4, 5 lanes their 4, 2, 1 pairs and
then a 4-pair chunk of output 0 (6 chunks) or of a |h| = 1 output (2 chunks
each), which the owner adds through LDS.

Which slot holds which role, the pair order inside each piece and the
blocks' LDS slot swizzle are free; the values in LAYOUT and FWD_LAYOUT were
searched (simulated annealing on the CPU) against the LDS rules measured on
MI355X (LDS_SETS, WRITE_SETS below): the block reads of every step and the
result traffic after the last one (partials, chunks, puts)."""
from __future__ import annotations

NB, FULL = 32, 31


def popc(x):
    return bin(x).count("1")


def subsets(m):
    out, S = [], 0
    for _ in range(1 << popc(m)):
        out.append(S)
        S = (S - m) & m
    return out


# ---- backward -------------------------------------------------------------------
def plist(o, phase, lc=True):
    """Partners of output o in a phase: 'A' the ga pairs, 'B' the gb pairs
    (lc: ga partners contain o, gb partners are inside o; rc: the other way)."""
    sup = (phase == "A") == lc
    return [o | S for S in subsets(FULL & ~o)] if sup else subsets(o)


def roles(phase, lc=True):
    """The 32 lane roles of a phase: ('F', o), ('H', o, k), ('Q', o, k), ('D', o1, o2)."""
    rs, singles = [], []
    for o in range(NB):
        s = len(plist(o, phase, lc))
        if s == 8:
            rs.append(("F", o))
        elif s == 16:
            rs += [("H", o, 0), ("H", o, 1)]
        elif s == 32:
            rs += [("Q", o, k) for k in range(4)]
        else:
            singles.append(o)
    singles.sort(key=lambda o: (-len(plist(o, phase, lc)), o))
    for i in range(8):
        rs.append(("D", singles[i], singles[15 - i]))
    assert len(rs) == 32
    return rs


def role_steps(role, phase, lc=True):
    """The 8 steps (o, p) or None (idle) of a role, pieces 0 and 1 = steps 0-3, 4-7."""
    if role[0] == "F":
        return [(role[1], p) for p in plist(role[1], phase, lc)]
    if role[0] in ("H", "Q"):
        o, k = role[1], role[2]
        return [(o, p) for p in plist(o, phase, lc)[8 * k:8 * k + 8]]
    l1 = [(role[1], p) for p in plist(role[1], phase, lc)]
    l2 = [(role[2], p) for p in plist(role[2], phase, lc)]
    return l1 + [None] * (4 - len(l1)) + l2 + [None] * (4 - len(l2))


def partial_slots(phase, lc=True):
    """Partial slot of each helper role (H k = 1, Q k = 1..3) and the first slot
    and count of each owner (H k = 0, Q k = 0); slots 0-7 phase A, 8-15 phase B."""
    base = 0 if phase == "A" else 8
    slots, owners, nxt = {}, {}, base
    for r in roles(phase, lc):
        if r[0] == "H" and r[2] == 0:
            owners[r] = (nxt, 1)
            slots[("H", r[1], 1)] = nxt
            nxt += 1
    for r in roles(phase, lc):
        if r[0] == "Q" and r[2] == 0:
            owners[r] = (nxt, 3)
            for k in (1, 2, 3):
                slots[("Q", r[1], k)] = nxt
                nxt += 1
    assert nxt - base == 8
    return slots, owners


class Layout:
    """Slot of each role, pair order inside pieces, LDS slot swizzle."""

    def __init__(self, slotA, slotB, ordA, ordB, swz):  # noqa: D107
        self.slotA, self.slotB, self.ordA, self.ordB, self.swz = slotA, slotB, ordA, ordB, swz

    @staticmethod
    def default():
        ident = [list(range(8)) for _ in range(32)]
        return Layout(list(range(32)), list(range(32)), ident, [list(x) for x in ident],
                      [((b >> 1) ^ (b >> 3)) & 3 for b in range(32)])


def steps_by_slot(lc=True, lay=None):
    """steps[slot][t] = (o, p) or None, t = 0..15 (0-7 ga, 8-15 gb)."""
    lay = lay or LAYOUT[lc]
    rA, rB = roles("A", lc), roles("B", lc)
    out = []
    for s in range(NB):
        a, b = lay.slotA[s], lay.slotB[s]
        na, nb = role_steps(rA[a], "A", lc), role_steps(rB[b], "B", lc)
        out.append([na[lay.ordA[a][t]] for t in range(8)] + [nb[lay.ordB[b][t]] for t in range(8)])
    return out


def outputs_by_slot(lc=True, lay=None):
    """Per slot and phase: (type, block1, block2, partial slot, count) with type
    'F' (out = y1 + y2 -> block1), 'D' (y1 -> block1, y2 -> block2), 'help'
    (y1 + y2 -> partial slot), 'own' (y1 + y2 + count partials from slot on -> block1)."""
    lay = lay or LAYOUT[lc]
    res = []
    for s in range(NB):
        row = []
        for phase, slots_ in (("A", lay.slotA), ("B", lay.slotB)):
            r = roles(phase, lc)[slots_[s]]
            ps, own = partial_slots(phase, lc)
            if r[0] == "F":
                row.append(("F", r[1], 0, 0, 0))
            elif r[0] == "D":
                row.append(("D", r[1], r[2], 0, 0))
            elif r in own:
                row.append(("own", r[1], 0, own[r][0], own[r][1]))
            else:
                row.append(("help", r[1], 0, ps[r], 0))
        res.append(tuple(row))
    return res


# ds_read_b128 on gfx950 serves a wave in four cycles of 16 lanes: each 32-lane
# half in two sets split by the parity of lane bits 2-4 ({0-3, 12-15, 20-23,
# 24-27} and {4-7, 8-11, 16-19, 28-31}); a set takes one cycle per distinct
# address on its busiest 16-byte bank group (address bits 4-7), and lanes
# reading the same address share it. Fitted to SQ_LDS_BANK_CONFLICT over 139
# address patterns on MI355X. A problem's 32 lanes are one half.
LDS_SETS = [[s for s in range(32) if popc(s & 28) % 2 == k] for k in (0, 1)]


def lds_conflicts(lc=True, lay=None):
    """Extra LDS cycles of one problem's block reads: per step, lane set (LDS_SETS)
    and operand (partner, gc), the largest number of distinct blocks on one
    16-byte bank group, minus one."""
    lay = lay or LAYOUT[lc]
    steps = steps_by_slot(lc, lay)
    total = 0
    for t in range(16):
        for lanes in LDS_SETS:
            for kind in (0, 1):
                groups = {}
                for s in lanes:
                    st = steps[s][t]
                    if st is None:
                        addr, bank = ("z",), (0, 0)
                    else:
                        o, p = st
                        blk = p if kind == 0 else o ^ p
                        addr, bank = (kind, blk), (blk & 3, lay.swz[blk])
                    groups.setdefault(bank, set()).add(addr)
                total += max(len(v) for v in groups.values()) - 1
    return total


def _set_cost(items, sets, gmask):
    """Extra cycles of one instruction: per lane set, the largest number of
    distinct addresses on one bank group (address bits 4 and up, masked), minus one."""
    tot = 0
    for lanes in sets:
        groups = {}
        for s, a in items:
            if s in lanes:
                groups.setdefault((a >> 4) & gmask, set()).add(a)
        if groups:
            tot += max(len(v) for v in groups.values()) - 1
    return tot


# ds_write_b128 serves 8 consecutive lanes per cycle over 32 banks: bank group =
# address bits 4-6 (fitted the same way, 87 patterns).
WRITE_SETS = [set(range(8 * i, 8 * i + 8)) for i in range(4)]
READ_SETS = [set(x) for x in LDS_SETS]


def lds_write_conflicts(lc=True, lay=None):
    """Extra LDS cycles of one problem's result traffic, per 16-byte chunk q (the
    same for every q): helpers' partial stores, owners' partial reads, and the
    blocks put into the staging rows (D lanes' two blocks and the others' one are
    separate instructions). Reads count 0.7 of a cycle per conflict, as measured."""
    lay = lay or LAYOUT[lc]
    outs = outputs_by_slot(lc, lay)
    tot = 0.0
    for ph in (0, 1):
        put1, put2, putf, helpers = [], [], [], []
        owner_reads = [[], [], []]
        for s, o in enumerate(outs):
            kind, b1, b2, ps, cnt = o[ph]
            if kind == "D":
                put1.append((s, 16 * ((b1 << 2) | lay.swz[b1])))
                put2.append((s, 16 * ((b2 << 2) | lay.swz[b2])))
            elif kind == "help":
                helpers.append((s, 64 * ps))
            else:
                putf.append((s, 16 * ((b1 << 2) | lay.swz[b1])))
                for k in range(cnt):
                    owner_reads[k].append((s, 64 * (ps + k)))
        tot += sum(_set_cost(x, WRITE_SETS, 7) for x in (put1, put2, putf, helpers))
        tot += 0.7 * sum(_set_cost(x, READ_SETS, 15) for x in owner_reads)
    return tot


# searched layouts (conflict units per problem and chunk q, reads (lds_conflicts) + result traffic
# (lds_write_conflicts): lc 3 + 0, rc 1 + 0.7; Layout.default(): 43 + 18.4)
LAYOUT = {
    True: Layout(
        slotA=[24, 27, 16, 30, 14, 21, 19, 4, 0, 25, 5, 15, 23, 18, 1, 20, 7, 17, 9, 10, 6, 31, 13, 26, 2, 22, 12, 29, 28, 11, 8, 3],
        slotB=[22, 26, 20, 25, 4, 23, 24, 6, 21, 5, 28, 0, 18, 29, 8, 12, 27, 11, 2, 13, 14, 15, 16, 10, 7, 31, 1, 30, 3, 19, 17, 9],
        ordA=[[1, 0, 3, 2, 6, 5, 4, 7], [2, 3, 0, 1, 5, 7, 6, 4], [3, 1, 0, 2, 5, 4, 6, 7], [0, 1, 3, 2, 4, 6, 7, 5], [1, 2, 0, 3, 6, 5, 4, 7], [0, 3, 1, 2, 6, 4, 5, 7], [1, 0, 2, 3, 7, 4, 5, 6], [1, 2, 0, 3, 6, 7, 5, 4], [0, 1, 2, 3, 7, 6, 4, 5], [1, 0, 2, 3, 5, 6, 4, 7], [2, 3, 0, 1, 7, 6, 5, 4], [3, 1, 0, 2, 4, 6, 7, 5], [1, 0, 2, 3, 4, 6, 5, 7], [3, 0, 1, 2, 7, 5, 4, 6], [0, 2, 3, 1, 7, 4, 6, 5], [3, 0, 1, 2, 5, 7, 4, 6], [0, 1, 2, 3, 7, 5, 4, 6], [0, 3, 1, 2, 4, 7, 5, 6], [0, 2, 1, 3, 6, 7, 5, 4], [3, 2, 0, 1, 6, 7, 5, 4], [1, 3, 2, 0, 5, 4, 7, 6], [1, 3, 0, 2, 6, 5, 4, 7], [2, 0, 3, 1, 6, 4, 7, 5], [0, 3, 2, 1, 7, 6, 5, 4], [0, 2, 1, 3, 5, 4, 6, 7], [2, 1, 0, 3, 6, 7, 4, 5], [2, 0, 1, 3, 5, 4, 6, 7], [2, 0, 3, 1, 5, 4, 6, 7], [0, 1, 2, 3, 7, 4, 5, 6], [2, 1, 3, 0, 5, 4, 6, 7], [2, 1, 3, 0, 4, 5, 7, 6], [2, 3, 1, 0, 6, 5, 4, 7]],
        ordB=[[2, 3, 0, 1, 5, 6, 7, 4], [0, 2, 1, 3, 7, 6, 5, 4], [0, 2, 3, 1, 7, 6, 4, 5], [3, 1, 2, 0, 5, 6, 4, 7], [2, 3, 0, 1, 5, 6, 7, 4], [0, 1, 3, 2, 7, 6, 5, 4], [3, 1, 2, 0, 6, 7, 5, 4], [2, 0, 1, 3, 4, 7, 5, 6], [0, 1, 2, 3, 5, 4, 6, 7], [0, 2, 1, 3, 6, 4, 7, 5], [0, 3, 1, 2, 7, 6, 5, 4], [3, 2, 0, 1, 6, 4, 5, 7], [3, 0, 2, 1, 5, 4, 6, 7], [3, 0, 2, 1, 6, 5, 4, 7], [1, 2, 0, 3, 7, 5, 4, 6], [0, 2, 1, 3, 4, 6, 7, 5], [1, 0, 3, 2, 5, 7, 6, 4], [3, 1, 2, 0, 4, 5, 6, 7], [1, 0, 3, 2, 5, 7, 6, 4], [2, 1, 3, 0, 4, 5, 6, 7], [3, 0, 2, 1, 5, 4, 6, 7], [0, 2, 1, 3, 7, 6, 5, 4], [3, 0, 2, 1, 6, 5, 4, 7], [1, 3, 2, 0, 5, 7, 4, 6], [3, 1, 0, 2, 5, 7, 4, 6], [2, 1, 0, 3, 7, 5, 6, 4], [2, 1, 0, 3, 6, 7, 5, 4], [3, 0, 1, 2, 7, 5, 4, 6], [3, 0, 2, 1, 6, 5, 4, 7], [1, 2, 0, 3, 6, 7, 5, 4], [0, 3, 2, 1, 6, 5, 7, 4], [0, 3, 2, 1, 4, 5, 6, 7]],
        swz=[2, 1, 3, 1, 1, 3, 2, 3, 0, 2, 1, 0, 2, 2, 1, 0, 3, 0, 0, 2, 3, 3, 2, 2, 1, 1, 0, 3, 1, 0, 3, 1]),
    False: Layout(
        slotA=[30, 5, 29, 26, 11, 21, 9, 3, 23, 2, 22, 15, 27, 8, 0, 16, 1, 31, 7, 19, 6, 10, 28, 20, 14, 25, 18, 24, 13, 12, 17, 4],
        slotB=[12, 31, 24, 2, 4, 1, 6, 8, 14, 13, 30, 19, 29, 21, 17, 26, 5, 7, 22, 28, 20, 18, 27, 16, 25, 15, 3, 9, 11, 10, 23, 0],
        ordA=[[3, 0, 1, 2, 4, 6, 7, 5], [1, 0, 3, 2, 5, 4, 7, 6], [3, 0, 1, 2, 6, 5, 7, 4], [1, 0, 3, 2, 5, 4, 7, 6], [0, 2, 1, 3, 7, 4, 6, 5], [0, 3, 2, 1, 5, 7, 4, 6], [3, 0, 1, 2, 7, 6, 4, 5], [0, 1, 3, 2, 5, 7, 6, 4], [3, 0, 2, 1, 4, 6, 7, 5], [1, 3, 2, 0, 5, 4, 6, 7], [3, 0, 2, 1, 5, 4, 6, 7], [0, 1, 2, 3, 5, 6, 7, 4], [0, 1, 3, 2, 5, 6, 7, 4], [2, 3, 1, 0, 7, 5, 4, 6], [0, 3, 2, 1, 6, 5, 4, 7], [0, 1, 3, 2, 7, 6, 5, 4], [2, 1, 3, 0, 5, 7, 4, 6], [0, 3, 2, 1, 6, 7, 4, 5], [2, 0, 3, 1, 5, 4, 7, 6], [2, 0, 1, 3, 6, 7, 4, 5], [2, 1, 0, 3, 4, 5, 6, 7], [1, 2, 3, 0, 4, 7, 6, 5], [2, 1, 3, 0, 4, 7, 5, 6], [3, 1, 0, 2, 4, 5, 7, 6], [1, 2, 3, 0, 5, 4, 6, 7], [3, 1, 2, 0, 5, 4, 6, 7], [3, 1, 0, 2, 7, 4, 5, 6], [3, 0, 2, 1, 7, 4, 5, 6], [3, 1, 0, 2, 6, 5, 4, 7], [3, 0, 2, 1, 6, 4, 7, 5], [1, 2, 3, 0, 4, 6, 5, 7], [2, 3, 1, 0, 7, 5, 4, 6]],
        ordB=[[3, 2, 1, 0, 6, 4, 7, 5], [1, 2, 3, 0, 6, 7, 4, 5], [2, 0, 1, 3, 5, 7, 4, 6], [3, 1, 2, 0, 5, 6, 4, 7], [1, 2, 3, 0, 6, 4, 5, 7], [2, 3, 1, 0, 4, 5, 7, 6], [1, 2, 3, 0, 5, 4, 6, 7], [2, 0, 1, 3, 4, 5, 7, 6], [0, 3, 1, 2, 5, 6, 4, 7], [0, 3, 1, 2, 4, 7, 5, 6], [2, 3, 0, 1, 4, 7, 6, 5], [2, 3, 0, 1, 6, 7, 4, 5], [2, 0, 1, 3, 6, 7, 5, 4], [2, 1, 3, 0, 7, 4, 5, 6], [0, 3, 1, 2, 4, 5, 6, 7], [3, 2, 0, 1, 7, 5, 6, 4], [3, 0, 2, 1, 7, 4, 6, 5], [3, 0, 2, 1, 7, 4, 6, 5], [0, 2, 1, 3, 7, 6, 5, 4], [2, 3, 1, 0, 5, 7, 4, 6], [1, 3, 0, 2, 4, 7, 5, 6], [0, 3, 2, 1, 4, 7, 5, 6], [1, 3, 2, 0, 7, 6, 5, 4], [2, 3, 0, 1, 7, 4, 5, 6], [1, 2, 0, 3, 4, 7, 6, 5], [3, 0, 2, 1, 4, 7, 6, 5], [0, 3, 2, 1, 5, 7, 4, 6], [1, 2, 0, 3, 5, 7, 4, 6], [2, 3, 0, 1, 6, 4, 7, 5], [3, 2, 1, 0, 4, 7, 6, 5], [1, 3, 2, 0, 5, 6, 7, 4], [0, 3, 1, 2, 6, 5, 4, 7]],
        swz=[1, 3, 3, 1, 2, 0, 0, 0, 0, 1, 1, 2, 1, 2, 1, 0, 3, 2, 2, 3, 2, 0, 0, 3, 3, 1, 2, 2, 3, 3, 3, 1]),
}



# prod_bwd_inner5 stages a row once for both schedules, so its lc and rc layouts
# share one block swizzle (searched jointly; per problem and chunk q, reads +
# result traffic: lc 8 + 0, rc 9 + 0)
INNER_LAYOUT = {
    True: Layout(
        slotA=[30, 26, 2, 29, 8, 7, 6, 20, 17, 22, 28, 14, 23, 24, 27, 19, 21, 15, 5, 4, 1, 31, 18, 0, 9, 10, 11, 13, 25, 16, 3, 12],
        slotB=[13, 18, 7, 25, 23, 4, 15, 14, 9, 19, 16, 1, 30, 24, 31, 21, 3, 8, 10, 2, 22, 26, 27, 11, 29, 20, 6, 28, 5, 12, 0, 17],
        ordA=[[1, 3, 0, 2, 5, 4, 7, 6], [2, 1, 3, 0, 6, 7, 4, 5], [2, 1, 0, 3, 5, 4, 7, 6], [2, 3, 1, 0, 5, 4, 6, 7], [2, 1, 3, 0, 5, 7, 4, 6], [2, 3, 1, 0, 6, 5, 7, 4], [3, 1, 2, 0, 5, 7, 4, 6], [3, 2, 1, 0, 6, 4, 5, 7], [1, 3, 2, 0, 4, 7, 6, 5], [1, 2, 0, 3, 6, 5, 4, 7], [3, 0, 2, 1, 4, 7, 5, 6], [2, 0, 3, 1, 5, 7, 4, 6], [1, 2, 0, 3, 4, 5, 6, 7], [2, 1, 3, 0, 7, 6, 4, 5], [2, 3, 1, 0, 6, 5, 7, 4], [2, 3, 0, 1, 5, 6, 4, 7], [2, 1, 0, 3, 4, 6, 7, 5], [3, 2, 1, 0, 4, 6, 7, 5], [2, 1, 0, 3, 7, 6, 4, 5], [3, 2, 1, 0, 4, 7, 6, 5], [2, 1, 3, 0, 5, 4, 7, 6], [3, 1, 2, 0, 4, 6, 7, 5], [1, 2, 3, 0, 4, 5, 7, 6], [3, 0, 1, 2, 5, 4, 6, 7], [1, 3, 2, 0, 7, 4, 5, 6], [1, 3, 0, 2, 4, 7, 5, 6], [0, 2, 1, 3, 5, 6, 4, 7], [2, 1, 0, 3, 7, 6, 5, 4], [1, 3, 0, 2, 6, 5, 4, 7], [1, 2, 0, 3, 6, 4, 5, 7], [1, 3, 2, 0, 5, 4, 7, 6], [1, 3, 2, 0, 7, 6, 4, 5]],
        ordB=[[3, 2, 0, 1, 7, 4, 6, 5], [0, 1, 2, 3, 5, 6, 4, 7], [0, 1, 2, 3, 4, 5, 6, 7], [0, 3, 2, 1, 7, 5, 4, 6], [1, 2, 0, 3, 7, 4, 6, 5], [2, 3, 1, 0, 7, 6, 5, 4], [0, 1, 2, 3, 7, 5, 4, 6], [0, 3, 1, 2, 4, 6, 7, 5], [3, 1, 2, 0, 6, 4, 5, 7], [1, 2, 3, 0, 5, 4, 7, 6], [2, 3, 1, 0, 6, 5, 4, 7], [2, 3, 0, 1, 4, 7, 6, 5], [3, 1, 2, 0, 6, 4, 5, 7], [0, 1, 2, 3, 6, 5, 7, 4], [2, 1, 3, 0, 4, 5, 6, 7], [0, 3, 2, 1, 7, 4, 6, 5], [0, 1, 2, 3, 5, 4, 7, 6], [0, 1, 2, 3, 6, 5, 7, 4], [2, 3, 1, 0, 4, 7, 6, 5], [0, 2, 1, 3, 6, 4, 7, 5], [0, 2, 3, 1, 7, 4, 6, 5], [1, 0, 3, 2, 4, 7, 5, 6], [1, 2, 0, 3, 4, 6, 5, 7], [0, 3, 1, 2, 4, 5, 7, 6], [0, 3, 1, 2, 5, 7, 6, 4], [3, 2, 1, 0, 4, 6, 7, 5], [3, 1, 2, 0, 5, 6, 7, 4], [3, 1, 0, 2, 5, 6, 7, 4], [3, 2, 1, 0, 4, 7, 6, 5], [2, 3, 1, 0, 7, 4, 6, 5], [1, 3, 2, 0, 5, 4, 7, 6], [1, 3, 2, 0, 5, 7, 6, 4]],
        swz=[2, 3, 0, 2, 1, 0, 2, 3, 0, 2, 3, 1, 2, 1, 2, 0, 3, 1, 1, 0, 3, 2, 1, 2, 1, 0, 3, 3, 2, 3, 0, 1]),
    False: Layout(
        slotA=[29, 24, 25, 28, 3, 10, 22, 30, 7, 0, 6, 21, 27, 15, 20, 19, 17, 4, 1, 14, 18, 16, 12, 26, 13, 31, 5, 2, 9, 11, 8, 23],
        slotB=[4, 10, 21, 27, 0, 31, 16, 3, 14, 2, 8, 11, 12, 20, 24, 26, 18, 7, 17, 23, 13, 5, 30, 25, 22, 9, 6, 1, 19, 15, 29, 28],
        ordA=[[0, 2, 3, 1, 6, 7, 4, 5], [1, 0, 3, 2, 5, 6, 4, 7], [3, 2, 1, 0, 7, 6, 4, 5], [0, 3, 2, 1, 5, 4, 6, 7], [1, 2, 3, 0, 6, 5, 4, 7], [2, 1, 0, 3, 5, 7, 6, 4], [2, 3, 1, 0, 4, 5, 6, 7], [2, 3, 0, 1, 4, 7, 5, 6], [1, 0, 2, 3, 7, 4, 5, 6], [0, 1, 2, 3, 7, 6, 4, 5], [3, 1, 0, 2, 6, 5, 7, 4], [2, 3, 0, 1, 7, 6, 4, 5], [1, 3, 0, 2, 5, 6, 7, 4], [1, 3, 2, 0, 6, 5, 7, 4], [3, 2, 1, 0, 5, 4, 7, 6], [0, 3, 1, 2, 4, 6, 5, 7], [1, 3, 2, 0, 7, 6, 4, 5], [2, 0, 1, 3, 6, 4, 5, 7], [1, 3, 0, 2, 5, 6, 7, 4], [0, 2, 3, 1, 4, 7, 5, 6], [3, 2, 1, 0, 7, 6, 5, 4], [1, 0, 2, 3, 5, 7, 4, 6], [3, 0, 1, 2, 7, 6, 5, 4], [2, 0, 3, 1, 6, 7, 5, 4], [1, 3, 2, 0, 6, 7, 4, 5], [2, 3, 1, 0, 6, 7, 4, 5], [2, 3, 1, 0, 4, 6, 5, 7], [2, 3, 1, 0, 4, 7, 5, 6], [1, 3, 0, 2, 4, 7, 5, 6], [1, 3, 2, 0, 7, 6, 4, 5], [0, 2, 1, 3, 7, 4, 6, 5], [1, 3, 2, 0, 4, 7, 5, 6]],
        ordB=[[3, 2, 0, 1, 5, 6, 7, 4], [0, 2, 1, 3, 4, 7, 5, 6], [1, 3, 2, 0, 4, 6, 5, 7], [1, 2, 3, 0, 6, 4, 5, 7], [0, 3, 1, 2, 4, 6, 5, 7], [0, 2, 3, 1, 5, 4, 6, 7], [2, 3, 1, 0, 4, 6, 5, 7], [2, 1, 0, 3, 4, 6, 7, 5], [3, 1, 0, 2, 6, 7, 5, 4], [2, 0, 3, 1, 4, 6, 5, 7], [2, 3, 0, 1, 6, 5, 4, 7], [3, 1, 2, 0, 6, 4, 5, 7], [3, 0, 2, 1, 6, 7, 5, 4], [3, 2, 1, 0, 7, 4, 6, 5], [2, 1, 0, 3, 4, 6, 5, 7], [0, 2, 3, 1, 5, 7, 6, 4], [3, 2, 0, 1, 6, 4, 7, 5], [3, 0, 2, 1, 7, 4, 5, 6], [1, 0, 2, 3, 5, 6, 7, 4], [1, 0, 3, 2, 4, 5, 7, 6], [3, 0, 2, 1, 7, 6, 4, 5], [2, 3, 0, 1, 6, 7, 4, 5], [2, 1, 0, 3, 7, 6, 4, 5], [2, 1, 3, 0, 5, 6, 7, 4], [2, 3, 1, 0, 6, 7, 5, 4], [1, 3, 2, 0, 6, 5, 4, 7], [1, 3, 0, 2, 5, 4, 6, 7], [2, 3, 1, 0, 6, 5, 7, 4], [3, 1, 2, 0, 7, 6, 4, 5], [2, 0, 3, 1, 6, 7, 4, 5], [2, 3, 0, 1, 7, 5, 6, 4], [2, 0, 3, 1, 5, 7, 4, 6]],
        swz=[2, 3, 0, 2, 1, 0, 2, 3, 0, 2, 3, 1, 2, 1, 2, 0, 3, 1, 1, 0, 3, 2, 1, 2, 1, 0, 3, 3, 2, 3, 0, 1]),
}
assert INNER_LAYOUT[True].swz == INNER_LAYOUT[False].swz

# ---- forward ----------------------------------------------------------------------
FT = 8


def fwd_list(o):
    return subsets(FULL & ~o)


def fwd_chunks():
    return [(0, k) for k in range(6)] + [(1 << b, k) for b in range(5) for k in range(2)]


FHELPERS = [h for h in range(NB) if popc(h) >= 3]


class FwdLayout:
    def __init__(self, perm, assign, order, swz):
        self.perm, self.assign, self.order, self.swz = perm, assign, order, swz

    @staticmethod
    def default():
        return FwdLayout(list(range(32)), dict(zip(FHELPERS, fwd_chunks())), {h: list(range(FT)) for h in range(NB)},
                         [((b >> 1) ^ (b >> 3)) & 3 for b in range(32)])


def fwd_natural_steps(h, assign):
    m = popc(h)
    own = [(h, S) for S in fwd_list(h)]
    if m <= 2:
        return own[:8]
    owner, k = assign[h]
    return own + [None] * (4 - len(own)) + [(owner, S) for S in fwd_list(owner)[8 + 4 * k:12 + 4 * k]]


def fwd_steps_by_slot(lay=None):
    lay = lay or FWD_LAYOUT
    return [[fwd_natural_steps(lay.perm[s], lay.assign)[lay.order[lay.perm[s]][t]] for t in range(FT)]
            for s in range(NB)]


def fwd_chunk_slot(owner, k):
    return k if owner == 0 else 6 + 2 * (owner.bit_length() - 1) + k


def fwd_outputs_by_slot(lay=None):
    """Per slot: (own block, 'y1' | 'y1+y2', first chunk slot added, chunk count, chunk slot written or -1)."""
    lay = lay or FWD_LAYOUT
    res = []
    for s in range(NB):
        h = lay.perm[s]
        m = popc(h)
        if m == 2:
            res.append((h, "y1+y2", 0, 0, -1))
        elif m >= 3:
            owner, k = lay.assign[h]
            res.append((h, "y1", 0, 0, fwd_chunk_slot(owner, k)))
        elif m == 1:
            res.append((h, "y1+y2", fwd_chunk_slot(h, 0), 2, -1))
        else:
            res.append((h, "y1+y2", 0, 6, -1))
    return res


def fwd_lds_conflicts(lc=True, lay=None):
    lay = lay or FWD_LAYOUT
    steps = fwd_steps_by_slot(lay)
    total = 0
    for t in range(FT):
        for lanes in LDS_SETS:
            for kind in (0, 1):
                groups = {}
                for s in lanes:
                    st = steps[s][t]
                    if st is None:
                        addr, bank = ("z",), (0, 0)
                    else:
                        o, S = st
                        ablk, bblk = (S, S | o) if lc else (S | o, S)
                        blk = ablk if kind == 0 else bblk
                        addr, bank = (kind, blk), (blk & 3, lay.swz[blk])
                    groups.setdefault(bank, set()).add(addr)
                total += max(len(v) for v in groups.values()) - 1
    return total


def fwd_chunk_swz(c):
    """Slot swizzle of chunk slot c: its float4 q sits at 4 c + (q ^ fwd_chunk_swz(c))."""
    return (c >> 1) & 3


def fwd_lds_write_conflicts(lay=None):
    """The forward's result traffic, averaged over the chunk's float4 q: helpers'
    chunk stores, owners' chunk reads (all owners run the longest count's
    iterations) and the puts of every lane's own block."""
    lay = lay or FWD_LAYOUT
    outs = fwd_outputs_by_slot(lay)

    def chunk(c, q):
        return 16 * (4 * c + (q ^ fwd_chunk_swz(c)))

    tot = float(_set_cost([(s, 16 * ((o[0] << 2) | lay.swz[o[0]])) for s, o in enumerate(outs)], WRITE_SETS, 7))
    for q in range(4):
        tot += 0.25 * _set_cost([(s, chunk(o[4], q)) for s, o in enumerate(outs) if o[4] >= 0], WRITE_SETS, 7)
        for k in range(6):
            tot += 0.25 * 0.7 * _set_cost([(s, chunk(o[2] + k, q)) for s, o in enumerate(outs) if k < o[3]],
                                          READ_SETS, 15)
    return tot


# searched layout (lc: reads 0, result traffic 1.4)
FWD_LAYOUT = FwdLayout(
    perm=[12, 27, 30, 21, 25, 4, 26, 19, 23, 24, 22, 8, 29, 13, 10, 9, 28, 11, 5, 18, 16, 3, 7, 14, 2, 1, 31, 0, 6, 20, 17, 15],
    assign={7: (1, 0), 11: (16, 1), 13: (2, 0), 14: (4, 0), 15: (16, 0), 19: (2, 1), 21: (0, 2), 22: (0, 4), 23: (4, 1), 25: (8, 0), 26: (1, 1), 27: (0, 3), 28: (0, 1), 29: (0, 5), 30: (0, 0), 31: (8, 1)},
    order={0: [1, 2, 0, 3, 5, 7, 4, 6], 1: [2, 0, 1, 3, 6, 4, 7, 5], 2: [2, 0, 1, 3, 7, 5, 6, 4], 3: [0, 3, 2, 1, 7, 6, 5, 4], 4: [2, 1, 0, 3, 4, 6, 7, 5], 5: [0, 3, 2, 1, 4, 7, 5, 6], 6: [0, 2, 3, 1, 4, 5, 7, 6], 7: [0, 1, 2, 3, 6, 5, 7, 4], 8: [2, 0, 1, 3, 7, 4, 6, 5], 9: [3, 0, 1, 2, 7, 4, 6, 5], 10: [0, 3, 1, 2, 6, 4, 7, 5], 11: [1, 2, 3, 0, 7, 6, 5, 4], 12: [3, 0, 1, 2, 6, 4, 7, 5], 13: [3, 1, 2, 0, 6, 5, 7, 4], 14: [1, 3, 2, 0, 6, 4, 5, 7], 15: [3, 1, 0, 2, 7, 6, 4, 5], 16: [2, 1, 0, 3, 5, 6, 4, 7], 17: [2, 3, 0, 1, 4, 6, 5, 7], 18: [2, 0, 3, 1, 5, 6, 4, 7], 19: [1, 2, 3, 0, 5, 4, 7, 6], 20: [2, 3, 0, 1, 4, 6, 7, 5], 21: [3, 1, 2, 0, 6, 7, 5, 4], 22: [1, 2, 3, 0, 7, 6, 4, 5], 23: [3, 0, 1, 2, 7, 6, 5, 4], 24: [2, 0, 3, 1, 7, 4, 6, 5], 25: [0, 3, 1, 2, 4, 5, 7, 6], 26: [0, 3, 1, 2, 7, 5, 6, 4], 27: [2, 0, 3, 1, 7, 6, 4, 5], 28: [0, 2, 3, 1, 7, 5, 4, 6], 29: [2, 3, 0, 1, 4, 6, 7, 5], 30: [2, 1, 3, 0, 4, 5, 6, 7], 31: [2, 1, 3, 0, 7, 6, 5, 4]},
    swz=[3, 2, 2, 2, 1, 3, 1, 1, 1, 0, 3, 0, 2, 2, 1, 3, 2, 1, 0, 3, 0, 0, 2, 1, 0, 1, 0, 2, 3, 3, 3, 0])


# ---- header -------------------------------------------------------------------------
_TYPE = {"F": 0, "D": 1, "help": 2, "own": 3}


def header_text():
    lines = ["// Generated by gen_contr5_schedule.py (lane schedules of prod_bwd_contr5, prod_bwd_inner5 and prod_fwd_contr5); do not edit.",
             "#pragma once", "", "namespace clf {", ""]
    for lays, pre in ((LAYOUT, "kContr5"), (INNER_LAYOUT, "kContr5In")):
        for lc, tag in ((True, "Lc"), (False, "Rc")):
            lay = lays[lc]
            steps = steps_by_slot(lc, lay)
            lines.append(f"// {pre}Steps{tag}[slot][t]: output block | partner block << 5 | idle << 11 (t < 8: ga, t >= 8: gb)")
            lines.append(f"__constant__ unsigned short {pre}Steps{tag}[32][16] = {{")
            for s in range(NB):
                lines.append("    {" + ", ".join(str(2048 if x is None else x[0] | (x[1] << 5)) for x in steps[s]) + "},")
            lines.append("};")
            lines.append(f"// {pre}Out{tag}[slot][phase]: type (0 F, 1 D, 2 helper, 3 owner) | block1 << 2 | block2 << 7 |")
            lines.append("// partial slot << 12 | partial count << 16")
            lines.append(f"__constant__ unsigned {pre}Out{tag}[32][2] = {{")
            for s, row in enumerate(outputs_by_slot(lc, lay)):
                enc = [_TYPE[t] | (b1 << 2) | (b2 << 7) | (ps << 12) | (cnt << 16) for t, b1, b2, ps, cnt in row]
                lines.append("    {" + ", ".join(str(v) for v in enc) + "},")
            lines.append("};")
            if lays is LAYOUT or lc:
                swz = sum(lay.swz[b] << (2 * b) for b in range(NB))
                lines.append(f"constexpr unsigned long long {pre}Swz{tag if lays is LAYOUT else ''} = 0x{swz:016x}ull;")
            lines.append("")
    steps = fwd_steps_by_slot()
    lines.append("// kContr5Fwd[slot][t]: output block | S << 5 | idle << 11 (pair (a[S], b[S | o]) for lc)")
    lines.append("__constant__ unsigned short kContr5Fwd[32][8] = {")
    for s in range(NB):
        lines.append("    {" + ", ".join(str(2048 if x is None else x[0] | (x[1] << 5)) for x in steps[s]) + "},")
    lines.append("};")
    lines.append("// kContr5FwdOut[slot]: own block | sum of both pieces << 5 | first chunk slot added << 6 |")
    lines.append("// chunk count << 10 | chunk slot written + 1 << 13")
    lines.append("__constant__ unsigned kContr5FwdOut[32] = {")
    enc = []
    for h, how, c0, cnt, cw in fwd_outputs_by_slot():
        enc.append(h | ((how == "y1+y2") << 5) | (c0 << 6) | (cnt << 10) | ((cw + 1) << 13))
    lines.append("    " + ", ".join(str(v) for v in enc) + ",")
    lines.append("};")
    swz = sum(FWD_LAYOUT.swz[b] << (2 * b) for b in range(NB))
    lines.append(f"constexpr unsigned long long kContr5FwdSwz = 0x{swz:016x}ull;")
    lines.append("")
    lines.append("}  // namespace clf")
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "contr5_schedule.h")
    with open(path, "w") as f:
        f.write(header_text())
    print("bwd conflicts lc/rc:", lds_conflicts(True), lds_conflicts(False), "+", lds_write_conflicts(True),
          lds_write_conflicts(False), "fwd:", fwd_lds_conflicts(), "+", fwd_lds_write_conflicts())
