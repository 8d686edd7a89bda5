"""The blocked-kernel algorithm (tests/kernel_model.py, a CPU restatement of
cliffordcuda_amd/csrc/products.hip) equals the oracle for every op, on metrics
that take the blocked path, forward and backward."""
import numpy as np
import pytest
import torch

from oracle import clifford_oracle as O
from tests import kernel_model as K

CASES = [
    (4, (1, 1, 1, 1)),
    (5, (1, 1, 1, 1, 1)),
    (5, (-1, -1, -1, -1, 1)),
    (6, (1, 1, 1, 1, -1, 0)),
    (6, (1, 1, 1, 1, 0, -1)),
    (7, (1, 1, 1, 1, 1, 1, -1)),
    (7, (-1, -1, -1, -1, -1, 0, 1)),
]


@pytest.mark.parametrize("n,metric", CASES)
@pytest.mark.parametrize("op", O.OPS)
def test_model_forward_backward(op, n, metric):
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive is undefined for degenerate metrics")
    g = torch.Generator().manual_seed(n)
    a = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    b = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    gc = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    a.requires_grad_()
    b.requires_grad_()
    c = O.einsum_product(op, a, b, metric)
    ga, gb = torch.autograd.grad(c, (a, b), gc)
    cm = K.forward(op, a.detach().numpy(), b.detach().numpy(), metric)
    np.testing.assert_allclose(cm, c.detach().numpy(), atol=1e-10)
    gam, gbm = K.backward(op, a.detach().numpy(), b.detach().numpy(), gc.numpy(), metric)
    np.testing.assert_allclose(gam, ga.numpy(), atol=1e-10)
    np.testing.assert_allclose(gbm, gb.numpy(), atol=1e-10)


@pytest.mark.parametrize("n,metric,T", [(6, (1, 1, 1, 1, 1, -1), 2), (7, (-1, -1, -1, -1, 1, 0, -1), 2),
                                        (7, (1, 1, 1, 1, 1, 1, 1), 4)])
@pytest.mark.parametrize("op", O.OPS)
def test_tiled_model_forward_backward(op, n, metric, T):
    """The tiled kernels' index scheme (aligned input tiles, partner tile at
    I0 ^ K0, regressive gc tile at (fullh ^ H0 ^ M0) & ~(T - 1)) with tiles
    smaller than the row, against the oracle."""
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive is undefined for degenerate metrics")
    g = torch.Generator().manual_seed(n + T)
    a, b, gc = (torch.randn(2, 1 << n, generator=g, dtype=torch.float64) for _ in range(3))
    aq, bq = a.clone().requires_grad_(), b.clone().requires_grad_()
    c_ref = O.einsum_product(op, aq, bq, list(metric))
    c_ref.backward(gc)
    np.testing.assert_allclose(K.forward_tiled(op, a.numpy(), b.numpy(), metric, T), c_ref.detach().numpy(),
                               atol=1e-9)
    ga, gb = K.backward_tiled(op, a.numpy(), b.numpy(), gc.numpy(), metric, T)
    np.testing.assert_allclose(ga, aq.grad.numpy(), atol=1e-9)
    np.testing.assert_allclose(gb, bq.grad.numpy(), atol=1e-9)


@pytest.mark.parametrize("op", list(K.OPS.values()))
def test_balanced_schedule_covers_every_valid_pair_once(op):
    """The partner families enumerate exactly the valid block pairs of each
    output (every role, n = 4 .. 10, without and with null generators in the
    high part: pairs meeting on a null generator are left out), each once; an
    output of an op with no valid pair gets exactly one (zero) pair so that it
    is written; the inner product's forward partners stand for an lc and an rc
    half each (the same pair twice only for output block 0); the lanes' ranges
    with heads/tails rebuild each output once; the kernel's lane-parallel
    schedule (scan + binary search) equals the reference schedule."""
    rng = np.random.default_rng(op)
    for n in range(4, 11):
        NB = 1 << (n - 4)
        full = NB - 1
        nuls = sorted({0, full & (NB >> 1), full & 0b101, full & 0b110})
        for nul in nuls:
            for role in range(3):
                cls = K.bal_class(op, role)
                seen = []
                for o in range(NB):
                    for part in K.bal_partners(op, role, o, full, cls, nul):
                        if cls == 3:
                            seen += [(part, part | o), (part | o, part)] if o else [(part, part)]
                        else:
                            seen.append(K.bal_block_pair(role, o, part))
                valid = {(ih, jh) for ih in range(NB) for jh in range(NB)
                         if K.hi_sign(op, ih, jh, 0, nul, full, 0, 0)[0]}
                assert len(seen) == len(set(seen)), (n, nul, role)
                extra = set(seen) - valid
                assert valid <= set(seen), (n, nul, role)
                out_of = [[ih ^ jh, ih, jh][role] for ih, jh in extra]
                # one placeholder per output whose pairs all vanish, none elsewhere
                empty = {o for o in range(NB) if not any([ih ^ jh, ih, jh][role] == o for ih, jh in valid)}
                assert sorted(out_of) == sorted(empty), (n, nul, role)
                assert nul or not extra
                vals = {(o, part): rng.standard_normal(16) for o in range(NB)
                        for part in K.bal_partners(op, role, o, full, cls, nul)}
                out = K.bal_run(op, role, NB, lambda o, part: vals[(o, part)], cls, nul)
                for o in range(NB):
                    parts = K.bal_partners(op, role, o, full, cls, nul)
                    assert (o in out) == bool(parts)
                    if parts:
                        np.testing.assert_allclose(out[o], sum(vals[(o, part)] for part in parts), atol=1e-12)
                T, lanes, pre = K.bal_schedule(op, role, NB, cls, nul)
                assert T * NB >= pre[-1] > (T - 1) * NB or pre[-1] == 0
                # the kernel's lane-parallel computation gives the same schedule
                T2, lanes2 = K.bal_schedule_lanes(op, role, NB, cls, nul)
                assert T2 == T and len(lanes2) == len(lanes)
                for l1, l2 in zip(lanes, lanes2):
                    assert (l1 is None) == (l2 is None)
                    if l1 is not None:
                        assert {k: int(v) for k, v in l1.items()} == {k: int(v) for k, v in l2.items()}


@pytest.mark.parametrize("metric", [(1,) * 5, (-1,) * 6, (1,) * 4 + (0, -1, 1), (-1,) * 4 + (1, 0, -1, 1)],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
def test_inner_fused_forward_round(metric):
    """The balanced forward of the inner product (one round: lc and rc halves of
    every pair of the class-3 family, the doubly counted il = jl terms of
    output block 0 removed once) equals the oracle's inner product, with and
    without null generators in the high part."""
    n = len(metric)
    rng = np.random.default_rng(n)
    a = rng.standard_normal((2, 1 << n))
    b = rng.standard_normal((2, 1 << n))
    ref = O.einsum_product("inner", torch.tensor(a), torch.tensor(b), list(metric)).numpy()
    np.testing.assert_allclose(K.inner_fused_forward(a, b, list(metric)), ref, atol=1e-10)


@pytest.mark.parametrize("metric", [(1,) * 5, (-1,) * 6, (1,) * 4 + (0, -1, 1), (-1,) * 4 + (1, 0, -1, 1)],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
def test_inner_union_backward_round(metric):
    """The balanced backward of the inner product (class-4 families: all
    partners of an output; low terms split by class: shared ones always,
    lc-only ones when the left block is inside the right, rc-only ones when the
    right block is inside the left) gives the oracle's gradients, with and
    without null generators in the high part."""
    n = len(metric)
    rng = np.random.default_rng(n + 1)
    a = rng.standard_normal((2, 1 << n))
    b = rng.standard_normal((2, 1 << n))
    gc = rng.standard_normal((2, 1 << n))
    at = torch.tensor(a, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    O.einsum_product("inner", at, bt, list(metric)).backward(torch.tensor(gc))
    ga, gb = K.inner_union_backward(a, b, gc, list(metric))
    np.testing.assert_allclose(ga, at.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bt.grad.numpy(), atol=1e-10)


@pytest.mark.parametrize("metric", [(1,) * 4, (-1,) * 4, (1,) * 4 + (-1,), (1,) * 6, (-1,) * 5 + (1,),
                                    (1,) * 6 + (-1,), (-1,) * 7, (1, 1, 1, 1, -1, 1, -1), (-1,) * 4 + (1, -1, 1),
                                    (1,) * 8, (1,) * 7 + (-1,), (-1,) * 4 + (1, -1, 1, -1)],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
def test_inner_frame_backward(metric):
    """The per-lane-frame backward of the inner product (4 <= n <= 7): sub
    pairs run as sup pairs on reversed partner blocks into reversed-frame
    accumulators, with the complement sign factors s_lo(~i, ~j) =
    s_lo(i, j) (-1)^{w1(i) + w2(j)} [parity terms for a negative low metric];
    at n = 7 helper lanes take the last pairs of outputs 0 and 7. Gives the
    oracle's gradients."""
    n = len(metric)
    rng = np.random.default_rng(n + 7)
    a = rng.standard_normal((2, 1 << n))
    b = rng.standard_normal((2, 1 << n))
    gc = rng.standard_normal((2, 1 << n))
    at = torch.tensor(a, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    O.einsum_product("inner", at, bt, list(metric)).backward(torch.tensor(gc))
    ga, gb = K.inner_frame_backward(a, b, gc, list(metric))
    np.testing.assert_allclose(ga, at.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bt.grad.numpy(), atol=1e-10)


@pytest.mark.parametrize("metric", [(1,) * 4, (-1,) * 4, (1,) * 4 + (-1,), (-1,) * 5 + (1,), (1,) * 6 + (-1,),
                                    (-1,) * 7, (1, 1, 1, 1, -1, 1, -1), (1,) * 8, (-1,) * 4 + (1, -1, 1, -1)],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("op", ["lc", "rc"])
def test_contraction_frame_backward(op, metric):
    """The contractions' backward on the inner product's frame schedule with
    one accumulator per lane: every step runs the ga sup pattern, gb steps
    through s_rc(q, o) = s_lc(o, q) rho(o) rho(q) rho(o ^ q) (o inside q, rho
    the reversion sign). Gives the oracle's gradients."""
    n = len(metric)
    rng = np.random.default_rng(n + 11)
    a, b, gc = (rng.standard_normal((2, 1 << n)) for _ in range(3))
    at = torch.tensor(a, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    O.einsum_product(op, at, bt, list(metric)).backward(torch.tensor(gc))
    ga, gb = K.contraction_frame_backward(K.OPS[op], a, b, gc, list(metric))
    np.testing.assert_allclose(ga, at.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bt.grad.numpy(), atol=1e-10)


@pytest.mark.parametrize("metric", [(1,) * 4, (-1,) * 5, (1,) * 6 + (-1,), (1, 1, 1, 1, -1, 1, -1), (1,) * 8],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
def test_wedge_frame_backward(metric):
    """The wedge product's backward on the frame schedule (ga[h] over the sup
    steps, gb[~h] over the sub steps, one disjoint pattern with the
    reversion-sign factorisation for gb) gives the oracle's gradients."""
    n = len(metric)
    rng = np.random.default_rng(n + 13)
    a, b, gc = (rng.standard_normal((2, 1 << n)) for _ in range(3))
    at = torch.tensor(a, requires_grad=True)
    bt = torch.tensor(b, requires_grad=True)
    O.einsum_product("wedge", at, bt, list(metric)).backward(torch.tensor(gc))
    ga, gb = K.wedge_frame_backward(a, b, gc, list(metric))
    np.testing.assert_allclose(ga, at.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bt.grad.numpy(), atol=1e-10)


def test_reversion_sign_factorisation():
    """s_rc(q, o) = s_lc(o, q) rho(o) rho(q) rho(o ^ q) for every o inside q
    of a 4-bit low block, either low metric: the identity that lets one sign
    pattern serve both gradients of a contraction."""
    for lowneg in (False, True):
        for o in range(16):
            for q in range(16):
                if o & ~q:
                    continue
                lhs = K.low_sign(K.RC, lowneg, q, o)
                rhs = K.low_sign(K.LC, lowneg, o, q) * K._rho(o) * K._rho(q) * K._rho(o ^ q)
                assert lhs == rhs, (lowneg, o, q)
    for o in range(16):  # the wedge product's disjoint pairs
        for q in range(16):
            if o & q:
                continue
            lhs = K.low_sign(K.WEDGE, False, q, o)
            assert lhs == K.low_sign(K.WEDGE, False, o, q) * K._rho(o) * K._rho(q) * K._rho(o | q), (o, q)


def test_inner_frame_schedule_covers_every_pair():
    """Every related (output, partner) block pair of the inner product's
    backward is walked once in sub and once in sup mode when the blocks are
    equal, once otherwise, within the kernel's step count (7 at n = 7, 11 at
    n = 8)."""
    for nh in range(5):
        NB = 1 << nh
        full = NB - 1
        T = K.frame_steps_count(nh)
        seen = {}
        for h in range(NB):
            for t in range(T):
                o, p, sub = K.frame_step(nh, h, t)
                idle = (o, p) == (h, h) and not sub and t >= (1 << K.popc(h)) + (1 << (nh - K.popc(h)))
                if not idle:
                    seen[(o, p, sub)] = seen.get((o, p, sub), 0) + 1
        want = {}
        for o in range(NB):
            for p in range(NB):
                if (p & ~o) == 0:
                    want[(o, p, True)] = 1
                if (o & ~p) == 0:
                    want[(o, p, False)] = 1
        assert seen == want, nh


def test_inner_fwd7_schedule_covers_every_pair():
    """The n = 7 forward's four steps per lane (kFwd7Sched, as compiled) walk
    every (output block o, partner S inside ~o) pair of the fused round exactly
    once, and each lane's steps fit the kernel's output points: outputs 3, 5, 6
    are complete after step 1 and output 7 after step 0 (lanes 3 and 7 then
    take partners of output 0), outputs 0, 1, 2, 4 after step 3."""
    seen = {}
    last = {}
    for h in range(8):
        for t in range(4):
            st = K.fwd7_step(h, t)
            if st is None:
                continue
            o, S = st
            if o != h:
                assert h in (3, 7) and o == 0 and t >= 2
            else:
                last[o] = max(last.get(o, -1), t)
            seen[(o, S)] = seen.get((o, S), 0) + 1
    want = {(o, S): 1 for o in range(8) for S in K.subsets(7 & ~o)}
    assert seen == want
    assert last[7] == 0 and max(last[3], last[5], last[6]) <= 1


def _fwd7_unsearched(h, t):
    """The schedule before the search: own partners in subset order, lanes 3
    and 7 taking output 0's partners 4, 5 and 6, 7; idle steps read (0, o)."""
    if h == 0:
        return t
    if h == 3:
        return (3 << 3 | (0, 4)[t]) if t < 2 else t + 2
    if h == 7:
        return 7 << 3 if t == 0 else (0x80 | 7 if t == 1 else t + 4)
    parts = K.subsets(7 & ~h)
    return (h << 3 | parts[t]) if t < len(parts) else (0x80 | h)


@pytest.mark.parametrize("op", ["inner", "lc", "rc", "wedge", "regressive"])
def test_fwd7_schedule_lds_conflicts(op):
    """Under the measured b128 rules, the searched schedule and row term of
    prod_fwd_out7 have no bank conflicts in their block reads or row-order
    output stores for any of the five ops; the schedule before the search (row
    term r & 3) had 12 to 28 extra cycles per chunk and half-wave."""
    assert K.fwd7_lds_conflicts(op) == (0, 0)
    old = [[_fwd7_unsearched(h, t) for t in range(4)] for h in range(8)]
    reads, writes = K.fwd7_lds_conflicts(op, sched=old, rowx=0xE4)
    assert reads >= 12 and writes == 0


def _frame7_unsearched():
    """The n = 7 frame schedule before the search (ascending partner lists,
    idle steps reading (0, h)), as codes."""
    out = [[0] * 7 for _ in range(8)]
    for h in range(8):
        for t in range(7):
            if h == 0:
                o, p, sub = (0, 0, True) if t == 0 else (0, t - 1, False)
            elif h == 7:
                o, p, sub = (7, 7, False) if t == 0 else (7, t - 1, True)
            elif t == 6 and h in (1, 2, 5, 6):
                o, p, sub = (0, 5 + h, False) if h < 4 else (7, h + 1, True)
            else:
                cs = 1 << K.popc(h)
                subs = K.subsets(h)
                sups = [h | S for S in K.subsets(7 & ~h)]
                if t < cs:
                    o, p, sub = h, subs[t], True
                elif t < cs + len(sups):
                    o, p, sub = h, sups[t - cs], False
                else:
                    out[h][t] = 0x80 | h
                    continue
            out[h][t] = p | o << 3 | (0x40 if sub else 0)
    return out


@pytest.mark.parametrize("op", ["inner", "lc", "rc", "wedge"])
def test_frame7_schedule_lds_conflicts(op):
    """Under the measured b128 rules, the searched n = 7 frame schedule with
    its block swizzle and row term reads without bank conflicts in the inner
    product's and the contractions' backward and with 2 extra cycles per chunk
    in the wedge's (and the regressive product's); the row-order stores stay
    conflict-free. The schedule before the search had 20 to 28."""
    reads, writes = K.frame7_lds_conflicts(op)
    assert reads == (2 if op == "wedge" else 0) and writes == 0
    old_reads, _ = K.frame7_lds_conflicts(op, sched=_frame7_unsearched(), rowx=0xE4, swz=0)
    assert old_reads >= 20


def test_contr5_header_is_the_generators():
    """csrc/contr5_schedule.h is what gen_contr5_schedule.py writes."""
    import os
    sched = K.contr5_schedule_module()
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "cliffordcuda_amd", "csrc",
                        "contr5_schedule.h")
    assert open(path).read() == sched.header_text()


@pytest.mark.parametrize("lc", [True, False])
@pytest.mark.parametrize("which", ["LAYOUT", "INNER_LAYOUT"])
def test_contr5_schedule_covers_every_pair_once(lc, which):
    """Every ga pair (steps 0-7) and gb pair (steps 8-15) of a 5-high-bit
    problem appears exactly once across the 32 lanes, every output is written
    once per phase, and every helper partial is read by one owner (the
    contraction kernels' layouts and the inner kernel's)."""
    sched = K.contr5_schedule_module()
    lay = getattr(sched, which)[lc]
    steps = sched.steps_by_slot(lc, lay)
    for phase, lo in (("A", 0), ("B", 8)):
        seen = sorted(s for row in steps for s in row[lo:lo + 8] if s is not None)
        want = sorted((o, p) for o in range(32) for p in sched.plist(o, phase, lc))
        assert seen == want
    outs = sched.outputs_by_slot(lc, lay)
    for ph in range(2):
        blocks, written, read = [], set(), []
        for row in outs:
            typ, b1, b2, ps, cnt = row[ph]
            if typ == "D":
                blocks += [b1, b2]
            elif typ in ("F", "own"):
                blocks.append(b1)
            if typ == "help":
                written.add(ps)
            if typ == "own":
                read += list(range(ps, ps + cnt))
        assert sorted(blocks) == list(range(32))
        assert sorted(read) == sorted(written) and len(read) == 8


def test_contr5_fwd_schedule_covers_every_pair_once():
    sched = K.contr5_schedule_module()
    seen = sorted(s for row in sched.fwd_steps_by_slot() for s in row if s is not None)
    assert seen == sorted((o, S) for o in range(32) for S in sched.fwd_list(o))
    written = sorted(cw for h, how, c0, cnt, cw in sched.fwd_outputs_by_slot() if cw >= 0)
    read = sorted(c0 + k for h, how, c0, cnt, cw in sched.fwd_outputs_by_slot() for k in range(cnt))
    assert written == read == list(range(16))
    assert sorted(h for h, *_ in sched.fwd_outputs_by_slot()) == list(range(32))


def test_contr5_lds_conflicts_recorded():
    """The searched layouts' conflict units (per problem and chunk: block reads,
    then the result traffic) stay at their recorded values."""
    sched = K.contr5_schedule_module()
    assert sched.lds_conflicts(True) <= 3 and sched.lds_conflicts(False) <= 1
    assert sched.lds_write_conflicts(True) <= 0 and sched.lds_write_conflicts(False) <= 0.71
    assert sched.fwd_lds_conflicts() <= 0 and sched.fwd_lds_write_conflicts() <= 1.41


# SQ_LDS_BANK_CONFLICT per instruction measured on MI355X (rocprofv3 --pmc, one
# address pattern per dispatch, 8 ds_read_b128 or ds_write_b128 per iteration):
# lane l's byte offset -> (reads, writes)
_L = range(64)
_LDS_MEASURED = {
    "lane_x16": ([16 * l for l in _L], 0.0, 0.0),
    "dup4": ([16 * (l >> 2) for l in _L], 0.0, 0.0),
    "qw_same_group": ([16 * (l >> 4) + 256 * (l & 15) for l in _L], 19.88, 56.0),
    "mod4_same_group": ([16 * (l & 3) + 256 * (l >> 2) for l in _L], 8.58, 8.0),
    "stride256": ([256 * (l % 48) for l in _L], 41.16, 56.0),
    "pair_0_9": ([4096 if l == 9 else 16 * l for l in _L], 0.74, 1.0),
    "pair_0_8": ([4096 if l == 8 else 16 * l for l in _L], 0.74, 0.0),
    "first16_one_group": ([0 if l == 0 else 4096 + 256 * l if l < 16 else 16 * l for l in _L], 10.89, 14.0),
}


@pytest.mark.parametrize("name", sorted(_LDS_MEASURED))
def test_lds_rules_reproduce_measured_conflicts(name):
    """The read and write rules the layouts are searched against reproduce the
    measured conflict counts: reads at 0.7 counted cycles per extra address
    (about 0.69-0.75 measured), writes at one."""
    sched = K.contr5_schedule_module()
    addrs, reads, writes = _LDS_MEASURED[name]
    rsets = [set(h + s for s in lanes) for h in (0, 32) for lanes in sched.LDS_SETS]
    wsets = [set(range(8 * i, 8 * i + 8)) for i in range(8)]
    items = list(enumerate(addrs))
    r_units = sched._set_cost(items, rsets, 15)
    w_units = sched._set_cost(items, wsets, 7)
    assert w_units == writes
    assert abs(0.7 * r_units - reads) <= 0.1 * max(reads, 1.0) + 0.3 * (r_units > 15)


@pytest.mark.parametrize("op", [K.LC, K.RC])
@pytest.mark.parametrize("metric", [(1,) * 9, (-1,) * 4 + (1, -1, 1, 1, -1), (1,) * 4 + (-1,) * 5])
def test_contraction5_backward_n9(op, metric):
    g = torch.Generator().manual_seed(9)
    a, b, gc = (torch.randn(2, 512, generator=g, dtype=torch.float64) for _ in range(3))
    ga, gb = K.contraction5_backward(op, a.numpy(), b.numpy(), gc.numpy(), metric)
    at, bt = a.clone().requires_grad_(), b.clone().requires_grad_()
    O.einsum_product("lc" if op == K.LC else "rc", at, bt, metric).backward(gc)
    np.testing.assert_allclose(ga, at.grad.numpy(), rtol=0, atol=1e-10)
    np.testing.assert_allclose(gb, bt.grad.numpy(), rtol=0, atol=1e-10)


@pytest.mark.parametrize("op", [K.LC, K.RC])
@pytest.mark.parametrize("metric", [(1,) * 9, (-1,) * 4 + (1, -1, 1, 1, -1), (1,) * 4 + (-1,) * 5])
def test_contraction5_forward_n9(op, metric):
    g = torch.Generator().manual_seed(19)
    a, b = (torch.randn(2, 512, generator=g, dtype=torch.float64) for _ in range(2))
    c = K.contraction5_forward(op, a.numpy(), b.numpy(), metric)
    ref = O.einsum_product("lc" if op == K.LC else "rc", a, b, metric)
    np.testing.assert_allclose(c, ref.numpy(), rtol=0, atol=1e-10)


@pytest.mark.parametrize("metric", [(1,) * 9 + (0,), (1,) * 4 + (-1, 1, 1, -1, 1, 0)])
def test_contraction5_forward_null_top(metric):
    g = torch.Generator().manual_seed(20)
    a, b = (torch.randn(2, 1024, generator=g, dtype=torch.float64) for _ in range(2))
    c = K.contraction5_forward(K.LC, a.numpy(), b.numpy(), metric)
    np.testing.assert_allclose(c, O.einsum_product("lc", a, b, metric).numpy(), rtol=0, atol=1e-10)


@pytest.mark.parametrize("metric", [(1,) * 9 + (0,), (1,) * 4 + (-1, 1, 1, -1, 1, 0), (-1,) * 9 + (0,)])
def test_contraction5_backward_null_top(metric):
    g = torch.Generator().manual_seed(10)
    a, b, gc = (torch.randn(2, 1024, generator=g, dtype=torch.float64) for _ in range(3))
    ga, gb = K.contraction5_backward(K.LC, a.numpy(), b.numpy(), gc.numpy(), metric)
    at, bt = a.clone().requires_grad_(), b.clone().requires_grad_()
    O.einsum_product("lc", at, bt, metric).backward(gc)
    np.testing.assert_allclose(ga, at.grad.numpy(), rtol=0, atol=1e-10)
    np.testing.assert_allclose(gb, bt.grad.numpy(), rtol=0, atol=1e-10)


@pytest.mark.parametrize("metric", [(1,) * 9, (-1,) * 4 + (1, -1, 1, 1, -1), (1,) * 9 + (0,),
                                    (-1,) * 4 + (1, 1, -1, 1, -1, 0)])
def test_inner5_backward(metric):
    """prod_bwd_inner5's decomposition (lc and rc schedules, the element diagonal
    taken off once, the null-top routing with the grade involution) equals the
    oracle's inner-product gradients."""
    n = len(metric)
    g = torch.Generator().manual_seed(11)
    a, b, gc = (torch.randn(2, 1 << n, generator=g, dtype=torch.float64) for _ in range(3))
    ga, gb = K.inner5_backward(a.numpy(), b.numpy(), gc.numpy(), metric)
    at, bt = a.clone().requires_grad_(), b.clone().requires_grad_()
    O.einsum_product("inner", at, bt, metric).backward(gc)
    np.testing.assert_allclose(ga, at.grad.numpy(), rtol=0, atol=1e-10)
    np.testing.assert_allclose(gb, bt.grad.numpy(), rtol=0, atol=1e-10)
