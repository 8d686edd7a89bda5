"""CPU model of the blocked product kernels in cliffordcuda_amd/csrc/products.hip.

Restates, step by step, what the HIP kernels compute: the split of a blade
index into (high block, 4-bit low part), the compile-time low sign pattern
``low_sign``, the run-time high sign ``hi_sign``, the parity flip of the b
operand, the INNER block-relation variants, the regressive output permutation
and the fused backward. tests/test_kernel_model.py compares it with the oracle,
so the sign factorisation the kernels rely on is checked on the CPU before any
GPU run.
"""
import numpy as np

GEOM, WEDGE, INNER, LC, RC, REGR = range(6)
OPS = {"geom": GEOM, "wedge": WEDGE, "inner": INNER, "lc": LC, "rc": RC, "regressive": REGR}


def popc(x):
    return bin(x).count("1")


def reorder(i, j):
    return sum(popc(i >> (b + 1)) for b in range(32) if (j >> b) & 1)


def bitsum(x):
    return sum(a for a in range(32) if (x >> a) & 1)


def low_sign(var, lowneg, il, jl):
    pred = {GEOM: True, WEDGE: (il & jl) == 0,
            INNER: ((il & ~jl) & 15) == 0 or ((jl & ~il) & 15) == 0,
            LC: ((il & ~jl) & 15) == 0, RC: ((jl & ~il) & 15) == 0,
            REGR: ((il | jl) & 15) == 15}[var]
    if not pred:
        return 0
    p = reorder(il, jl)
    if var == REGR:
        p += bitsum(il) + bitsum(jl)
    elif lowneg:
        p += popc(il & jl)
    return -1 if p & 1 else 1


def hi_sign(op, ih, jh, negh, nulh, fullh, nm1, mu):
    par = reorder(ih, jh)
    if op == GEOM:
        ok = (ih & jh & nulh) == 0
        par += popc(ih & jh & negh)
    elif op == WEDGE:
        ok = (ih & jh) == 0
    elif op in (INNER, LC, RC):
        rel = {INNER: ((ih & ~jh) == 0) or ((jh & ~ih) == 0), LC: (ih & ~jh) == 0, RC: (jh & ~ih) == 0}[op]
        ok = rel and (ih & jh & nulh) == 0
        par += popc(ih & jh & negh)
    else:
        ok = (ih | jh) == fullh
        par += (popc(ih & 0xAAAAAAAA) + popc(jh & 0xAAAAAAAA) + nm1 * popc(jh) + mu)
    return ok, (-1.0 if par & 1 else 1.0)


def cross_pi(op, x, nm1):
    return (popc(x) + (nm1 if op == REGR else 0)) & 1


def variant(op, ih, jh):
    if op != INNER:
        return op
    l, r = (ih & ~jh) == 0, (jh & ~ih) == 0
    return INNER if (l and r) else (LC if l else RC)


def _tables(lowneg):
    return {v: np.array([[low_sign(v, lowneg, il, jl) for jl in range(16)] for il in range(16)], dtype=np.float64)
            for v in range(6)}


PARITY16 = np.array([popc(e) & 1 for e in range(16)])


def plan(op, metric):
    n = len(metric)
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    nul = sum(1 << k for k, m in enumerate(metric) if m == 0)
    if op in (WEDGE, REGR):
        lowneg = False
    else:
        assert (nul & 15) == 0 and (neg & 15) in (0, 15), "generic path"
        lowneg = (neg & 15) == 15
    return dict(n=n, negh=neg >> 4, nulh=nul >> 4, nm1=(n - 1) & 1, mu=popc(neg) & 1,
                fullh=(1 << (n - 4)) - 1, lowneg=lowneg)


def forward(op_name, a, b, metric):
    op = OPS[op_name]
    P = plan(op, metric)
    T = _tables(P["lowneg"])
    NB = 1 << (P["n"] - 4)
    A = a.reshape(a.shape[0], NB, 16)
    B = b.reshape(b.shape[0], NB, 16)
    out = np.zeros_like(A)
    for kh in range(NB):
        acc = np.zeros((a.shape[0], 16))
        for ih in range(NB):
            jh = ih ^ kh
            ok, s = hi_sign(op, ih, jh, P["negh"], P["nulh"], P["fullh"], P["nm1"], P["mu"])
            if not ok:
                continue
            pi = cross_pi(op, ih, P["nm1"])
            bt = B[:, jh, :] * s * np.where(PARITY16 & pi, -1.0, 1.0)
            tab = T[variant(op, ih, jh)]
            for t in range(16):
                il = np.arange(16)
                acc[:, t] += (tab[il, il ^ t] * A[:, ih, il] * bt[:, il ^ t]).sum(-1)
        if op == REGR:
            out[:, P["fullh"] ^ kh, :] = acc[:, ::-1]
        else:
            out[:, kh, :] = acc
    return out.reshape(a.shape)


def backward(op_name, a, b, gc, metric):
    op = OPS[op_name]
    P = plan(op, metric)
    T = _tables(P["lowneg"])
    NB = 1 << (P["n"] - 4)
    A = a.reshape(a.shape[0], NB, 16)
    B = b.reshape(b.shape[0], NB, 16)
    G = gc.reshape(gc.shape[0], NB, 16)
    GA = np.zeros_like(A)
    GB = np.zeros_like(A)
    il = np.arange(16)
    for h in range(NB):
        pi_h = cross_pi(op, h, P["nm1"])
        for m in range(NB):
            x = h ^ m
            g = G[:, P["fullh"] ^ x, ::-1] if op == REGR else G[:, x, :]
            oka, sa = hi_sign(op, h, m, P["negh"], P["nulh"], P["fullh"], P["nm1"], P["mu"])
            okb, sb = hi_sign(op, m, h, P["negh"], P["nulh"], P["fullh"], P["nm1"], P["mu"])
            if oka:
                bt = B[:, m, :] * sa * np.where(PARITY16 & pi_h, -1.0, 1.0)
                tab = T[variant(op, h, m)]
                for jl in range(16):
                    GA[:, h, :] += tab[il, jl] * bt[:, jl:jl + 1] * g[:, il ^ jl]
            if okb:
                pm = cross_pi(op, m, P["nm1"])
                fl = np.where(PARITY16 & pm, -1.0, 1.0)
                at = A[:, m, :] * sb * fl
                gt = g * fl
                tab = T[variant(op, m, h)]
                for jl in range(16):
                    GB[:, h, jl] += (tab[il, jl] * at[:, il] * gt[:, il ^ jl]).sum(-1)
    return GA.reshape(a.shape), GB.reshape(a.shape)


# ---- tiled kernels (prod_fwd_tiled / prod_bwd_tiled) ------------------------
# A workgroup owns the T output blocks K0 .. K0 + T - 1 and walks input tiles
# I0 = 0, T, 2T, ...; the partner blocks of a tile are the aligned tile at
# I0 ^ K0, read at local index (ih & (T-1)) ^ (kh & (T-1)). The kernels use
# T = 256; the model takes T as a parameter so small n exercise several tiles.


def forward_tiled(op_name, a, b, metric, T):
    op = OPS[op_name]
    P = plan(op, metric)
    tabs = _tables(P["lowneg"])
    NB = 1 << (P["n"] - 4)
    assert NB % T == 0
    A = a.reshape(a.shape[0], NB, 16)
    B = b.reshape(b.shape[0], NB, 16)
    out = np.zeros_like(A)
    il16 = np.arange(16)
    for K0 in range(0, NB, T):
        acc = np.zeros((a.shape[0], T, 16))
        for I0 in range(0, NB, T):
            la = A[:, I0:I0 + T, :]
            J0 = I0 ^ K0
            lb = B[:, J0:J0 + T, :]
            for lane in range(T):
                kh = K0 + lane
                for il in range(T):
                    ih = I0 + il
                    jh = ih ^ kh
                    ok, s = hi_sign(op, ih, jh, P["negh"], P["nulh"], P["fullh"], P["nm1"], P["mu"])
                    if not ok:
                        continue
                    pi = cross_pi(op, ih, P["nm1"])
                    bt = lb[:, il ^ (kh & (T - 1)), :] * s * np.where(PARITY16 & pi, -1.0, 1.0)
                    tab = tabs[variant(op, ih, jh)]
                    for t in range(16):
                        acc[:, lane, t] += (tab[il16, il16 ^ t] * la[:, il, il16] * bt[:, il16 ^ t]).sum(-1)
        for lane in range(T):
            kh = K0 + lane
            if op == REGR:
                out[:, P["fullh"] ^ kh, :] = acc[:, lane, ::-1]
            else:
                out[:, kh, :] = acc[:, lane, :]
    return out.reshape(a.shape)


def backward_tiled(op_name, a, b, gc, metric, T):
    op = OPS[op_name]
    P = plan(op, metric)
    tabs = _tables(P["lowneg"])
    NB = 1 << (P["n"] - 4)
    fullh = P["fullh"]
    A = a.reshape(a.shape[0], NB, 16)
    B = b.reshape(b.shape[0], NB, 16)
    G = gc.reshape(gc.shape[0], NB, 16)
    GA = np.zeros_like(A)
    GB = np.zeros_like(A)
    il = np.arange(16)
    for H0 in range(0, NB, T):
        for M0 in range(0, NB, T):
            G0 = ((fullh ^ H0 ^ M0) & ~(T - 1)) if op == REGR else (H0 ^ M0)
            la, lb, lg = A[:, M0:M0 + T, :], B[:, M0:M0 + T, :], G[:, G0:G0 + T, :]
            for hl in range(T):
                h = H0 + hl
                pi_h = cross_pi(op, h, P["nm1"])
                for ml in range(T):
                    m = M0 + ml
                    oka, sa = hi_sign(op, h, m, P["negh"], P["nulh"], fullh, P["nm1"], P["mu"])
                    okb, sb = hi_sign(op, m, h, P["negh"], P["nulh"], fullh, P["nm1"], P["mu"])
                    if not (oka or okb):
                        continue
                    g = lg[:, (T - 1) ^ hl ^ ml, ::-1] if op == REGR else lg[:, hl ^ ml, :]
                    if oka:
                        bt = lb[:, ml, :] * sa * np.where(PARITY16 & pi_h, -1.0, 1.0)
                        tab = tabs[variant(op, h, m)]
                        for jl in range(16):
                            GA[:, h, :] += tab[il, jl] * bt[:, jl:jl + 1] * g[:, il ^ jl]
                    if okb:
                        pm = cross_pi(op, m, P["nm1"])
                        fl = np.where(PARITY16 & pm, -1.0, 1.0)
                        at = la[:, ml, :] * sb * fl
                        gt = g * fl
                        tab = tabs[variant(op, m, h)]
                        for jl in range(16):
                            GB[:, h, jl] += (tab[il, jl] * at[:, il] * gt[:, il ^ jl]).sum(-1)
    return GA.reshape(a.shape), GB.reshape(a.shape)


# ---- balanced kernels (prod_fwd_bal / prod_bwd_bal) -------------------------
# A row's valid (output block, partner block) pairs, ordered by output block
# and, inside an output, by the kernel's subset enumeration, are dealt out to
# the NB lanes of the row in equal contiguous ranges of T = ceil(total / NB).
# ROLE 0: output kh, partner ih (jh = ih ^ kh); ROLE 1: output ih (ga),
# partner jh; ROLE 2: output jh (gb), partner ih. A lane closes a segment when
# its output's pairs end or its range ends: a segment that began in an earlier
# lane is a "head" (written to LDS), a segment that began here and ends here
# is stored, and a last segment that continues in later lanes is a "tail",
# to which its lane adds the heads of the later lanes after the loop.


def bal_family(op, role, o, full, cls=0, nul=0):
    """List of (base, mask, first, count) sub-families: partners base | S for the
    subsets S of mask in the kernel's order, from index first, one sub-family
    after the other. The inner product uses class 3 for its forward (one
    family; each partner S stands for the lc half (S, S | o) and the rc half
    (S | o, S)) and class 4 for its backward (the lc-side partners, the pair
    ih = jh included, then the rc-side partners).
    nul: high-part null generators; pairs whose blocks share one are zero for
    the metric ops and are left out. An output whose pairs are all zero keeps
    one zero pair so that it is still written."""
    co = ~o & full
    nco, no = 1 << popc(co), 1 << popc(o)
    con, onn = co & ~nul, o & ~nul   # partner bits that never meet a null
    if op == GEOM:
        m = full & ~(nul & ~o) if role == 0 else full & ~(nul & o)
        return [(0, m, 0, 1 << popc(m))]
    if op == WEDGE:
        return [(0, o, 0, no) if role == 0 else (0, co, 0, nco)]
    if op == LC:
        return [[(0, con, 0, 1 << popc(con)), (o, 0, 0, 1) if o & nul else (o, co, 0, nco),
                 (0, onn, 0, 1 << popc(onn))][role]]
    if op == RC:
        return [[(o, con, 0, 1 << popc(con)), (0, onn, 0, 1 << popc(onn)),
                 (o, 0, 0, 1) if o & nul else (o, co, 0, nco)][role]]
    if op == REGR:
        return [(co, o, 0, no)]
    strict = (1 << popc(onn)) - (1 if onn == o else 0)  # subsets of onn strictly inside o
    if role == 0:
        assert cls == 3
        return [(0, con, 0, 1 << popc(con))]
    assert cls == 4
    if role == 1:   # output ih = o: jh = o | S, then jh strictly inside o
        return [(o, co, 0, 0 if o & nul else nco), (0, onn, 0, strict)]
    return [(0, onn, 0, 1 << popc(onn)), (o, co, 1, 0 if o & nul else nco - 1)]


def bal_class(op, role):
    """The class the kernels run for an op and role."""
    return (3 if role == 0 else 4) if op == INNER else 0


def subsets(m):
    """Subsets of m in the kernel's order: S <- (S - m) & m from 0."""
    out, S = [], 0
    for _ in range(1 << popc(m)):
        out.append(S)
        S = (S - m) & m
    return out


def bal_partners(op, role, o, full, cls=0, nul=0):
    return [base | S for base, mask, first, count in bal_family(op, role, o, full, cls, nul)
            for S in subsets(mask)[first:first + count]]


def bal_block_pair(role, o, part):
    """(ih, jh) of a pair."""
    return [(part, part ^ o), (o, part), (part, o)][role]


def bal_schedule(op, role, NB, cls=0, nul=0):
    full = NB - 1
    counts = [len(bal_partners(op, role, o, full, cls, nul)) for o in range(NB)]
    pre = np.concatenate([[0], np.cumsum(counts)])
    total = int(pre[-1])
    T = -(-total // NB)
    lanes = []
    for lr in range(NB):
        p0, p1 = lr * T, min(lr * T + T, total)
        if p1 <= p0:
            lanes.append(None)
            continue
        o0 = int(np.searchsorted(pre, p0, side="right") - 1)
        ol = int(np.searchsorted(pre, p1 - 1, side="right") - 1)
        cont0 = p0 > pre[o0]
        tail = p1 < pre[ol + 1] and not (ol == o0 and cont0)
        lanes.append(dict(p0=p0, p1=p1, o0=o0, s0=int(p0 - pre[o0]), cont0=cont0, tail=tail, olast=ol,
                          last_lane=int((pre[ol + 1] - 1) // T)))
    return T, lanes, pre


def bal_schedule_lanes(op, role, NB, cls=0, nul=0):
    """The kernel's computation of the same schedule (bal_schedule in
    csrc/products.hip): lane lr counts output lr's pairs, a shuffle-up
    inclusive scan over the NB lanes, then a binary search with shuffles for
    the largest output whose exclusive offset is <= p0 (and p1 - 1)."""
    full = NB - 1
    c = [len(bal_partners(op, role, lr, full, cls, nul)) for lr in range(NB)]
    inc = list(c)
    d = 1
    while d < NB:
        inc = [inc[lr] + (inc[lr - d] if lr >= d else 0) for lr in range(NB)]
        d *= 2
    pre = [inc[lr] - c[lr] for lr in range(NB)]
    total = inc[NB - 1]
    T = -(-total // NB)

    def largest_le(v):
        lo, step = 0, NB // 2
        while step > 0:
            if pre[lo + step] <= v:
                lo += step
            step //= 2
        return lo

    lanes = []
    for lr in range(NB):
        p0, p1 = lr * T, min(lr * T + T, total)
        if p1 <= p0:
            lanes.append(None)
            continue
        o0, ol = largest_le(p0), largest_le(p1 - 1)
        s0 = p0 - pre[o0]
        last_end = inc[ol]
        tail = p1 < last_end and not (ol == o0 and s0 > 0)
        lanes.append(dict(p0=p0, p1=p1, o0=o0, s0=s0, cont0=s0 > 0, tail=tail, olast=ol,
                          last_lane=(last_end - 1) // T))
    return T, lanes


def bal_run(op, role, NB, pair_value, cls=0, nul=0):
    """Emulate the lanes of one row for one class: pair_value(o, part) ->
    contribution (16,) array (zero for pairs the metric kills). Returns out[o]
    as the kernel stores (or adds) it: complete segments, then tails + heads."""
    full = NB - 1
    T, lanes, pre = bal_schedule(op, role, NB, cls, nul)
    out = {}
    heads = {}
    tails = {}
    for lr, sc in enumerate(lanes):
        if sc is None:
            continue
        o, s, first = sc["o0"], sc["s0"], True
        partners = bal_partners(op, role, o, full, cls, nul)
        acc = np.zeros(16)
        for p in range(sc["p0"], sc["p1"]):
            acc = acc + pair_value(o, partners[s])
            s += 1
            done = s == len(partners)
            if done or p + 1 == sc["p1"]:
                if first and sc["cont0"]:
                    heads[lr] = acc
                elif done:
                    assert o not in out
                    out[o] = acc
                else:
                    tails[lr] = (o, acc)
                if done:
                    acc = np.zeros(16)
                    s, first = 0, False
                    o += 1
                    while o < NB and not bal_partners(op, role, o, full, cls, nul):
                        o += 1
                    if o < NB:
                        partners = bal_partners(op, role, o, full, cls, nul)
    for lr, (o, acc) in tails.items():
        assert lanes[lr]["tail"] and lanes[lr]["olast"] == o
        for l2 in range(lr + 1, lanes[lr]["last_lane"] + 1):
            acc = acc + heads[l2]
        assert o not in out
        out[o] = acc
    return out


def inner_fused_forward(a, b, metric):
    """The inner product's fused forward round at the level of full blade
    indices: for every output block o and partner S of the class-3 family, the
    lc half (ih = S, jh = S | o, low pattern il inside jl) and the rc half
    (ih = S | o, jh = S, low pattern jl inside il); for o = 0 both halves are
    (S, S) and the shared terms il = jl are taken off the scalar once."""
    import torch
    from oracle import clifford_oracle as O
    n = len(metric)
    sig = O.sign_value_table(n, metric).double().numpy()
    nul = sum(1 << k for k, m in enumerate(metric) if m == 0)
    NB = 1 << (n - 4)
    full = NB - 1
    c = np.zeros(a.shape[:-1] + (1 << n,))
    for o in range(NB):
        for S in bal_partners(INNER, 0, o, full, 3, nul >> 4):
            for il in range(16):
                for jl in range(16):
                    for ih, jh, ok in ((S, S | o, (il & ~jl) == 0), (S | o, S, (jl & ~il) == 0)):
                        if not ok:
                            continue
                        i, j = (ih << 4) | il, (jh << 4) | jl
                        c[..., i ^ j] += sig[i, j] * a[..., i] * b[..., j]
                if o == 0:
                    i = (S << 4) | il
                    c[..., 0] -= sig[i, i] * a[..., i] * b[..., i]
    return c


def inner_union_backward(a, b, gc, metric):
    """The inner product's backward round at the level of full blade indices:
    for every output block o and partner m of the class-4 families, the terms
    (il, jl) with il = jl always, il strictly inside jl when the left block is
    inside the right one, jl strictly inside il when the right block is inside
    the left one. Returns (ga, gb)."""
    from oracle import clifford_oracle as O
    n = len(metric)
    sig = O.sign_value_table(n, metric).double().numpy()
    nul = sum(1 << k for k, m in enumerate(metric) if m == 0) >> 4
    NB = 1 << (n - 4)
    full = NB - 1
    ga = np.zeros(a.shape)
    gb = np.zeros(b.shape)

    def terms(ih, jh):
        lc, rc = (ih & ~jh) == 0, (jh & ~ih) == 0
        for il in range(16):
            for jl in range(16):
                if il == jl or (lc and (il & ~jl) == 0) or (rc and (jl & ~il) == 0):
                    yield (ih << 4) | il, (jh << 4) | jl

    for o in range(NB):
        for m in bal_partners(INNER, 1, o, full, 4, nul):
            for i, j in terms(o, m):
                ga[..., i] += sig[i, j] * b[..., j] * gc[..., i ^ j]
        for m in bal_partners(INNER, 2, o, full, 4, nul):
            for i, j in terms(m, o):
                gb[..., j] += sig[i, j] * a[..., i] * gc[..., i ^ j]
    return ga, gb


# helper lanes of outputs 0 and full (each takes FRAME_HELP[nh][2] of their
# last pairs in the wave's last steps)
FRAME_HELP = {3: (7, ((1, 2), (5, 6)), 1), 4: (11, ((3, 5, 6), (9, 10, 12)), 2)}


def frame_steps_count(nh):
    return FRAME_HELP[nh][0] if nh in FRAME_HELP else (1 << nh) + 1


def frame_step(nh, h, t):
    """Step t of lane h in prod_bwd_inner_frame: (output block o, partner
    block p, sub mode). Sub partners (subsets of h, ascending) first, then sup
    partners (h | S, ascending); at nh = 3 the same lists in the searched
    orders that prod_bwd_*_frame compile (kFrame7Sched). At nh = 3 and 4 outputs 0 and full keep their
    first T steps (output full walks its sup pair (full, full) first, then its
    sub pairs) and helper lanes that finished their own lists take the rest in
    the wave's last steps (nh = 3: quad lanes 1, 2 and 5, 6, one pair each at
    step 6; nh = 4: lanes 3, 5, 6 and 9, 10, 12, two pairs each at steps 9
    and 10); other lanes idle there."""
    full = (1 << nh) - 1
    if nh == 3:  # the compiled table (frame7_tables); an idle step as (h, h, False)
        code = frame7_tables()[0][h][t]
        return (h, h, False) if code & 0x80 else ((code >> 3) & 7, code & 7, bool(code & 0x40))
    if nh in FRAME_HELP:
        T, (h0, hf), c = FRAME_HELP[nh]
        if h == 0:
            return (0, 0, True) if t == 0 else (0, t - 1, False)
        if h == full:
            return (full, full, False) if t == 0 else (full, t - 1, True)
        if t >= T - c and h in h0 + hf:
            k = t - (T - c)
            if h in h0:
                return 0, T - 1 + c * h0.index(h) + k, False
            return full, T - 1 + c * hf.index(h) + k, True
    cs = 1 << popc(h)
    cnt = cs + (1 << (nh - popc(h)))
    subs = subsets(h)
    sups = [h | S for S in subsets(full & ~h)]
    if t < cs:
        return h, subs[t], True
    if t < cnt:
        return h, sups[t - cs], False
    return h, h, False


def _frame_w1(k):
    return ((k >> 1) ^ (k >> 3)) & 1


def _frame_w2(k):
    return (k ^ (k >> 2)) & 1


def inner_frame_backward(a, b, gc, metric):
    """The inner product's backward as prod_bwd_inner_frame computes it
    (4 <= n <= 7, low generators of one metric value, no null generator).
    Lane h accumulates both gradient blocks h in the sup pattern only
    (partner element q containing output element o):
        ga: acc[o] += s_lo(o, q)  Wb[q] g[o ^ q]
        gb: acc[o] += s_lo(q, o)  Wa[q] gt[o ^ q]
    A sub pair (partner inside the output) reads its partner block reversed
    (position q holds element ~q) into an accumulator kept in the reversed
    frame (position o holds output ~o). The partner's flips are the pair's
    high sign, the cross sign on odd elements (|o| for ga, |p| for gb) and, in
    sub mode, w2 (ga) or w1 (gb) plus the parity for a negative low metric;
    gt is g with odd elements flipped when |p| is odd. The frame turn is
    acc[k] <- f(k) acc[15 - k] with f = w1 (ga) or w2 (gb) [+ parity]. The
    pair (h, h) in sub mode reads gc element 0 of block 0 as zero, so its
    diagonal (the only terms reading it) counts once. At nh = 3 the helper
    lanes' sums are added to outputs 0 and 7 after step 6. Returns (ga, gb)."""
    n = len(metric)
    nh = n - 4
    NB = 1 << nh
    full = NB - 1
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    assert all(m != 0 for m in metric) and (neg & 15) in (0, 15)
    lowneg = (neg & 15) == 15
    negh = neg >> 4
    help_ = nh in FRAME_HELP
    T = frame_steps_count(nh)
    h0, hf, c = (FRAME_HELP[nh][1][0], FRAME_HELP[nh][1][1], FRAME_HELP[nh][2]) if help_ else ((), (), 0)
    fa = [(_frame_w1(k) ^ (lowneg & popc(k))) & 1 for k in range(16)]
    fb = [(_frame_w2(k) ^ (lowneg & popc(k))) & 1 for k in range(16)]
    rows = a.shape[:-1]
    ca = [np.zeros(rows + (16,)) for _ in range(NB)]
    cb = [np.zeros(rows + (16,)) for _ in range(NB)]
    ga = np.zeros(a.shape)
    gb = np.zeros(b.shape)

    def turn(acc, f):
        return np.stack([(-1.0 if f[k] else 1.0) * acc[..., 15 - k] for k in range(16)], -1)

    def is_turn(t):
        return 1 <= t <= (NB // 2 if help_ else NB) and (t & (t - 1)) == 0

    ctl = []
    for h in range(NB):
        cs = 1 << popc(h)
        edge = help_ and h in (0, full)
        ctl.append((1 if edge else cs, None, T - 1 if edge else cs + (1 << (nh - popc(h))) - 1))
    for t in range(T):
        for h in range(NB):
            if is_turn(t) and ctl[h][0] == t:
                ca[h], cb[h] = turn(ca[h], fa), turn(cb[h], fb)
            o, p, sub = frame_step(nh, h, t)
            X = o ^ p
            g = gc[..., X * 16:(X + 1) * 16].copy()
            if sub and p == o:  # the diagonal of (o, o) counts in sup mode only
                g[..., 0] = 0.0
            podd, oodd = popc(p) & 1, popc(o) & 1
            gt = np.stack([g[..., x] * (-1.0 if (popc(x) & 1 and podd) else 1.0) for x in range(16)], -1)
            _, s_ga = hi_sign(INNER, o, p, negh, 0, full, 0, 0)
            _, s_gb = hi_sign(INNER, p, o, negh, 0, full, 0, 0)
            wa, wb = [], []
            for q in range(16):
                e = 15 - q if sub else q
                par = popc(q) & 1
                fla = s_ga * (-1 if par and oodd else 1) * (-1 if sub and (_frame_w2(q) ^ (lowneg & par)) else 1)
                flb = s_gb * (-1 if par and podd else 1) * (-1 if sub and (_frame_w1(q) ^ (lowneg & par)) else 1)
                wa.append(fla * b[..., p * 16 + e])
                wb.append(flb * a[..., p * 16 + e])
            for oo in range(16):
                for q in range(16):
                    if oo & ~q & 15:
                        continue
                    ca[h][..., oo] += low_sign(LC, lowneg, oo, q) * wa[q] * g[..., oo ^ q]
                    cb[h][..., oo] += low_sign(RC, lowneg, q, oo) * wb[q] * gt[..., oo ^ q]
        if help_ and t == T - 1:
            ca[0] = ca[0] + sum(ca[x] for x in h0)
            cb[0] = cb[0] + sum(cb[x] for x in h0)
            ca[full] = turn(ca[full] + sum(ca[x] for x in hf), fa)
            cb[full] = turn(cb[full] + sum(cb[x] for x in hf), fb)
        for h in range(NB):
            if ctl[h][2] == t:
                ga[..., h * 16:(h + 1) * 16] = ca[h]
                gb[..., h * 16:(h + 1) * 16] = cb[h]
            if help_ and t == T - c - 1 and h in h0 + hf:  # helpers start from zero
                ca[h] = np.zeros(rows + (16,))
                cb[h] = np.zeros(rows + (16,))
    return ga, gb


def _rho(k):
    """Reversion sign of a blade of grade |k|: (-1)^(|k| (|k| - 1) / 2)."""
    return -1.0 if (popc(k) >> 1) & 1 else 1.0


def contraction_frame_backward(op, a, b, gc, metric):
    """The left (LC) or right (RC) contraction's backward as
    prod_bwd_contr_frame computes it: the inner product's frame schedule
    (frame_step) with one accumulator per lane. A step yields ga (lc: sup
    pairs, rc: sub pairs) or gb (lc: sub pairs, rc: sup pairs) and every step
    runs the ga sup pattern acc[o] += s_lc(o, q) w[q] g[o ^ q]. A gb step uses
    s_rc(q, o) = s_lc(o, q) rho(o) rho(q) rho(o ^ q) (rho: the reversion sign;
    o inside q): its partner and gc blocks take rho(q), rho(x) on top of the
    inner kernel's flips and the result takes rho(o) when stored. A lane
    stores its first output when its first mode ends (turned to the normal
    frame if that mode was sub) and starts from zero, and its second at the
    end of its list; outputs 0 and full add their helpers' sums first.
    Returns (ga, gb)."""
    n = len(metric)
    nh = n - 4
    NB = 1 << nh
    full = NB - 1
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    assert op in (LC, RC) and all(m != 0 for m in metric) and (neg & 15) in (0, 15)
    lowneg = (neg & 15) == 15
    negh = neg >> 4
    help_ = nh in FRAME_HELP
    T = frame_steps_count(nh)
    h0, hf, c = (FRAME_HELP[nh][1][0], FRAME_HELP[nh][1][1], FRAME_HELP[nh][2]) if help_ else ((), (), 0)
    fa = [(_frame_w1(k) ^ (lowneg & popc(k))) & 1 for k in range(16)]
    fb = [(_frame_w2(k) ^ (lowneg & popc(k))) & 1 for k in range(16)]
    rows = a.shape[:-1]
    acc = [np.zeros(rows + (16,)) for _ in range(NB)]
    ga = np.zeros(a.shape)
    gb = np.zeros(b.shape)

    def yields_gb(sub):
        return sub if op == LC else not sub

    def result(x, sub):
        """the stored block of an accumulator that ran in mode sub"""
        if yields_gb(sub):
            x = x * np.array([_rho(k) for k in range(16)])
        if sub:
            f = fb if yields_gb(sub) else fa
            x = np.stack([(-1.0 if f[k] else 1.0) * x[..., 15 - k] for k in range(16)], -1)
        return x

    def put(h, x, sub):
        dst = gb if yields_gb(sub) else ga
        dst[..., h * 16:(h + 1) * 16] = result(x, sub)

    for t in range(T):
        for h in range(NB):
            o, p, sub = frame_step(nh, h, t)
            X = o ^ p
            g = gc[..., X * 16:(X + 1) * 16]
            podd, oodd = popc(p) & 1, popc(o) & 1
            w = []
            for q in range(16):
                e = 15 - q if sub else q
                par = popc(q) & 1
                if yields_gb(sub):
                    _, s = hi_sign(INNER, p, o, negh, 0, full, 0, 0)
                    f = s * (-1 if par and podd else 1) * (-1 if sub and (_frame_w1(q) ^ (lowneg & par)) else 1)
                    w.append(f * _rho(q) * a[..., p * 16 + e])
                else:
                    _, s = hi_sign(INNER, o, p, negh, 0, full, 0, 0)
                    f = s * (-1 if par and oodd else 1) * (-1 if sub and (_frame_w2(q) ^ (lowneg & par)) else 1)
                    w.append(f * b[..., p * 16 + e])
            if yields_gb(sub):
                gg = [g[..., x] * (-1.0 if (popc(x) & 1 and podd) else 1.0) * _rho(x) for x in range(16)]
            else:
                gg = [g[..., x] for x in range(16)]
            for oo in range(16):
                for q in range(16):
                    if oo & ~q & 15:
                        continue
                    acc[h][..., oo] += low_sign(LC, lowneg, oo, q) * w[q] * gg[oo ^ q]
        for h in range(NB):
            o, p, sub = frame_step(nh, h, t)
            last = t == T - 1
            edge = help_ and h in (0, full)
            if edge:
                if t == 0:  # the one-pair first mode of outputs 0 and full
                    put(h, acc[h], sub)
                    acc[h] = np.zeros(rows + (16,))
                elif last:
                    put(h, acc[h] + sum(acc[x] for x in (h0 if h == 0 else hf)), sub)
                continue
            cs = 1 << popc(h)
            end = cs + (1 << (nh - popc(h))) - 1
            if t == cs - 1:  # sub pairs done: the first output
                put(h, acc[h], True)
                acc[h] = np.zeros(rows + (16,))
            if t == end:
                put(h, acc[h], False)
            if help_ and t == T - c - 1 and h in h0 + hf:  # helpers start from zero
                acc[h] = np.zeros(rows + (16,))
    return ga, gb


def wedge_frame_backward(a, b, gc, metric):
    """The wedge product's backward as prod_bwd_contr_frame<WEDGE> computes it
    on the frame schedule: lane h takes ga[h] over its sup steps (partner
    b[p ^ h], gc block p) and gb[~h] over its sub steps (partner a[p], gc
    block ~h ^ p), both on the disjoint pattern acc[o] += s_w(o, q) w[q]
    g[o | q]; a gb step uses s_w(q, o) = s_w(o, q) rho(o) rho(q) rho(o | q)
    (o, q disjoint). No partner block is read reversed. Returns (ga, gb)."""
    n = len(metric)
    nh = n - 4
    NB = 1 << nh
    full = NB - 1
    help_ = nh in FRAME_HELP
    T = frame_steps_count(nh)
    h0, hf, c = (FRAME_HELP[nh][1][0], FRAME_HELP[nh][1][1], FRAME_HELP[nh][2]) if help_ else ((), (), 0)
    rows = a.shape[:-1]
    acc = [np.zeros(rows + (16,)) for _ in range(NB)]
    ga = np.zeros(a.shape)
    gb = np.zeros(b.shape)
    rho = np.array([_rho(k) for k in range(16)])

    def put(h, x, sub):
        if sub:
            gb[..., (full ^ h) * 16:((full ^ h) + 1) * 16] = x * rho
        else:
            ga[..., h * 16:(h + 1) * 16] = x

    for t in range(T):
        for h in range(NB):
            o, p, sub = frame_step(nh, h, t)
            if sub:   # gb[~o]: ih = p, jh = ~o
                jh = full ^ o
                X = p | jh
                _, s = hi_sign(WEDGE, p, jh, 0, 0, full, 0, 0)
                cm = popc(p) & 1
                w = [s * (-1 if (popc(q) & 1 and cm) else 1) * _rho(q) * a[..., p * 16 + q] for q in range(16)]
                g = gc[..., X * 16:(X + 1) * 16]
                gg = [g[..., x] * (-1.0 if (popc(x) & 1 and cm) else 1.0) * _rho(x) for x in range(16)]
            else:     # ga[o]: ih = o, jh = p ^ o
                jh = p ^ o
                _, s = hi_sign(WEDGE, o, jh, 0, 0, full, 0, 0)
                cm = popc(o) & 1
                w = [s * (-1 if (popc(q) & 1 and cm) else 1) * b[..., jh * 16 + q] for q in range(16)]
                g = gc[..., p * 16:(p + 1) * 16]
                gg = [g[..., x] for x in range(16)]
            for oo in range(16):
                for q in range(16):
                    if oo & q:
                        continue
                    acc[h][..., oo] += low_sign(WEDGE, False, oo, q) * w[q] * gg[oo | q]
        for h in range(NB):
            o, p, sub = frame_step(nh, h, t)
            edge = help_ and h in (0, full)
            if edge:
                if t == 0:
                    put(h, acc[h], sub)
                    acc[h] = np.zeros(rows + (16,))
                elif t == T - 1:
                    put(h, acc[h] + sum(acc[x] for x in (h0 if h == 0 else hf)), sub)
                continue
            cs = 1 << popc(h)
            end = cs + (1 << (nh - popc(h))) - 1
            if t == cs - 1:
                put(h, acc[h], True)
                acc[h] = np.zeros(rows + (16,))
            if t == end:
                put(h, acc[h], False)
            if help_ and t == T - c - 1 and h in h0 + hf:
                acc[h] = np.zeros(rows + (16,))
    return ga, gb


def _products_hip():
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "cliffordcuda_amd", "csrc",
                        "products.hip")
    return open(path).read()


def frame7_tables():
    """(kFrame7Sched, kFrame7RowX, kFrame7Swz) as the n = 7 frame kernels
    compile them: per lane h and step t the code p | o << 3 | sub << 6 |
    idle << 7 (an idle step's o and p name the gc and partner blocks it reads),
    the row term and the block swizzle of the LDS slots (2-bit entries)."""
    import re
    text = _products_hip()
    body = re.search(r"kFrame7Sched\[7\] = \{(.*?)\};", text, re.S).group(1)
    steps = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]+)ull", body)]
    assert len(steps) == 7
    rowx = int(re.search(r"kFrame7RowX = (0x[0-9a-fA-F]+)u;", text).group(1), 16)
    swz = int(re.search(r"kFrame7Swz = (0x[0-9a-fA-F]+)u;", text).group(1), 16)
    return [[(steps[t] >> (8 * h)) & 0xff for t in range(7)] for h in range(8)], rowx, swz


def frame7_lds_conflicts(op, sched=None, rowx=None, swz=None):
    """Extra LDS cycles of the n = 7 frame kernels' block reads per chunk and
    32-lane half (rows 0..3; rows 4..7 repeat it) and of their row-order output
    stores, under the measured rules of gen_contr5_schedule. op: "inner"
    (prod_bwd_inner_frame: gc, b and a blocks), "lc", "rc", "wedge" (also the
    regressive product's reads; prod_bwd_contr_frame: gc and one partner
    block). Lane r * 8 + h reads row r's block X at slot 4 X + (swz(X) ^
    rowx(r)), in sub mode the partner's slots reversed (^ 3; not the wedge)."""
    g = contr5_schedule_module()
    if sched is None:
        sched, rowx, swz = frame7_tables()
    sw = (lambda b: (swz >> (2 * b)) & 3) if swz else (lambda b: ((b >> 1) ^ (b >> 3)) & 3)
    rx = lambda r: (rowx >> (2 * (r & 3))) & 3
    slot = lambda r, X, rev=False: r * 512 + 16 * ((X << 2) | (sw(X) ^ rx(r) ^ (3 if rev else 0)))
    reads = 0
    for t in range(7):
        ins = {}
        for lane in range(32):
            h, r = lane & 7, lane >> 3
            c = sched[h][t]
            o, p, sub = (c >> 3) & 7, c & 7, bool(c & 0x40)
            if c & 0x80:
                X, W, rev = o, p, False
            elif op == "inner":
                X, W, rev = o ^ p, p, sub
            elif op == "wedge":
                gbs = sub
                X, W, rev = ((7 ^ o ^ p) if gbs else p), (p if gbs else p ^ o), False
            else:
                X, W, rev = o ^ p, p, sub
            ins.setdefault("g", []).append((lane, 8192 + slot(r, X)))
            ins.setdefault("w", []).append((lane, slot(r, W, rev)))
            if op == "inner":
                ins.setdefault("w2", []).append((lane, 4096 + slot(r, W, rev)))
        reads += sum(g._set_cost(v, g.READ_SETS, 15) for v in ins.values())
    writes = g._set_cost([(lane, slot(lane >> 3, lane & 7)) for lane in range(32)], g.WRITE_SETS, 7)
    return reads, writes


def fwd7_tables():
    """(kFwd7Sched, kFwd7RowX) as prod_fwd_out7 compiles them, read from
    csrc/products.hip: per lane h and step t the pair code (o << 3 | p, or
    0x80 | S << 3 | So for an idle step; byte h of the step's constant), and
    the row term of the LDS slots (entry r & 3 at bits 2 (r & 3))."""
    import os
    import re
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "cliffordcuda_amd", "csrc",
                        "products.hip")
    text = open(path).read()
    rowx = int(re.search(r"kFwd7RowX = (0x[0-9a-fA-F]+)u;", text).group(1), 16)
    body = re.search(r"kFwd7Sched\[4\] = \{(.*?)\};", text, re.S).group(1)
    steps = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]+)ull", body)]
    assert len(steps) == 4
    return [[(steps[t] >> (8 * h)) & 0xff for t in range(4)] for h in range(8)], rowx


def fwd7_step(h, t):
    """Step t of lane h in prod_fwd_out7 (n = 7): (output block o, partner S)
    or None (idle)."""
    code = fwd7_tables()[0][h][t]
    return None if code & 0x80 else ((code >> 3) & 7, code & 7)


def fwd7_read_blocks(op, code):
    """Blocks (S, So) that a step with this code reads: a[S] and b[So] for the
    lc half (the wedge's pair (S, ~o ^ S), the regressive's (o | S, ~S)), a[So]
    and b[S] for the rc half; an idle step names its blocks."""
    full = 7
    if code & 0x80:
        return (code >> 3) & 7, code & 7
    o, p = (code >> 3) & 7, code & 7
    if op == "regressive":
        return o | p, full ^ p
    if op == "wedge":
        return p, full ^ o ^ p
    return p, p | o


def fwd7_lds_conflicts(op, sched=None, rowx=None, swz=None):
    """Extra LDS cycles of prod_fwd_out7's block reads (per chunk, one 32-lane
    half: rows 0..3; rows 4..7 repeat it) and of its row-order output stores,
    under the measured rules of gen_contr5_schedule (READ_SETS, WRITE_SETS).
    Lane r * 8 + h reads row r's blocks at slot 4 X + (swz(X) ^ rowx(r))."""
    g = contr5_schedule_module()
    if sched is None or rowx is None:
        ts, tr = fwd7_tables()
        sched = ts if sched is None else sched
        rowx = tr if rowx is None else rowx
    swz = swz or (lambda b: ((b >> 1) ^ (b >> 3)) & 3)
    rx = lambda r: (rowx >> (2 * (r & 3))) & 3
    slot = lambda r, X, arr: arr * 4096 + r * 512 + 16 * ((X << 2) | (swz(X) ^ rx(r)))
    kL = op != "rc"
    kR = op in ("inner", "rc")
    reads = 0
    for t in range(4):
        ins = {"as": [], "bo": [], "ao": [], "bs": []}
        for lane in range(32):
            h, r = lane & 7, lane >> 3
            S, So = fwd7_read_blocks(op, sched[h][t])
            if kL:
                ins["as"].append((lane, slot(r, S, 0)))
                ins["bo"].append((lane, slot(r, So, 1)))
            if kR:
                ins["ao"].append((lane, slot(r, So, 0)))
                ins["bs"].append((lane, slot(r, S, 1)))
        reads += sum(g._set_cost(v, g.READ_SETS, 15) for v in ins.values() if v)
    ob = (lambda h: 7 ^ h) if op == "wedge" else (lambda h: h)
    writes = g._set_cost([(lane, slot(lane >> 3, ob(lane & 7), 0)) for lane in range(32)], g.WRITE_SETS, 7)
    return reads, writes


# ---- prod_bwd_contr5 / prod_fwd_contr5: contractions on 5 high bits -----------
def contr5_schedule_module():
    """cliffordcuda_amd/csrc/gen_contr5_schedule.py, the generator of the lane
    schedules the kernels compile in (contr5_schedule.h)."""
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "cliffordcuda_amd", "csrc",
                        "gen_contr5_schedule.py")
    spec = importlib.util.spec_from_file_location("gen_contr5_schedule", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _contr5_problem(op, a, b, gc, negh, lowneg, sched, lay=None):
    """One n = 9 problem as prod_bwd_contr5 runs it: per lane slot, steps 0-7
    ga pairs and 8-15 gb pairs (the blocked backward's per-pair arithmetic),
    four 4-step pieces, then per phase the slot's outputs (F, D, H/Q owners
    adding their helpers' partials in slot order). Returns (ga, gb)."""
    lc = op == LC
    steps, outs = sched.steps_by_slot(lc, lay), sched.outputs_by_slot(lc, lay)
    T = _tables(lowneg)
    rows = a.shape[:-1]
    il = np.arange(16)
    full = 31

    def pair(t, o, p):
        g = gc[..., (o ^ p) * 16:((o ^ p) + 1) * 16]
        acc = np.zeros(rows + (16,))
        if t < 8:  # ga[o] over partner b[p]
            ok, s = hi_sign(op, o, p, negh, 0, full, 0, 0)
            assert ok
            bt = b[..., p * 16:(p + 1) * 16] * s * np.where(PARITY16 & (popc(o) & 1), -1.0, 1.0)
            tab = T[op]
            for jl in range(16):
                acc += tab[il, jl] * bt[..., jl:jl + 1] * g[..., il ^ jl]
        else:  # gb[o] over partner a[p]
            ok, s = hi_sign(op, p, o, negh, 0, full, 0, 0)
            assert ok
            fl = np.where(PARITY16 & (popc(p) & 1), -1.0, 1.0)
            at = a[..., p * 16:(p + 1) * 16] * s * fl
            gt = g * fl
            tab = T[op]
            for jl in range(16):
                acc[..., jl] += (tab[il, jl] * at[..., il] * gt[..., il ^ jl]).sum(-1)
        return acc

    pieces = []
    for slot in range(32):
        ys = []
        for t0 in (0, 4, 8, 12):
            acc = np.zeros(rows + (16,))
            for t in range(t0, t0 + 4):
                if steps[slot][t] is not None:
                    acc = acc + pair(t, *steps[slot][t])
            ys.append(acc)
        pieces.append(ys)
    partial = {}
    for slot in range(32):
        for ph in range(2):
            typ, b1, b2, ps, cnt = outs[slot][ph]
            if typ == "help":
                partial[ps] = pieces[slot][2 * ph] + pieces[slot][2 * ph + 1]
    ga = np.zeros(a.shape)
    gb = np.zeros(b.shape)
    seen = set()

    def put(ph, blk, x):
        assert (ph, blk) not in seen
        seen.add((ph, blk))
        (ga if ph == 0 else gb)[..., blk * 16:(blk + 1) * 16] = x

    for slot in range(32):
        for ph in range(2):
            typ, b1, b2, ps, cnt = outs[slot][ph]
            y1, y2 = pieces[slot][2 * ph], pieces[slot][2 * ph + 1]
            if typ == "F":
                put(ph, b1, y1 + y2)
            elif typ == "D":
                put(ph, b1, y1)
                put(ph, b2, y2)
            elif typ == "own":
                u = y1 + y2
                for k in range(cnt):
                    u = u + partial[ps + k]
                put(ph, b1, u)
    assert len(seen) == 64
    return ga, gb


def contraction5_backward(op, a, b, gc, metric):
    """prod_bwd_contr5's backward: lc or rc at n = 9 (no null generator), or lc
    at n = 10 whose only null generator is e9 (two n = 9 problems sharing a0:
    ga0 = ga9(b0, gc0) + ga9(b1, gc1), ga1 = 0, gb0 = gb9(a0, gc0), gb1 =
    gb9(a0, gc1)). Returns (ga, gb)."""
    sched = contr5_schedule_module()
    n = len(metric)
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    lowneg = (neg & 15) == 15
    negh = (neg >> 4) & 31
    if n == 9:
        assert 0 not in metric
        return _contr5_problem(op, a, b, gc, negh, lowneg, sched)
    assert n == 10 and op == LC and metric[9] == 0 and 0 not in metric[:9]
    h = 512
    ga0p, gb0 = _contr5_problem(LC, a[..., :h], b[..., :h], gc[..., :h], negh, lowneg, sched)
    ga1p, gb1 = _contr5_problem(LC, a[..., :h], b[..., h:], gc[..., h:], negh, lowneg, sched)
    ga = np.concatenate([ga0p + ga1p, np.zeros_like(a[..., h:])], -1)
    return ga, np.concatenate([gb0, gb1], -1)


def contraction5_forward(op, a, b, metric):
    """prod_fwd_contr5's forward: lc or rc at n = 9, lc at n = 10 with a null
    top generator (c0 = lc9(a0, b0), c1 = lc9(a0, b1)). Per slot, 8 steps of
    pairs (a[S], b[S | o]) (rc: (a[S | o], b[S])) in two pieces, helper chunks
    added by their owners."""
    sched = contr5_schedule_module()
    n = len(metric)
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    lowneg = (neg & 15) == 15
    negh = (neg >> 4) & 31
    T = _tables(lowneg)
    full = 31

    def problem(a9, b9):
        steps, outs = sched.fwd_steps_by_slot(), sched.fwd_outputs_by_slot()
        rows = a9.shape[:-1]
        pieces = []
        for slot in range(32):
            ys = []
            for t0 in (0, 4):
                acc = np.zeros(rows + (16,))
                for t in range(t0, t0 + 4):
                    st = steps[slot][t]
                    if st is None:
                        continue
                    o, S = st
                    ih, jh = (S, S | o) if op == LC else (S | o, S)
                    ok, s = hi_sign(op, ih, jh, negh, 0, full, 0, 0)
                    assert ok
                    bt = b9[..., jh * 16:(jh + 1) * 16] * s * np.where(PARITY16 & (popc(ih) & 1), -1.0, 1.0)
                    av = a9[..., ih * 16:(ih + 1) * 16]
                    tab = T[op]
                    for tt in range(16):
                        l = np.arange(16)
                        acc[..., tt] += (tab[l, l ^ tt] * av[..., l] * bt[..., l ^ tt]).sum(-1)
                ys.append(acc)
            pieces.append(ys)
        chunks = {}
        for slot in range(32):
            h, how, c0, cnt, cw = outs[slot]
            if cw >= 0:
                chunks[cw] = pieces[slot][1]
        c = np.zeros(a9.shape)
        for slot in range(32):
            h, how, c0, cnt, cw = outs[slot]
            u = pieces[slot][0] + pieces[slot][1] if how == "y1+y2" else pieces[slot][0]
            for k in range(cnt):
                u = u + chunks[c0 + k]
            c[..., h * 16:(h + 1) * 16] = u
        return c

    if n == 9:
        return problem(a, b)
    assert n == 10 and op == LC and metric[9] == 0
    return np.concatenate([problem(a[..., :512], b[..., :512]), problem(a[..., :512], b[..., 512:])], -1)


def _inner5_diag(a, b, gc, negh, lowneg):
    """The element diagonal (i, i) of the (o, o) block pairs, which the lc and the
    rc schedules both count: factor F(o, il) = s_hi(o, o) (-1)^{|il| |o|} s_lo(il, il),
    returned as the corrections (-F b_i gc_0, -F a_i gc_0) for (ga, gb)."""
    f = np.zeros(a.shape[-1])
    for o in range(32):
        _, s = hi_sign(LC, o, o, negh, 0, 31, 0, 0)
        for il in range(16):
            lo = low_sign(LC, lowneg, il, il)
            f[o * 16 + il] = s * lo * (-1.0 if (popc(il) * popc(o)) & 1 else 1.0)
    g0 = gc[..., :1]
    return -f * b * g0, -f * a * g0


def inner5_backward(a, b, gc, metric):
    """prod_bwd_inner5: the inner product's backward on the lc and rc lane schedules
    of prod_bwd_contr5 (the lc pairs, the rc pairs, then the element diagonal of the
    (o, o) block pairs taken off once). n = 9 without a null generator, or n = 10
    whose only null generator is e9: with a = a0 + a1 e9 and b = b0 + b1 e9,
    c0 = inner9(a0, b0) and c1 = lc9(a0, b1) + rc9(a1, beta b0) (beta: the grade
    involution, from moving e9 past the blades of b), so
    ga0 = inner9_ga(b0, gc0) + lc9_ga(b1, gc1), ga1 = rc9_ga(beta b0, gc1),
    gb0 = inner9_gb(a0, gc0) + beta rc9_gb(a1, gc1), gb1 = lc9_gb(a0, gc1)."""
    sched = contr5_schedule_module()
    n = len(metric)
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    lowneg = (neg & 15) == 15
    negh = (neg >> 4) & 31

    lays = sched.INNER_LAYOUT

    def inner9(a9, b9, g9):
        gal, gbl = _contr5_problem(LC, a9, b9, g9, negh, lowneg, sched, lays[True])
        gar, gbr = _contr5_problem(RC, a9, b9, g9, negh, lowneg, sched, lays[False])
        ca, cb = _inner5_diag(a9, b9, g9, negh, lowneg)
        return gal + gar + ca, gbl + gbr + cb

    if n == 9:
        assert 0 not in metric
        return inner9(a, b, gc)
    assert n == 10 and metric[9] == 0 and 0 not in metric[:9]
    h = 512
    beta = np.array([-1.0 if popc(j) & 1 else 1.0 for j in range(h)])
    a0, a1, b0, b1, g0, g1 = a[..., :h], a[..., h:], b[..., :h], b[..., h:], gc[..., :h], gc[..., h:]
    ga0, gb0 = inner9(a0, b0, g0)
    gal, gb1 = _contr5_problem(LC, a0, b1, g1, negh, lowneg, sched, lays[True])
    ga1, gbr = _contr5_problem(RC, a1, beta * b0, g1, negh, lowneg, sched, lays[False])
    return np.concatenate([ga0 + gal, ga1], -1), np.concatenate([gb0 + beta * gbr, gb1], -1)
