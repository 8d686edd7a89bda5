"""CPU model of the matrix-representation geometric product (csrc/rep.hip).

For Cl(p,q) with p - q = 0 or 2 (mod 8) and n = 2k, the algebra is the real
matrix algebra M_m(R), m = 2^k. Generators are real Pauli products
gamma_g = P(x_g, z_g), P(x, z)[r][c] = [c == r ^ x] (-1)^{popc(z & c)}, with
P(x1,z1) P(x2,z2) = (-1)^{popc(z1 & x2)} P(x1^x2, z1^z2). A blade I maps to
phi(e_I) = sign(I) P(x_I, z_I). Conversion a -> phi(a): a signed permutation
into t[x][z], then a Walsh-Hadamard transform over z for each x,
W[x][c] = sum_z t[x][z] (-1)^{popc(z & c)}, and phi(a)[r][c] = W[r ^ c][c].
"""
import numpy as np


def popc(v):
    return bin(v).count("1")


def find_generators(metric):
    """n mutually anticommuting real Pauli products on k = n/2 qubits with
    squares (-1)^{popc(z & x)} = metric[g]; deterministic backtracking."""
    n = len(metric)
    if n % 2 or 0 in metric:
        return None
    if (metric.count(1) - metric.count(-1)) % 8 not in (0, 2):
        return None   # not a real matrix algebra of size 2^(n/2)
    k = n // 2
    cands = [(x, z) for x in range(1 << k) for z in range(1 << k) if (x or z)]

    def sq(c):
        return -1 if popc(c[0] & c[1]) & 1 else 1

    def anti(c, d):
        return (popc(c[1] & d[0]) + popc(d[1] & c[0])) & 1 == 1

    chosen = []

    def rec(g):
        if g == n:
            return True
        for c in cands:
            if sq(c) != metric[g]:
                continue
            if all(anti(c, d) for d in chosen):
                chosen.append(c)
                if rec(g + 1):
                    return True
                chosen.pop()
        return False

    if not rec(0):
        return None
    return chosen


def blade_tables(metric, gens):
    n = len(metric)
    label, sign = [], []
    for I in range(1 << n):
        x = z = 0
        s = 1
        for g in range(n):
            if (I >> g) & 1:
                gx, gz = gens[g]
                if popc(z & gx) & 1:
                    s = -s
                x ^= gx
                z ^= gz
        label.append((x, z))
        sign.append(s)
    return label, sign


def pauli(x, z, m):
    P = np.zeros((m, m))
    for r in range(m):
        c = r ^ x
        P[r, c] = -1.0 if popc(z & c) & 1 else 1.0
    return P


def wht(v):
    v = v.copy()
    h = 1
    m = v.shape[-1]
    while h < m:
        for i in range(0, m, 2 * h):
            a = v[..., i:i + h].copy()
            b = v[..., i + h:i + 2 * h].copy()
            v[..., i:i + h] = a + b
            v[..., i + h:i + 2 * h] = a - b
        h *= 2
    return v


def to_matrix(a, label, sign, m):
    t = np.zeros(a.shape[:-1] + (m, m))
    for I, (x, z) in enumerate(label):
        t[..., x, z] = sign[I] * a[..., I]
    W = wht(t)                      # W[x][c]
    M = np.zeros_like(W)
    for r in range(m):
        for c in range(m):
            M[..., r, c] = W[..., r ^ c, c]
    return M


def from_matrix(M, label, sign, m):
    W = np.zeros_like(M)
    for x in range(m):
        for c in range(m):
            W[..., x, c] = M[..., x ^ c, c]
    t = wht(W) / m                  # t[x][z]
    out = np.zeros(M.shape[:-2] + (m * m,))
    for I, (x, z) in enumerate(label):
        out[..., I] = sign[I] * t[..., x, z]
    return out


# ---- lane-level model of the m = 16 matrix-core kernels -------------------
# One wave converts four rows (row b on lanes 16b .. 16b+15, lane x = l % 16
# holds W[x][.]). MFMA operands come from xor shuffles inside each 16-lane
# row: A[x][k] = W_a[x ^ k][k]; the second operand uses the transposed
# conversion (signs (-1)^{popc(x & z)} folded into t), so that
# B[k][x] = phi(b)^T[x][k] = W'_b[x ^ k][k]. The 4-block 16x16x1 MFMA leaves
# C_b[4g + t][j] in lane 16g + j, register 4b + t; the relayout stores it at
# W_c[i ^ j][j] with a row stride of 20 floats, where lane (b, x) reads row x.

RELAYOUT_STRIDE = 20


def transpose_signs(label):
    """(-1)^{popc(x & z)} per blade: phi(a')  = phi(a)^T for a'_I = that sign * a_I."""
    return [-1 if popc(x & z) & 1 else 1 for (x, z) in label]


def lane_W(rows, label, sign):
    """W[b][x][c] for a (4, 256) group: the per-lane gather + WHT."""
    m = 16
    t = np.zeros((rows.shape[0], m, m))
    for I, (x, z) in enumerate(label):
        t[:, x, z] = sign[I] * rows[:, I]
    return wht(t)


def xor_operand(W):
    """Operand register k of lane (b, x): W[b][x ^ k][k]."""
    m = W.shape[-1]
    op = np.zeros_like(W)
    for x in range(m):
        for k in range(m):
            op[:, x, k] = W[:, x ^ k, k]
    return op


def mfma_4block_16x16x1(opA, opB):
    """acc[l][4b + t] after sum_k of the 4-block MFMA with lane (b, i) giving
    A_b[i][k] = opA[b][i][k] and lane (b, j) giving B_b[k][j] = opB[b][j][k]."""
    acc = np.zeros((64, 16))
    for b in range(4):
        Cb = opA[b] @ opB[b].T            # C_b[i][j] = sum_k A_b[i][k] B_b[k][j]
        for l in range(64):
            g, j = l // 16, l % 16
            for t in range(4):
                acc[l, 4 * b + t] = Cb[4 * g + t, j]
    return acc


def relayout(acc, S=RELAYOUT_STRIDE):
    """LDS round trip of the product: returns W_c[b][x][c] read back by lane (b, x)."""
    lds = np.full(4 * 16 * S, np.nan)
    for l in range(64):
        g, j = l // 16, l % 16
        for b in range(4):
            for t in range(4):
                i = 4 * g + t
                lds[b * 16 * S + (i ^ j) * S + j] = acc[l, 4 * b + t]
    Wc = np.zeros((4, 16, 16))
    for b in range(4):
        for x in range(16):
            Wc[b, x] = lds[b * 16 * S + x * S: b * 16 * S + x * S + 16]
    return Wc


def lane_unconvert(Wc, label, sign):
    t = wht(Wc) / 16.0
    out = np.zeros((Wc.shape[0], 256))
    for I, (x, z) in enumerate(label):
        out[:, I] = sign[I] * t[:, x, z]
    return out


def kernel16_fwd(a, b, label, sign):
    st = transpose_signs(label)
    Wa = lane_W(a, label, sign)
    Wbt = lane_W(b, label, [s * u for s, u in zip(sign, st)])
    return lane_unconvert(relayout(mfma_4block_16x16x1(xor_operand(Wa), xor_operand(Wbt))), label, sign)


def kernel16_bwd(a, b, gc, label, sign):
    st = [s * u for s, u in zip(sign, transpose_signs(label))]
    Wb, Wg = lane_W(b, label, sign), lane_W(gc, label, sign)
    Wat, Wgt = lane_W(a, label, st), lane_W(gc, label, st)
    ga = lane_unconvert(relayout(mfma_4block_16x16x1(xor_operand(Wg), xor_operand(Wb))), label, sign)
    gb = lane_unconvert(relayout(mfma_4block_16x16x1(xor_operand(Wat), xor_operand(Wgt))), label, sign)
    return ga, gb


def odd_row_xor(label, stride=256):
    """Smallest multiple of 4 that, xor-ed into the blade offsets of the odd
    rows, makes every gather of a 32-lane half-wave (two rows) hit 32 distinct
    banks; 0 if none does."""
    inv = {lab: I for I, lab in enumerate(label)}
    for h in range(0, 256, 4):
        if all(len({inv[(x, z)] % 32 for x in range(16)} | {(stride + (inv[(x, z)] ^ h)) % 32 for x in range(16)}) == 32
               for z in range(16)):
            return h
    return 0


# ---- split representation for n' = 9 (p - q = 1 mod 8) and one null top generator ----
# Cl(p', q') with 9 generators and p' - q' = 1 (mod 8) is M_16(R) + M_16(R):
# generators 0..7 (a real-type signature) use the m = 16 tables above and
# phi_+-(e_8) = +-phi(E_8), E_8 = e_0 ... e_7 (phi(E_8)^2 = e_8^2 always holds
# then). Every label (x, z) is hit by one blade I0 without e_8 and one blade I1
# with it: t_+-[x][z] = s(I0) a_I0 +- s(I1) a_I1, and the inverse is
# a_I0 = s(I0) (t_+ + t_-) / 2, a_I1 = s(I1) (t_+ - t_-) / 2 (times 1/16 after
# the inverse WHT). T(a) = (phi_+(a), phi_-(a)) is orthogonal up to 32.


def split_tables(metric9):
    """label (x, z) and sign s(I) of each of the 512 blades of a 9-generator
    signature with p - q = 1 (mod 8); None if it does not split that way."""
    m9 = list(metric9)
    if len(m9) != 9 or 0 in m9 or (m9.count(1) - m9.count(-1)) % 8 != 1:
        return None
    gens = find_generators(m9[:8])
    lab8, sgn8 = blade_tables(m9[:8], gens)
    xE, zE = lab8[255]
    sE = sgn8[255]
    label, sign = [], []
    for I in range(512):
        Il = I & 255
        x, z = lab8[Il]
        s = sgn8[Il]
        if I >> 8:
            if popc(z & xE) & 1:
                s = -s
            s *= sE
            x, z = x ^ xE, z ^ zE
        label.append((x, z))
        sign.append(s)
    return label, sign


def split_to_matrices(a, label, sign, hat=False):
    """(..., 512) -> (..., 2, 16, 16): phi_+(a), phi_-(a) (hat: of the grade involution)."""
    tp = np.zeros(a.shape[:-1] + (16, 16))
    tm = np.zeros_like(tp)
    for I, (x, z) in enumerate(label):
        v = sign[I] * a[..., I] * ((-1) ** popc(I) if hat else 1)
        tp[..., x, z] += v
        tm[..., x, z] += -v if I >> 8 else v
    out = []
    for t in (tp, tm):
        W = wht(t)
        M = np.zeros_like(W)
        for r in range(16):
            for c in range(16):
                M[..., r, c] = W[..., r ^ c, c]
        out.append(M)
    return np.stack(out, axis=-3)


def split_from_matrices(M, label, sign):
    ts = []
    for s in range(2):
        W = np.zeros_like(M[..., s, :, :])
        for x in range(16):
            for c in range(16):
                W[..., x, c] = M[..., s, x ^ c, c]
        ts.append(wht(W) / 16.0)
    tp, tm = ts
    out = np.zeros(M.shape[:-3] + (512,))
    for I, (x, z) in enumerate(label):
        out[..., I] = sign[I] * ((tp[..., x, z] - tm[..., x, z]) if I >> 8 else (tp[..., x, z] + tm[..., x, z])) / 2.0
    return out


def pair_sum(pairs, label, sign):
    """T^{-1}(sum_p opA(T(X_p)) opB(T(Y_p))); pairs of (X, Y, transA, transB, hatX, hatY)."""
    acc = 0.0
    for X, Y, ta, tb, hx, hy in pairs:
        A = split_to_matrices(X, label, sign, hx)
        B = split_to_matrices(Y, label, sign, hy)
        if ta:
            A = np.swapaxes(A, -1, -2)
        if tb:
            B = np.swapaxes(B, -1, -2)
        acc = acc + A @ B
    return split_from_matrices(acc, label, sign)


def degenerate10_fwd(L, R, label, sign):
    """Cl(p', q', 1), null generator 9: (L0 + L1 e9)(R0 + R1 e9) = L0 R0 + (L0 R1 + L1 R0^) e9."""
    L0, L1, R0, R1 = L[..., :512], L[..., 512:], R[..., :512], R[..., 512:]
    c0 = pair_sum([(L0, R0, False, False, False, False)], label, sign)
    c1 = pair_sum([(L0, R1, False, False, False, False), (L1, R0, False, False, False, True)], label, sign)
    return np.concatenate([c0, c1], axis=-1)


def degenerate10_bwd(L, R, G, label, sign):
    L0, L1, R0, R1 = L[..., :512], L[..., 512:], R[..., :512], R[..., 512:]
    G0, G1 = G[..., :512], G[..., 512:]
    gL0 = pair_sum([(G0, R0, False, True, False, False), (G1, R1, False, True, False, False)], label, sign)
    gL1 = pair_sum([(G1, R0, False, True, False, True)], label, sign)
    gR0 = pair_sum([(L0, G0, True, False, False, False), (L1, G1, True, False, True, True)], label, sign)
    gR1 = pair_sum([(L0, G1, True, False, False, False)], label, sign)
    return np.concatenate([gL0, gL1], axis=-1), np.concatenate([gR0, gR1], axis=-1)


# ---- rotor sandwich through the Cl(8,0) representation (csrc/rotor_rep.hip) ----

def permlane_transpose(acc):
    """transpose_blocks: for each t, v_permlane32_swap of registers (t, 8 + t)
    and (4 + t, 12 + t) (upper 32 lanes of the first with lower 32 of the
    second), then v_permlane16_swap of (t, 4 + t) and (8 + t, 12 + t) (odd
    16-lane rows of the first with even rows of the second)."""
    op = acc.copy()

    def swap32(a, b):
        tmp = op[32:, a].copy()
        op[32:, a] = op[:32, b]
        op[:32, b] = tmp

    def swap16(a, b):
        for r in (0, 2):
            hi, lo = slice(16 * (r + 1), 16 * (r + 2)), slice(16 * r, 16 * (r + 1))
            tmp = op[hi, a].copy()
            op[hi, a] = op[lo, b]
            op[lo, b] = tmp

    for t in range(4):
        swap32(t, 8 + t)
        swap32(4 + t, 12 + t)
        swap16(t, 4 + t)
        swap16(8 + t, 12 + t)
    return op.reshape(4, 16, 16)      # [b][j][k]: B operand of the next product


def spin_planes(label, sign, n=8):
    """Per lex plane (p, q): (x, z, sign) with phi(e_p e_q) = sign P(x, z)."""
    out = []
    for p in range(n):
        for q in range(p + 1, n):
            I = (1 << p) | (1 << q)
            x, z = label[I]
            out.append((x, z, sign[I]))
    return out


def spin_matrix(cs, planes):
    """U = U_C ... U_1, U_k = cos(t/2) I + sin(t/2) phi(e_p e_q) for the chain's
    (c, s) = (cos t, sin t), as the compile kernel builds it row by row."""
    U = np.eye(16)
    for (p, q, c, s), (x, z, sg) in zip(cs, planes):
        if c >= 0:
            ch = np.sqrt(0.5 * (1 + c))
            sh = s / (2 * ch)
        else:
            sh = np.sqrt(0.5 * (1 - c)) * (-1 if s < 0 else 1)
            ch = s / (2 * sh)
        V = ch * U
        for r in range(16):
            rx = r ^ x
            f = sg * (-1 if popc(z & rx) & 1 else 1)
            V[r] += sh * f * U[rx]
        U = V
    return U


def rotor16_fwd(x, U, label, sign, transpose=False):
    """rotor16_apply_kernel: phi(y) = V^T phi(x) V, V = U (or U^T)."""
    V = U.T if transpose else U
    opV = np.broadcast_to(V.T, (4, 16, 16))     # lane x, register k: V[k][x]
    p = mfma_4block_16x16x1(xor_operand(lane_W(x, label, sign)), opV)
    acc = mfma_4block_16x16x1(opV, permlane_transpose(p))
    return lane_unconvert(relayout(acc), label, sign)


def rotor16_bwd(x, gy, U, label, sign, planes):
    """rotor16_bwd_kernel for one group of four rows: gx and the per-plane K."""
    st = [s * u for s, u in zip(sign, transpose_signs(label))]
    opU = np.broadcast_to(U, (4, 16, 16))       # lane x, register k: U[x][k]
    p = mfma_4block_16x16x1(xor_operand(lane_W(gy, label, sign)), opU)
    g = mfma_4block_16x16x1(opU, permlane_transpose(p))
    accm = mfma_4block_16x16x1(xor_operand(lane_W(x, label, st)), permlane_transpose(g))
    wgx = relayout(g)
    accm = accm + mfma_4block_16x16x1(xor_operand(lane_W(x, label, sign)), xor_operand(wgx))
    gx = lane_unconvert(wgx, label, sign)
    Mm = np.zeros((16, 16))
    for l in range(64):
        gq, j = l // 16, l % 16
        for t in range(4):
            Mm[4 * gq + t, j] = sum(accm[l, 4 * b + t] for b in range(4))
    K = []
    for (px, pz, sg) in planes:
        tot = sum(Mm[r, r ^ px] * (-1 if popc(pz & (r ^ px)) & 1 else 1) for r in range(16))
        K.append(-sg * tot / 32.0)
    return gx, np.array(K)


def spin_matrix_expm(biv, label, sign, n=8):
    """U = expm(phi(B)), B = sum_m b_m e_{i_m} e_{j_m} in lex order: the spin
    matrix as the compile kernel's second wave computes it (equal to the
    chain's spin_matrix up to an overall sign, which the sandwich ignores)."""
    import scipy.linalg
    B = np.zeros(1 << n)
    m = 0
    for i in range(n):
        for j in range(i + 1, n):
            B[(1 << i) | (1 << j)] = biv[m]
            m += 1
    return scipy.linalg.expm(to_matrix(B, label, sign, 1 << (n // 2)))


def spin_plane_masks(planes):
    """The kernel's plane table: (x, mask) with bit r of mask set where
    f(r) = sign (-1)^{popc(z & (r ^ x))} is -1."""
    out = []
    for x, z, sg in planes:
        mask = 0
        for r in range(16):
            if sg * (-1 if popc(z & (r ^ x)) & 1 else 1) < 0:
                mask |= 1 << r
        out.append((x, mask))
    return out


def mfma_f64_16x16x4(a_lanes, b_lanes):
    """v_mfma_f64_16x16x4: A[i][k] from lane 16k + i, B[k][j] from lane 16k + j;
    returns D[i][j] as d[lane, reg] with lane 16 (i % 4) + j, reg i // 4 (as
    measured on gfx950)."""
    A = np.array([[a_lanes[16 * k + i] for k in range(4)] for i in range(16)])
    Bm = np.array([[b_lanes[16 * k + j] for j in range(16)] for k in range(4)])
    D = A @ Bm
    d = np.zeros((64, 4))
    for i in range(16):
        for j in range(16):
            d[16 * (i % 4) + j, i // 4] = D[i, j]
    return d


def spin_expm_lanes(biv, masks, degree=8):
    """Lane model of the compile kernel's spin wave: Z's A operand, Horner steps
    on the D layout, squaring with the A operand from a row-major copy."""
    lanes = range(64)
    za = np.zeros((64, 4))
    for l in lanes:
        g, i = l >> 4, l & 15
        for m, (x, mask) in enumerate(masks):
            col = i ^ x
            fb = -biv[m] if (mask >> i) & 1 else biv[m]
            for c in range(4):
                if col == 4 * c + g:
                    za[l, c] += fb
    rs = np.abs(za).sum(1)
    rowsum = np.array([rs[i] + rs[16 + i] + rs[32 + i] + rs[48 + i] for i in range(16)])
    nrm, sq = rowsum.max(), 0
    while nrm > 0.25 and sq < 60:
        nrm *= 0.5
        sq += 1
    scale = 2.0 ** -sq
    eye = np.array([[1.0 if 4 * t + (l >> 4) == (l & 15) else 0.0 for t in range(4)] for l in lanes])

    def prod(a_op, e):
        acc = np.zeros((64, 4))
        for c in range(4):
            acc += mfma_f64_16x16x4(a_op[:, c], e[:, c])
        return acc

    e = eye.copy()
    for k in range(degree, 0, -1):
        e = eye + (scale / k) * prod(za, e)
    for _ in range(sq):
        E = np.zeros((16, 16))
        for l in lanes:
            for t in range(4):
                E[4 * t + (l >> 4), l & 15] = e[l, t]
        ea = np.array([[E[l & 15, 4 * c + (l >> 4)] for c in range(4)] for l in lanes])
        e = prod(ea, e)
    U = np.zeros((16, 16))
    for l in lanes:
        for t in range(4):
            U[4 * t + (l >> 4), l & 15] = e[l, t]
    return U


# ---- n = 7 on the 16 x 16 representation (csrc/rep7.hip) -------------------
# Seven anticommuting real Pauli products on 4 qubits represent every
# non-degenerate Cl(p, q), p + q = 7, in M_16(R). The labels of the 128 blades
# span a subspace L of (x, z) space whose x part is all of F_2^4, so each lane x
# holds the labels (x, z0(x) + v), v in V = {z : (0, z) in L}. When q is odd the
# pseudoscalar squares to +1 and the generators are chosen with product label
# (0, 0): phi(e_I) and phi(e_I E) then share a label, V has 4 elements and each
# label carries one even and one odd blade ("pair" mode). phi alone is not
# faithful then, but Phi(a) = (phi(a), phi(a^)) is (a^ the grade involution),
# with Phi^* Phi = 32. When q is even, V has 8 elements and each label one
# blade; phi is faithful and phi^* phi = 16 ("single" mode). A permutation of
# the basis, P(x, z) -> P(A x, A^{-T} z), puts V on the low bits of z, so that
# the lane's W[x][c] = sum_z t[x][z] (-1)^{popc(z & c)} is a small WHT over
# the low bits of c times a sign that depends on the lane and the high bits of c.


def _f2_basis(vecs):
    """Row-reduced basis (list of ints) of the span of vecs over GF(2)."""
    basis = []
    for v in vecs:
        for b in basis:
            v = min(v, v ^ b)
        if v:
            basis.append(v)
    return basis


def find_generators7(metric):
    """7 anticommuting real Pauli products on 4 qubits with squares metric[g],
    whose x parts span F_2^4; for q odd their product label must be (0, 0).
    Deterministic backtracking."""
    if len(metric) != 7 or 0 in metric:
        return None
    pair = metric.count(-1) % 2 == 1
    cands = [(x, z) for x in range(16) for z in range(16) if (x or z)]

    def sq(c):
        return -1 if popc(c[0] & c[1]) & 1 else 1

    def anti(c, d):
        return (popc(c[1] & d[0]) + popc(d[1] & c[0])) & 1 == 1

    chosen = []

    def rec(g):
        if g == 7:
            if len(_f2_basis([cx for cx, _ in chosen])) != 4:
                return False          # every lane x must hold labels
            x = z = 0
            for cx, cz in chosen:
                x ^= cx
                z ^= cz
            return not pair or (x == 0 and z == 0)
        for c in cands:
            if sq(c) != metric[g] or not all(anti(c, d) for d in chosen):
                continue
            chosen.append(c)
            if rec(g + 1):
                return True
            chosen.pop()
        return False

    return list(chosen) if rec(0) else None


def rep7_transform(gens):
    """Generators after the basis permutation that puts V = {z : (0, z) in L}
    on the low bits of z, and dim V."""
    L = _f2_basis([x | (z << 4) for x, z in gens] + [])
    # all of L, then its x = 0 part
    span = {0}
    for b in L:
        span |= {s ^ b for s in span}
    V = _f2_basis(sorted(v >> 4 for v in span if (v & 15) == 0))
    d = len(V)
    cols = list(V)
    for e in (1, 2, 4, 8):
        if len(_f2_basis(cols + [e])) > len(cols):
            cols.append(e)
    assert len(cols) == 4

    def M(v):           # M e_i = cols[i]
        r = 0
        for i in range(4):
            if (v >> i) & 1:
                r ^= cols[i]
        return r

    Minv = {M(v): v for v in range(16)}
    At = lambda x: sum(((popc(cols[i] & x) & 1) << i) for i in range(4))   # A = M^T
    out = [(At(x), Minv[z]) for x, z in gens]
    return out, d


def rep7_tables(metric):
    """(pair, ent, zhi): ent[x] = list of (blade, sign, transposed sign) in slot
    order (pair: slot i -> even blade, odd blade of label (x, zhi << 2 | i);
    single: slot i -> the blade of label (x, zhi << 3 | i)), zhi[x] the lane's
    high z bits."""
    gens = find_generators7(list(metric))
    if gens is None:
        return None
    gens, d = rep7_transform(gens)
    pair = d == 2
    label, sign = blade_tables(list(metric), gens)
    low = (1 << d) - 1
    ent = [[None] * (8 if pair else 8) for _ in range(16)]
    zhi = [None] * 16
    for I, (x, z) in enumerate(label):
        h = z >> d
        assert zhi[x] in (None, h)
        zhi[x] = h
        ts = sign[I] * (-1 if popc(x & z) & 1 else 1)
        k = 2 * (z & low) + (popc(I) & 1) if pair else (z & low)
        assert ent[x][k] is None
        ent[x][k] = (I, sign[I], ts)
    return pair, ent, zhi, gens


def _wht_small(v):
    return wht(np.asarray(v))


def rep7_lane_T(rows, ent, pair, transposed=False):
    """Per lane: the small-WHT values T (and T^ in pair mode) of each row.
    rows (B, 128) -> T (B, 16, 4|8), Th (B, 16, 4) or None."""
    B = rows.shape[0]
    si = 2 if transposed else 1
    if pair:
        u = np.zeros((B, 16, 4))
        w = np.zeros((B, 16, 4))
        for x in range(16):
            for i in range(4):
                E, O = ent[x][2 * i], ent[x][2 * i + 1]
                u[:, x, i] = E[si] * rows[:, E[0]]
                w[:, x, i] = O[si] * rows[:, O[0]]
        return _wht_small(u + w), _wht_small(u - w)
    t = np.zeros((B, 16, 8))
    for x in range(16):
        for i in range(8):
            e = ent[x][i]
            t[:, x, i] = e[si] * rows[:, e[0]]
    return _wht_small(t), None


def rep7_expand(T, zhi, pair):
    """W[b][x][c] = (-1)^{popc(zhi(x) & (c >> d))} T[b][x][c & low]."""
    d = 2 if pair else 3
    W = np.zeros(T.shape[:2] + (16,))
    for x in range(16):
        for c in range(16):
            s = -1 if popc(zhi[x] & (c >> d)) & 1 else 1
            W[:, x, c] = s * T[:, x, c & ((1 << d) - 1)]
    return W


def rep7_dest_operand(T, zhi, pair):
    """Operand register k of lane (b, x) as the kernels build it:
    s_x(k >> d) T[b][x ^ k][k & low]. It differs from xor_operand(rep7_expand(T))
    by the lane-independent sign s_k(k >> d), which both operands of step k
    carry and which therefore cancels in the product (zhi is linear in x)."""
    d = 2 if pair else 3
    low = (1 << d) - 1
    op = np.zeros(T.shape[:2] + (16,))
    for x in range(16):
        for k in range(16):
            s = -1 if popc(zhi[x] & (k >> d)) & 1 else 1
            op[:, x, k] = s * T[:, x ^ k, k & low]
    return op


# DPP row permutations of the operand builder (lane x reads lane perm(x)):
# quad_perm xor 1, 2, 3, row_half_mirror (xor 7), row_mirror (xor 15),
# row_ror:8 (a rotation by 8 in a 16-lane row: xor 8)
DPP_XOR = {"q1": 1, "q2": 2, "q3": 3, "hm": 7, "m": 15, "r8": 8}


def rep7_operand_dpp_plan(pair):
    """For each operand register k, the DPP stages (in order) that the kernels
    apply to source register k & low (operand7_d2 / operand7_d3)."""
    q = lambda j: [] if j == 0 else ["q%d" % j]
    plan = {}
    if pair:
        for j in range(4):
            plan[j] = q(j)
            plan[4 + j] = q(j ^ 3) + ["hm"]
            plan[12 + j] = q(j ^ 3) + ["m"]
            plan[8 + j] = q(j) + ["r8"]
    else:
        for j in range(8):
            if j < 4:
                plan[j] = q(j)
                plan[8 + j] = q(j) + ["r8"]
            else:
                plan[j] = q(j ^ 7) + ["hm"]
                plan[8 + j] = q(j ^ 7) + ["m"]
    return plan


def rep7_lane_Q(Wc, zhi, pair):
    """Q[b][x][i] = sum_c W_c[b][x][c] (-1)^{popc(z_i & c)}, z_i = zhi << d | i."""
    d = 2 if pair else 3
    Y = np.zeros(Wc.shape[:2] + (1 << d,))
    for x in range(16):
        for c in range(16):
            s = -1 if popc(zhi[x] & (c >> d)) & 1 else 1
            Y[:, x, c & ((1 << d) - 1)] += s * Wc[:, x, c]
    return _wht_small(Y)


def rep7_unconvert(Q, Qh, ent, pair):
    out = np.zeros((Q.shape[0], 128))
    for x in range(16):
        if pair:
            for i in range(4):
                E, O = ent[x][2 * i], ent[x][2 * i + 1]
                out[:, E[0]] = E[1] * (Q[:, x, i] + Qh[:, x, i]) / 32.0
                out[:, O[0]] = O[1] * (Q[:, x, i] - Qh[:, x, i]) / 32.0
        else:
            for i in range(8):
                e = ent[x][i]
                out[:, e[0]] = e[1] * Q[:, x, i] / 16.0
    return out


def _rep7_product(Xs, tabs, fwd_pairs):
    """Sum over (X, Y, X transposed conversion, Y transposed conversion) of the
    blockwise MFMA products, unconverted. X, Y: (4, 128) row groups."""
    pair, ent, zhi, _ = tabs
    accs = [0.0, 0.0]
    for X, Y, tx, ty in fwd_pairs:
        TX, ThX = rep7_lane_T(X, ent, pair, tx)
        TY, ThY = rep7_lane_T(Y, ent, pair, ty)
        accs[0] = accs[0] + mfma_4block_16x16x1(rep7_dest_operand(TX, zhi, pair),
                                                rep7_dest_operand(TY, zhi, pair))
        if pair:
            accs[1] = accs[1] + mfma_4block_16x16x1(rep7_dest_operand(ThX, zhi, pair),
                                                    rep7_dest_operand(ThY, zhi, pair))
    Q = rep7_lane_Q(relayout(accs[0]), zhi, pair)
    Qh = rep7_lane_Q(relayout(accs[1]), zhi, pair) if pair else None
    return rep7_unconvert(Q, Qh, ent, pair)


def kernel7_fwd(a, b, tabs):
    """The lanes of one wave on a (4, 128) group: c = a b."""
    return _rep7_product(None, tabs, [(a, b, False, True)])


def kernel7_bwd(a, b, gc, tabs):
    """ga = Phi^-adjoint(G B^T), gb = Phi^-adjoint(A^T G), scaled like the forward."""
    ga = _rep7_product(None, tabs, [(gc, b, False, False)])
    gb = _rep7_product(None, tabs, [(a, gc, True, True)])
    return ga, gb
