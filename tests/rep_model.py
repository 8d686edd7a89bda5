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
