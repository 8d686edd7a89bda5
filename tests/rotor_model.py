"""CPU model of the rotor kernels in cliffordcuda_amd/csrc/rotor.hip (math
level): expm of the generator, Givens factorisation, the blade-pair chain,
Gamma, dL/dQ = Q Gamma and the adjoint Frechet derivative of expm."""
import numpy as np
import scipy.linalg


def generator(biv, n):
    A = np.zeros((n, n))
    m = 0
    for i in range(n):
        for j in range(i + 1, n):
            A[i, j] = -2.0 * biv[m]
            A[j, i] = 2.0 * biv[m]
            m += 1
    return A


def givens(Q):
    n = Q.shape[0]
    E = Q.copy()
    cs = []
    for p in range(n - 1):
        for q in range(p + 1, n):
            a, b = E[p, p], E[q, p]
            r = np.hypot(a, b)
            c, s = (1.0, 0.0) if r < 1e-300 else (a / r, b / r)
            ep, eq = E[p].copy(), E[q].copy()
            E[p] = c * ep + s * eq
            E[q] = -s * ep + c * eq
            cs.append((p, q, c, s))
    return cs, E


def between(I, p, q):
    return bin(I & (((1 << q) - 1) & ~((2 << p) - 1))).count("1") & 1


def apply_plane(x, p, q, c, s):
    y = x.copy()
    D = x.shape[-1]
    for I in range(D):
        if (I >> p) & 1 and not (I >> q) & 1:
            J = I ^ ((1 << p) | (1 << q))
            sg = -s if between(I, p, q) else s
            y[..., I] = c * x[..., I] - sg * x[..., J]
            y[..., J] = c * x[..., J] + sg * x[..., I]
    return y


def apply(cs, x, transpose=False):
    seq = cs if transpose else cs[::-1]
    for p, q, c, s in seq:
        x = apply_plane(x, p, q, c, -s if transpose else s)
    return x


def gamma(x, gx, n):
    G = np.zeros((n, n))
    D = 1 << n
    for a in range(n):
        for b in range(n):
            for I in range(D):
                if not (I >> b) & 1:
                    continue
                if a == b:
                    G[b, b] += (x[..., I] * gx[..., I]).sum()
                elif not (I >> a) & 1:
                    J = I ^ ((1 << a) | (1 << b))
                    sg = -1.0 if between(I, min(a, b), max(a, b)) else 1.0
                    G[a, b] += sg * (x[..., I] * gx[..., J]).sum()
    return G


def compile_bwd(biv, n, dLdQ):
    A = generator(biv, n)
    Z = np.zeros((2 * n, 2 * n))
    Z[:n, :n] = A.T
    Z[n:, n:] = A.T
    Z[:n, n:] = dLdQ
    F = scipy.linalg.expm(Z)[:n, n:]
    out = []
    for i in range(n):
        for j in range(i + 1, n):
            out.append(-2.0 * (F[i, j] - F[j, i]))
    return np.array(out)
