"""CPU oracle for the Clifford product & rotor hot path (TEST INFRASTRUCTURE).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. The shipped package (``cliffordcuda_amd``) never routes through it.

It is a plain torch restatement (CPU, any float dtype; fp64 for parity) of the
reference library's einsum/Cayley-table path:

* ``sign_value_table``      follows ``src/cliffordcuda/extensions/ga/geom_prod.py:44-74``
* ``product_masks``         follows ``_shared/_einsum_refs.py:58-83``
* ``einsum_product``        follows ``_shared/_einsum_refs.py:26-55``
                            (outer product x sign/mask table -> XOR scatter-add)
* ``regressive``            follows ``_shared/_einsum_refs.py:86-124`` (dual o wedge o dual)
* graded ops                follow ``src/cliffordcuda/algebra.py:195-334``
* ``rotor_from_bivector`` / ``apply_bivector`` restate the composite of
  ``src/cliffordcuda/algebra.py:343-373`` (eigh-exp -> Givens factor ->
  Givens apply), which computes the Euclidean sandwich ``~R x R`` with
  ``R = exp(sum_m b_m e_{i_m} e_{j_m})`` and the bivector in
  ``torch.triu_indices(n, n, 1)`` order (``algebra.py:116-140``). The
  reference ignores the metric on this path, so the oracle does too.
* ``rotation_matrix`` / ``givens_factor`` / ``compile_bivector_cs`` restate
  ``compile_bivector`` (``algebra.py:343-352``: eigh-exp -> Givens factor,
  ``givens_factor.cu:23-55``), the (C(n,2), 2) cs tensor it returns;
  ``givens_chain_apply`` restates ``apply_rotor(cs, x)``
  (``givens_apply_mb_perm_packed.cu:33-64``, tables ``_utils/core.py:19-50``)
  and ``givens_chain_backward_ref`` its backward
  (``givens_apply_mb_perm_packed.cu:111-160``).

Pinning (how each function is checked independently of its own formula) is
listed per function below and exercised in ``tests/test_oracle.py``.
Autograd through these functions is the backward oracle.
"""
from __future__ import annotations

import math
from functools import lru_cache

import torch

OPS = ("geom", "wedge", "inner", "lc", "rc", "regressive")


def normalize_metric(n: int, metric) -> tuple:
    """metric=None -> Cl(n,0); else a length-n tuple in {-1,0,1}.
    Follows ``geom_prod.py:32-41``.
    Pinned by: tests/test_oracle.py::test_normalize_metric."""
    if metric is None:
        return (1,) * n
    metric = tuple(int(m) for m in metric)
    if len(metric) != n:
        raise ValueError(f"metric must have {n} entries, got {len(metric)}")
    if any(m not in (-1, 0, 1) for m in metric):
        raise ValueError(f"metric entries must be in {{-1, 0, 1}}, got {metric}")
    return metric


@lru_cache(maxsize=None)
def _sign_value_table_cached(n: int, metric: tuple) -> torch.Tensor:
    dim = 1 << n
    i = torch.arange(dim, dtype=torch.int64).view(dim, 1).expand(dim, dim)
    j = torch.arange(dim, dtype=torch.int64).view(1, dim).expand(dim, dim)
    parity = torch.zeros(dim, dim, dtype=torch.int64)
    # reorder parity: number of pairs (a, b), a > b, bit a of i and bit b of j
    for a in range(n):
        ia = (i >> a) & 1
        for b in range(a):
            parity += ia * ((j >> b) & 1)
    sign = 1 - 2 * (parity & 1)
    common = i & j
    for k in range(n):
        m = metric[k]
        if m == 1:
            continue
        hit = ((common >> k) & 1).bool()
        sign = torch.where(hit, sign * m, sign)
    return sign.to(torch.int8)


def sign_value_table(n: int, metric=None) -> torch.Tensor:
    """sigma[i, j] in {-1, 0, +1}: e_i e_j = sigma[i, j] e_{i^j} in Cl(p,q,r),
    bit-pattern blade order. Restates ``geom_prod.py:44-74``:
    (-1)^{#(a>b: i_a=1, j_b=1)} * prod_{k in i&j} metric[k].
    Pinned by: brute-force generator-list reordering (textbook canonical
    ordering with contraction), real matrix representations (gamma matrices),
    e_k^2 = metric[k], anticommutation and associativity."""
    return _sign_value_table_cached(n, normalize_metric(n, metric))


def product_masks(n: int, op: str) -> torch.Tensor:
    """(D, D) bool mask of the (i, j) terms each product keeps.
    Follows ``_einsum_refs.py:58-83``: geom all; wedge i&j==0; inner
    (i sub j) or (j sub i); lc i sub j; rc j sub i.
    Pinned by: grade-selection definitions on homogeneous inputs
    (wedge = <AB>_{r+s}, lc = <AB>_{s-r}, rc = <AB>_{r-s}, inner = <AB>_{|r-s|})."""
    dim = 1 << n
    i = torch.arange(dim, dtype=torch.int64).view(dim, 1).expand(dim, dim)
    j = torch.arange(dim, dtype=torch.int64).view(1, dim).expand(dim, dim)
    if op == "geom":
        return torch.ones(dim, dim, dtype=torch.bool)
    if op == "wedge":
        return (i & j) == 0
    if op == "inner":
        return ((i & ~j) == 0) | ((j & ~i) == 0)
    if op == "lc":
        return (i & j) == i
    if op == "rc":
        return (i & j) == j
    raise ValueError(f"unknown op {op!r}")


def _xor_scatter(a: torch.Tensor, b: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """out[..., k] = sum_{i, j: i^j=k} signs[i, j] a[..., i] b[..., j].
    The outer-product / scatter-add structure of ``_einsum_refs.py:26-55``,
    chunked over the batch so large rows stay within memory."""
    dim = a.shape[-1]
    idx = torch.arange(dim)
    xor_idx = (idx.view(-1, 1) ^ idx.view(1, -1)).reshape(-1)
    s = signs.to(a.dtype)
    rows = a.reshape(-1, dim)
    cols = b.reshape(-1, dim)
    chunk = max(1, (1 << 24) // (dim * dim))
    outs = []
    for r0 in range(0, rows.shape[0], chunk):
        ra, rb = rows[r0:r0 + chunk], cols[r0:r0 + chunk]
        outer = torch.einsum("bi,bj->bij", ra, rb) * s
        flat = outer.reshape(outer.shape[0], -1)
        out = torch.zeros(outer.shape[0], dim, dtype=a.dtype)
        out = out.scatter_add(1, xor_idx.expand_as(flat), flat)
        outs.append(out)
    if not outs:
        return torch.zeros_like(rows).reshape(a.shape)
    return torch.cat(outs, 0).reshape(a.shape)


def dual_perm_signs(n: int, metric) -> tuple:
    """dual(x)[k] = x[~k] * s[k], s[k] = sigma[~k, full] / I^2.
    Follows ``_einsum_refs.py:107-115``. Non-degenerate metrics only.
    Pinned by: dual(x) == x * I^{-1} computed with the geometric product."""
    metric = normalize_metric(n, metric)
    if 0 in metric:
        raise ValueError(f"dual undefined for degenerate metric {metric}")
    sigma = sign_value_table(n, metric).to(torch.float64)
    dim = 1 << n
    full = dim - 1
    isq = float(sigma[full, full])
    comp = torch.arange(dim) ^ full
    return comp, sigma[comp, full] / isq


def dual(x: torch.Tensor, metric) -> torch.Tensor:
    n = x.shape[-1].bit_length() - 1
    comp, s = dual_perm_signs(n, metric)
    return x.index_select(-1, comp) * s.to(x.dtype)


def einsum_product(op: str, a: torch.Tensor, b: torch.Tensor, metric=None) -> torch.Tensor:
    """The reference einsum product ``op`` (one of OPS) on (..., 2^n) inputs.
    geom/wedge/inner/lc/rc follow ``_einsum_refs.py:26-83``; regressive
    follows ``_einsum_refs.py:86-124`` as dual(dual(a) ^ dual(b))."""
    n = a.shape[-1].bit_length() - 1
    metric = normalize_metric(n, metric)
    if op == "regressive":
        if 0 in metric:
            raise ValueError(f"regressive product undefined for degenerate metric {metric}")
        return dual(einsum_product("wedge", dual(a, metric), dual(b, metric), metric), metric)
    signs = sign_value_table(n, metric).to(torch.float64) * product_masks(n, op)
    return _xor_scatter(a, b, signs)


# ── graded ops (algebra.py:195-334) ─────────────────────────────────────────

def grades(n: int) -> torch.Tensor:
    idx = torch.arange(1 << n)
    g = torch.zeros_like(idx)
    for k in range(n):
        g += (idx >> k) & 1
    return g


def reverse_signs(n: int) -> torch.Tensor:
    """grade k -> (-1)^{k(k-1)/2} (``algebra.py:195-205``)."""
    g = grades(n)
    return torch.where(((g * (g - 1) // 2) % 2) == 1, -1.0, 1.0).to(torch.float64)


def involution_signs(n: int) -> torch.Tensor:
    """grade k -> (-1)^k (``algebra.py:278-286``)."""
    return torch.where((grades(n) % 2) == 1, -1.0, 1.0).to(torch.float64)


def conjugation_signs(n: int) -> torch.Tensor:
    """grade k -> (-1)^{k(k+1)/2} (``algebra.py:288-296``)."""
    g = grades(n)
    return torch.where(((g * (g + 1) // 2) % 2) == 1, -1.0, 1.0).to(torch.float64)


def reverse(x):
    return x * reverse_signs(x.shape[-1].bit_length() - 1).to(x.dtype)


def grade_involution(x):
    return x * involution_signs(x.shape[-1].bit_length() - 1).to(x.dtype)


def clifford_conjugation(x):
    return x * conjugation_signs(x.shape[-1].bit_length() - 1).to(x.dtype)


def grade_projection(x, grade: int):
    """keep grade ``grade`` (``algebra.py:298-306``)."""
    n = x.shape[-1].bit_length() - 1
    return x * (grades(n) == grade).to(x.dtype)


def norm_weights(n: int, metric) -> torch.Tensor:
    """w[b] = prod_{i in b} metric[i] (``algebra.py:325-331``)."""
    metric = normalize_metric(n, metric)
    idx = torch.arange(1 << n)
    w = torch.ones(1 << n, dtype=torch.float64)
    for i in range(n):
        w = w * torch.where(((idx >> i) & 1).bool(), float(metric[i]), 1.0)
    return w


def norm_sq(x, metric):
    """<x ~x>_0 = sum_b x_b^2 w_b (``algebra.py:309-334``). Pinned by
    norm_sq(x) == geom(x, reverse(x))[:, 0] (reference ``test_norm_sq.py:46-63``)."""
    n = x.shape[-1].bit_length() - 1
    return (x * x * norm_weights(n, metric).to(x.dtype)).sum(-1)


# ── broadcast-weight layer (layers.py:30-50) ─────────────────────────────────

def layer_forward(op: str, x: torch.Tensor, w: torch.Tensor, metric=None) -> torch.Tensor:
    """``product(x, weight)`` with weight (1, 2^n) broadcast over the batch,
    x on the left (``layers.py:43-47``)."""
    return einsum_product(op, x, w.expand_as(x), metric)


# ── rotor (algebra.py:337-373, Euclidean semantics) ─────────────────────────

def bivector_blades(n: int):
    """slot m <-> (i_m, j_m) = triu_indices(n, n, 1)[:, m] <-> blade 2^i + 2^j
    (``algebra.py:124-126``, ``_rotor_apply_helpers.py:38-43``)."""
    ij = torch.triu_indices(n, n, offset=1)
    return [(int(i), int(j), (1 << int(i)) | (1 << int(j))) for i, j in ij.t()]


def bivector_to_multivector(biv: torch.Tensor, n: int) -> torch.Tensor:
    """(1, C(n,2)) lex-pair coefficients -> (1, 2^n) multivector sum b_m e_{i_m} e_{j_m}.
    (e_i e_j with i < j is the bit-pattern blade 2^i+2^j with sign +1.)"""
    out = torch.zeros(biv.shape[0], 1 << n, dtype=biv.dtype)
    for m, (_, _, blade) in enumerate(bivector_blades(n)):
        out = out.index_add(1, torch.tensor([blade]), biv[:, m:m + 1])
    return out


def rotor_from_bivector(biv: torch.Tensor, n: int, terms: int = 40) -> torch.Tensor:
    """R = exp(B) in the Euclidean Cl(n,0) by scaling-and-squaring of the
    Taylor series of the geometric-product exponential (fp64)."""
    B = bivector_to_multivector(biv, n)
    mag = float(B.detach().abs().sum())
    s = max(0, int(math.ceil(math.log2(mag + 1e-300))) + 2) if mag > 0.5 else 0
    Bs = B / (2 ** s)
    one = torch.zeros_like(B)
    one[:, 0] = 1.0
    R = one.clone()
    term = one.clone()
    for k in range(1, terms):
        term = einsum_product("geom", term, Bs) / k
        R = R + term
    for _ in range(s):
        R = einsum_product("geom", R, R)
    return R


def apply_bivector(biv: torch.Tensor, x: torch.Tensor, n: int | None = None) -> torch.Tensor:
    """y = ~R x R with R = exp(sum b_m e_{i_m} e_{j_m}) (Euclidean). Restates
    the composite ``compile_bivector`` + ``apply_rotor`` of ``algebra.py:343-373``.
    Pinned by: grade-1 action equals expm(-B), B = 2(M - M^T), M[i_m, j_m] = b_m
    (the matrix ``eigh_exp.cu:286-288`` builds), computed with an independent
    matrix exponential; grade and norm preservation; ~R R = 1."""
    if n is None:
        n = x.shape[-1].bit_length() - 1
    R = rotor_from_bivector(biv, n)
    Rr = reverse(R)
    Rb = R.expand_as(x)
    return einsum_product("geom", einsum_product("geom", Rr.expand_as(x), x), Rb)


def vector_rotation_matrix(biv: torch.Tensor, n: int) -> torch.Tensor:
    """The n x n matrix the sandwich applies to grade-1 coefficients: y_vec = Q v."""
    eye = torch.zeros(n, 1 << n, dtype=biv.dtype)
    for a in range(n):
        eye[a, 1 << a] = 1.0
    y = apply_bivector(biv, eye, n)
    cols = torch.stack([y[:, 1 << a] for a in range(n)], 0)  # (out a, in col)
    return cols


# ── the reference's Givens cs chain (algebra.py:343-369) ────────────────────

def plane_pairs(n: int):
    """Rotation planes (p, q), p < q, in lex order (``givens_factor.cu:23-24``)."""
    return [(p, q) for p in range(n - 1) for q in range(p + 1, n)]


def rotation_matrix(biv: torch.Tensor, n: int) -> torch.Tensor:
    """R = expm(B), B = 2 (M - M^T), M[i_m, j_m] = b_m: the matrix the reference
    exponentiates and factors (``eigh_exp.cu:283-288``; its closed form
    ``eigh_exp.cu:55-67`` is exp(B)). torch's fp64 matrix exponential, so the
    result is differentiable. Pinned by: R^T equals the grade-1 action of the
    sandwich (``vector_rotation_matrix``), itself pinned to scipy's expm(-B)."""
    M = torch.zeros(n, n, dtype=biv.dtype)
    ij = torch.triu_indices(n, n, offset=1)
    M = M.index_put((ij[0], ij[1]), biv.reshape(-1))
    return torch.linalg.matrix_exp(2.0 * (M - M.T))


def givens_factor(R: torch.Tensor) -> torch.Tensor:
    """cs (C(n,2), 2) of the reference's Givens factorisation
    (``givens_factor.cu:23-55``): for the planes (p, q) in lex order,
    a = A[p][p], b = A[q][p], r = sqrt(a^2 + b^2), c = a / r, s_raw = -b / r,
    rows p, q of A rotated (A[p] <- c A[p] - s_raw A[q], A[q] <- s_raw A[p] + c A[q]),
    and (c, -s_raw) stored at index C - 1 - k for the k-th plane (reversed).
    A zero column pair (r = 0) gives the identity (c, s) = (1, 0) here; the
    reference clamps r to 1e-12 and writes (0, 0) there.
    Differentiable (torch ops). Pinned by: reconstruction R = prod_k G_k^T with
    A_final = I (r >= 0 makes the factorisation unique), and the chain apply of
    the factors equals the independently pinned sandwich."""
    n = R.shape[-1]
    A = R.clone()
    pairs = plane_pairs(n)
    C = len(pairs)
    out = [None] * C
    for k, (p, q) in enumerate(pairs):
        a, b = A[p, p], A[q, p]
        r = torch.sqrt(a * a + b * b)
        if float(r.detach()) > 0.0:
            c, s_raw = a / r, -b / r
        else:
            c, s_raw = torch.ones_like(a), torch.zeros_like(a)
        rp, rq = A[p].clone(), A[q].clone()
        A = A.clone()
        A[p] = c * rp - s_raw * rq
        A[q] = s_raw * rp + c * rq
        out[C - 1 - k] = torch.stack([c, -s_raw])
    return torch.stack(out, 0)


def compile_bivector_cs(biv: torch.Tensor, n: int) -> torch.Tensor:
    """The reference's ``compile_bivector`` (``algebra.py:343-352``):
    Givens factors of R = expm(B), differentiable to the bivector."""
    return givens_factor(rotation_matrix(biv, n))


def plane_pair_table(n: int, p: int, q: int):
    """Blade pairs of plane (p, q) and their signs (``_utils/core.py:19-50``):
    i with bit p set and bit q clear, j = i ^ (2^p + 2^q), sign
    (-1)^{(|i| - 1 - |i & (2^p - 1)|) + |i >> (q + 1)|}."""
    ii, jj, sg = [], [], []
    for i in range(1 << n):
        if (i >> p) & 1 and not (i >> q) & 1:
            removal = bin(i).count("1") - 1 - bin(i & ((1 << p) - 1)).count("1")
            insert = bin(i >> (q + 1)).count("1")
            ii.append(i)
            jj.append(i ^ ((1 << p) | (1 << q)))
            sg.append(-1.0 if (removal + insert) & 1 else 1.0)
    return torch.tensor(ii), torch.tensor(jj), torch.tensor(sg, dtype=torch.float64)


def givens_chain_apply(cs: torch.Tensor, x: torch.Tensor, n: int | None = None) -> torch.Tensor:
    """The reference's ``apply_rotor(cs, x)`` forward
    (``givens_apply_mb_perm_packed.cu:33-64``): planes applied lex-first
    (cs index C-1 down to 0), each mapping the pair (x_i, x_j) to
    (c x_i + s sig x_j, -s sig x_i + c x_j); blades holding both or neither of
    p, q are unchanged. Any (c, s), unit or not. Differentiable to cs and x
    (autograd gives the exact derivative of this forward).
    Pinned by: with the factors of R it equals the sandwich ``apply_bivector``;
    one plane of angle t rotates e_p towards e_q in closed form."""
    if n is None:
        n = x.shape[-1].bit_length() - 1
    pairs = plane_pairs(n)
    C = len(pairs)
    y = x
    for k, (p, q) in enumerate(pairs):
        c, s = cs[C - 1 - k, 0], cs[C - 1 - k, 1]
        ii, jj, sg = plane_pair_table(n, p, q)
        sg = sg.to(x.dtype)
        xi, xj = y[..., ii], y[..., jj]
        y = y.clone()
        y[..., ii] = c * xi + s * sg * xj
        y[..., jj] = -s * sg * xi + c * xj
    return y


def givens_chain_backward_ref(cs: torch.Tensor, y: torch.Tensor, gy: torch.Tensor, n: int | None = None):
    """The reference's Givens-apply backward (``givens_apply_mb_perm_packed.cu:111-160``
    and ``mb_perm_packed.py:34-42``), restated: walk the planes from the last
    applied to the first, rebuild each plane's input from its output with the
    transposed pair map (the inverse only when c^2 + s^2 = 1), and accumulate
      grad_c += g_i v_i + g_j v_j,   grad_s += sig (g_i v_j - g_j v_i)
    with g the gradient of the plane's output and v its rebuilt input, summed
    over the batch; the gradient itself goes through the transposed map.
    Returns (grad_cs, grad_x); the reference returns no grad_x.
    Pinned by: equals autograd through ``givens_chain_apply`` for unit pairs."""
    if n is None:
        n = y.shape[-1].bit_length() - 1
    pairs = plane_pairs(n)
    C = len(pairs)
    v = y.clone()
    g = gy.clone()
    gcs = torch.zeros(C, 2, dtype=y.dtype)
    for k in reversed(range(C)):
        p, q = pairs[k]
        c, s = float(cs[C - 1 - k, 0]), float(cs[C - 1 - k, 1])
        ii, jj, sg = plane_pair_table(n, p, q)
        sg = sg.to(y.dtype)
        vi, vj, gi, gj = v[..., ii], v[..., jj], g[..., ii], g[..., jj]
        vi_pre = c * vi - s * sg * vj
        vj_pre = s * sg * vi + c * vj
        gcs[C - 1 - k, 0] = (gi * vi_pre + gj * vj_pre).sum()
        gcs[C - 1 - k, 1] = (sg * (gi * vj_pre - gj * vi_pre)).sum()
        v[..., ii], v[..., jj] = vi_pre, vj_pre
        g[..., ii], g[..., jj] = c * gi - s * sg * gj, s * sg * gi + c * gj
    return gcs, g


# ── multivector inverse (extensions/ga/inverse.py) ──────────────────────────

def inverse_dense(x: torch.Tensor, metric=None) -> torch.Tensor:
    """x^-1 for rows x (B, 2^n) by the dense solve L(x) y = e_0 with
    L[k, j] = sigma(j ^ k, j) x[j ^ k] (the left-multiplication matrix; the
    ground truth of the reference's tests/correctness/test_inverse.py:35-47).
    Differentiable (torch.linalg.solve). Pinned by: x y = y x = 1 with the
    oracle's geometric product."""
    n = x.shape[-1].bit_length() - 1
    metric = normalize_metric(n, metric)
    dim = 1 << n
    sig = sign_value_table(n, metric).to(x.dtype)
    k = torch.arange(dim).view(dim, 1)
    j = torch.arange(dim).view(1, dim)
    S = sig[j ^ k, j.expand(dim, dim)]
    L = S * x[:, j ^ k]
    e0 = torch.zeros(x.shape[0], dim, 1, dtype=x.dtype)
    e0[:, 0, 0] = 1.0
    return torch.linalg.solve(L, e0).squeeze(-1)


def product_coefficients(op: str, a: torch.Tensor, b: torch.Tensor, metric, ks) -> torch.Tensor:
    """Selected output coefficients c[:, k] (k in ks) of a product for large n,
    where the (2^n)^2 sign table does not fit: sigma(i, i ^ k) evaluated for
    one k at a time with the closed form of ``sign_value_table``
    (``geom_prod.py:44-74``) times the op's mask (``_einsum_refs.py:58-83``).
    Geometric, wedge, inner, lc and rc only. Pinned by: equals
    ``einsum_product`` on every coefficient at small n."""
    n = a.shape[-1].bit_length() - 1
    metric = normalize_metric(n, metric)
    dim = 1 << n
    i = torch.arange(dim, dtype=torch.int64)
    out = []
    for k in ks:
        j = i ^ k
        parity = torch.zeros(dim, dtype=torch.int64)
        for s in range(n):
            parity += ((i >> s) & 1) * _bits_below(j, s)
        sign = (1 - 2 * (parity & 1)).to(a.dtype)
        common = i & j
        for g, m in enumerate(metric):
            if m != 1:
                sign = torch.where(((common >> g) & 1).bool(), sign * m, sign)
        if op == "wedge":
            sign = sign * ((i & j) == 0)
        elif op == "inner":
            sign = sign * (((i & ~j) == 0) | ((j & ~i) == 0))
        elif op == "lc":
            sign = sign * ((i & j) == i)
        elif op == "rc":
            sign = sign * ((i & j) == j)
        elif op != "geom":
            raise ValueError(f"unsupported op {op!r}")
        out.append((a * b[:, j] * sign).sum(-1))
    return torch.stack(out, -1)


def _bits_below(j: torch.Tensor, s: int) -> torch.Tensor:
    """Number of set bits of j strictly below position s (the generators of j
    that e_s of i has to pass: pairs (s, t) with s > t, i_s = 1, j_t = 1)."""
    c = torch.zeros_like(j)
    for t in range(s):
        c += (j >> t) & 1
    return c
