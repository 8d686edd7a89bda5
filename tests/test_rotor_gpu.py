"""GPU parity of the rotor path (compile + sandwich, forward and backward to the
bivector and to x) against the fp64 oracle (Euclidean ~R x R, reference
algebra.py:343-373 semantics). Tolerance 1e-5 normwise, values and gradients."""
import pytest
import torch

import cliffordcuda_amd as cc
from oracle import clifford_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-5


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = float(ref.abs().max())
    return float((got - ref).abs().max()) / (den if den > 0 else 1.0)


def oracle_step(biv, x, gy, n):
    b64 = biv.double().requires_grad_()
    x64 = x.double().requires_grad_()
    y64 = O.apply_bivector(b64, x64, n)
    y64.backward(gy.double())
    return y64, b64.grad, x64.grad


def oracle_cs_step(biv, x, gy, n):
    """The reference's compile_bivector + apply_rotor restated (Givens factors
    of expm(B), plane chain), fp64, autograd to the bivector and x; pinned to
    the sandwich oracle in tests/test_oracle.py. Cheap at n = 11, 12, where the
    einsum sandwich's autograd graph would not fit."""
    b64 = biv.double().requires_grad_()
    x64 = x.double().requires_grad_()
    y64 = O.givens_chain_apply(O.compile_bivector_cs(b64, n), x64, n)
    y64.backward(gy.double())
    return y64, b64.grad, x64.grad


@pytest.mark.parametrize("n,metric", [(7, (1,) * 7), (8, (1,) * 7 + (-1,)), (9, (1,) * 9), (10, (1,) * 9 + (0,)),
                                      (11, (1,) * 11), (12, (1,) * 10 + (-1, -1))])
def test_apply_bivector_parity(n, metric):
    cl = cc.CliffordAlgebra(metric, device="cuda")
    g = torch.Generator().manual_seed(n)
    B = 24 if n < 10 else (6 if n == 10 else 5)
    biv = (0.1 ** 0.5) * torch.randn(1, n * (n - 1) // 2, generator=g)
    x = torch.randn(B, 1 << n, generator=g)
    gy = torch.randn(B, 1 << n, generator=g)
    bd = biv.cuda().requires_grad_()
    xd = x.cuda().requires_grad_()
    print(f"[case] rotor n={n} B={B}", flush=True)
    y = cl.apply_bivector(bd, xd)
    y.backward(gy.cuda())
    y64, gb64, gx64 = oracle_step(biv, x, gy, n) if n <= 10 else oracle_cs_step(biv, x, gy, n)
    assert rel_err(y, y64) <= TOL
    assert rel_err(xd.grad, gx64) <= TOL
    assert rel_err(bd.grad, gb64) <= TOL


@pytest.mark.parametrize("n", [7, 8, 9, 10, 11, 12])
def test_compile_bivector_returns_reference_cs(n):
    """compile_bivector returns the reference's (C(n,2), 2) Givens factors of
    expm(B) (planes in lex order, stored reversed, r >= 0), against the
    oracle's restatement of givens_factor.cu at 1e-5; a small and a large
    bivector (planes with c < 0)."""
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    C = n * (n - 1) // 2
    for scale in (0.1 ** 0.5, 2.0):
        biv = scale * torch.randn(1, C, generator=torch.Generator().manual_seed(40 + n))
        print(f"[case] compile cs n={n} scale={scale}", flush=True)
        cs = cl.compile_bivector(biv.cuda())
        assert cs.shape == (C, 2) and cs.dtype == torch.float32
        ref = O.compile_bivector_cs(biv.double(), n)
        assert rel_err(cs, ref) <= TOL, scale


def _unit_cs(C, seed):
    g = torch.Generator().manual_seed(seed)
    ang = 2.0 * torch.randn(C, generator=g)
    return torch.stack([ang.cos(), ang.sin()], 1)


@pytest.mark.parametrize("n", [7, 8, 10, 12])
def test_apply_rotor_on_hand_built_cs(n):
    """apply_rotor on a cs the caller built (unit pairs of random angles, a
    leaf that requires grad): values against the oracle chain, and the
    gradients to cs and to x against autograd through the oracle chain (for
    unit pairs the reference's backward rule is that derivative)."""
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    C = n * (n - 1) // 2
    cs = _unit_cs(C, n)
    g = torch.Generator().manual_seed(100 + n)
    B = 33 if n < 12 else 5
    x = torch.randn(B, 1 << n, generator=g)
    gy = torch.randn(B, 1 << n, generator=g)
    csd = cs.cuda().requires_grad_()
    xd = x.cuda().requires_grad_()
    print(f"[case] apply_rotor hand-built cs n={n} B={B}", flush=True)
    y = cl.apply_rotor(csd, xd)
    y.backward(gy.cuda())
    cs64 = cs.double().requires_grad_()
    x64 = x.double().requires_grad_()
    y64 = O.givens_chain_apply(cs64, x64, n)
    y64.backward(gy.double())
    assert rel_err(y, y64) <= TOL
    assert rel_err(xd.grad, x64.grad) <= TOL
    assert rel_err(csd.grad, cs64.grad) <= TOL


@pytest.mark.parametrize("n", [7, 9])
def test_apply_rotor_non_unit_cs_follows_reference_backward(n):
    """For pairs off the unit circle the reference rebuilds each plane's input
    with the transposed map; cs.grad follows that rule (the oracle's
    restatement of the reference backward), the values and x.grad are exact."""
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    C = n * (n - 1) // 2
    g = torch.Generator().manual_seed(7 * n)
    cs = _unit_cs(C, n) * (0.8 + 0.4 * torch.rand(C, 1, generator=g))
    x = torch.randn(17, 1 << n, generator=g)
    gy = torch.randn(17, 1 << n, generator=g)
    csd = cs.cuda().requires_grad_()
    xd = x.cuda().requires_grad_()
    y = cl.apply_rotor(csd, xd)
    y.backward(gy.cuda())
    x64 = x.double().requires_grad_()
    y64 = O.givens_chain_apply(cs.double(), x64, n)
    y64.backward(gy.double())
    gcs_ref, _ = O.givens_chain_backward_ref(cs.double(), y64.detach(), gy.double(), n)
    assert rel_err(y, y64) <= TOL
    assert rel_err(xd.grad, x64.grad) <= TOL
    assert rel_err(csd.grad, gcs_ref) <= TOL


@pytest.mark.parametrize("n", [8, 9, 11])
def test_compile_then_apply_gradients_on_every_path(n):
    """The reference's explicit composition apply_rotor(compile_bivector(b), x):
    the bivector gradient is the oracle's whichever way it flows: straight
    through the compiled state (cs untouched), through cs and the Givens
    factorisation's backward (cs.retain_grad(), which also exposes cs.grad),
    and a detached copy of cs as a leaf of its own."""
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    C = n * (n - 1) // 2
    g = torch.Generator().manual_seed(60 + n)
    biv = 0.5 * torch.randn(1, C, generator=g)
    x = torch.randn(9, 1 << n, generator=g)
    gy = torch.randn(9, 1 << n, generator=g)
    y64, gb64, gx64 = oracle_cs_step(biv, x, gy, n)
    b64 = biv.double().requires_grad_()
    cs64 = O.compile_bivector_cs(b64, n)
    cs64.retain_grad()
    O.givens_chain_apply(cs64, x.double(), n).backward(gy.double())
    for mode in ("state", "retain", "detached"):
        print(f"[case] compile->apply n={n} mode={mode}", flush=True)
        bd = biv.cuda().requires_grad_()
        xd = x.cuda().requires_grad_()
        cs = cl.compile_bivector(bd)
        if mode == "retain":
            cs.retain_grad()
        if mode == "detached":
            cs = cs.detach().requires_grad_()
        y = cl.apply_rotor(cs, xd)
        y.backward(gy.cuda())
        assert rel_err(y, y64) <= TOL, mode
        assert rel_err(xd.grad, gx64) <= TOL, mode
        if mode != "detached":
            assert rel_err(bd.grad, gb64) <= TOL, mode
        if mode != "state":
            assert rel_err(cs.grad, cs64.grad) <= TOL, mode


@pytest.mark.parametrize("n", [8, 9])
def test_compiled_cs_stays_in_the_graph(n):
    """apply_rotor on the untouched output of compile_bivector keeps cs in y's
    autograd graph, as the reference's GivensFactorFunc output is:
    torch.autograd.grad(y, cs) works and equals the oracle's cs gradient, a
    hook registered on the non-leaf cs fires, and the bivector gradient that
    then flows through cs's node is the oracle's."""
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    C = n * (n - 1) // 2
    g = torch.Generator().manual_seed(80 + n)
    biv = 0.5 * torch.randn(1, C, generator=g)
    x = torch.randn(7, 1 << n, generator=g)
    gy = torch.randn(7, 1 << n, generator=g)
    y64, gb64, gx64 = oracle_cs_step(biv, x, gy, n)
    b64 = biv.double().requires_grad_()
    cs64 = O.compile_bivector_cs(b64, n)
    cs64.retain_grad()
    O.givens_chain_apply(cs64, x.double(), n).backward(gy.double())
    print(f"[case] compiled cs in graph n={n}", flush=True)
    bd = biv.cuda().requires_grad_()
    xd = x.cuda().requires_grad_()
    cs = cl.compile_bivector(bd)
    y = cl.apply_rotor(cs, xd)
    (g_cs,) = torch.autograd.grad(y, (cs,), gy.cuda(), retain_graph=True)
    assert rel_err(g_cs, cs64.grad) <= TOL
    seen = []
    cs.register_hook(lambda g_: seen.append(g_.detach().clone()))
    y.backward(gy.cuda())
    assert len(seen) == 1 and rel_err(seen[0], cs64.grad) <= TOL
    assert rel_err(y, y64) <= TOL
    assert rel_err(xd.grad, gx64) <= TOL
    assert rel_err(bd.grad, gb64) <= TOL


def test_rotor_layer_c4_shape():
    """RotorLayer train mode on Cl(7,1), bivector ~ N(0, 0.1),
    x (131072, 256): full-batch forward + backward against the fp64 oracle.
    The upstream gradient is all ones and y = ~R x R is linear in x, so with
    S = sum_b x_b (fp64): the full-batch bivector gradient equals the oracle's
    bivector gradient on the single row S, sum_b y_b equals the oracle's
    sandwich of S, and every row of the x gradient equals the oracle's x
    gradient of one row (it does not depend on x)."""
    n = 8
    cl = cc.CliffordAlgebra([1] * 7 + [-1], device="cuda")
    layer = cc.RotorLayer(cl).train()
    g = torch.Generator().manual_seed(0)
    biv = (0.1 ** 0.5) * torch.randn(1, 28, generator=g)
    with torch.no_grad():
        layer.bivector.copy_(biv.cuda())
    B = 131072
    x = torch.randn(B, 256, generator=g)
    xd = x.cuda().requires_grad_()
    y = layer(xd)
    y.sum().backward()
    rows = torch.tensor([0, 1, 77, 4096, 65536, B - 1])
    y64, _, gx64 = oracle_step(biv, x[rows], torch.ones(len(rows), 256), n)
    assert rel_err(y[rows.cuda()], y64) <= TOL
    assert rel_err(xd.grad[rows.cuda()], gx64) <= TOL
    S = x.double().sum(0, keepdim=True)
    yS, gbS, gx1 = oracle_step(biv, S, torch.ones(1, 256), n)
    assert rel_err(y.detach().double().sum(0, keepdim=True), yS) <= TOL
    assert rel_err(layer.bivector.grad, gbS) <= TOL
    assert rel_err(xd.grad, gx1.expand(B, 256)) <= TOL


def test_compile_then_apply_eval_cache_and_properties():
    n = 8
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    layer = cc.RotorLayer(cl).eval()
    x = torch.randn(64, 256, device="cuda")
    with torch.no_grad():
        y1 = layer(x)
        layer.bivector.mul_(0.5)          # in-place edit must invalidate the eval cache
        y2 = layer(x)
        cs = cl.compile_bivector(layer.bivector)
        y3 = cl.apply_rotor(cs, x)
    assert not torch.allclose(y1, y2)
    torch.testing.assert_close(y2, y3)
    # norm and grade preservation of the sandwich
    torch.testing.assert_close(cl.norm_sq(y3), cl.norm_sq(x), rtol=1e-5, atol=1e-4)
    for k in range(n + 1):
        torch.testing.assert_close(cl.grade_projection(y3, k),
                                   cl.apply_rotor(cs, cl.grade_projection(x, k)), rtol=1e-5, atol=1e-5)


def _planes_bivector(n, angles, rot_seed=None):
    """Bivector of B = sum_k angle_k (e_{2k} e_{2k+1} plane), optionally turned
    by a random rotation Q (B -> Q B Q^T), so that equal-angle planes are not
    coordinate planes; b_m = B[i_m, j_m] / 2 (B = 2 (M - M^T))."""
    B = torch.zeros(n, n, dtype=torch.float64)
    for k, t in enumerate(angles):
        B[2 * k, 2 * k + 1] = t
        B[2 * k + 1, 2 * k] = -t
    if rot_seed is not None:
        g = torch.Generator().manual_seed(rot_seed)
        Q, _ = torch.linalg.qr(torch.randn(n, n, generator=g, dtype=torch.float64))
        B = Q @ B @ Q.T
    iu = torch.triu_indices(n, n, 1)
    return (B[iu[0], iu[1]] / 2).reshape(1, -1).float()


EQUAL_ANGLE_CASES = [
    (8, [0.7, 0.7], None),                  # two equal coordinate planes
    (8, [0.7, 0.7], 3),                     # two equal planes, turned
    (7, [0.7, 0.7, 0.7], None),             # three equal planes and the zero-angle axis e6
    (7, [0.7, 0.7, 0.7], 4),
    (8, [0.7, 0.7, 0.7, 0.0], 5),           # three equal planes and a zero-angle plane
    (8, [0.7, 0.7 + 1e-6, 0.3], 6),         # nearly equal: inside the reference's 1e-4 cut
    (8, [0.7, 0.7 + 1e-4, 0.3], 7),         # at the cut (eigh_exp.cu:236-237)
]


@pytest.mark.parametrize("scale", [1.0, 25.0])
@pytest.mark.parametrize("n,angles,rot", EQUAL_ANGLE_CASES)
def test_equal_and_large_angles(n, angles, rot, scale):
    """Equal plane angles, where the reference's eigenvector pair pick
    (eigh_exp.cu:297-306) and its 1e-4 cut of near-equal eigenvalues in the
    backward (:236-237) are fragile: the expm-based compile has no such
    branch. Scale 1 and scale 25 (angles up to 17.5 rad, scaling and squaring)
    are both held to the 1e-5 bar, on y, x's gradient and the bivector's
    gradient, with an all-ones and a random upstream gradient, through
    apply_bivector and through compile_bivector + apply_rotor."""
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    biv = _planes_bivector(n, [scale * t for t in angles], rot)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(8, 1 << n, generator=g)
    for gname, gy in (("ones", torch.ones(8, 1 << n)), ("randn", torch.randn(8, 1 << n, generator=g))):
        print(f"[case] equal angles n={n} {angles} rot={rot} scale={scale} gy={gname}", flush=True)
        y64, gb64, gx64 = oracle_step(biv, x, gy, n)
        bd = biv.cuda().requires_grad_()
        xd = x.cuda().requires_grad_()
        y = cl.apply_bivector(bd, xd)
        y.backward(gy.cuda())
        assert rel_err(y, y64) <= TOL
        assert rel_err(xd.grad, gx64) <= TOL
        assert rel_err(bd.grad, gb64) <= TOL
        bd2 = biv.cuda().requires_grad_()
        y2 = cl.apply_rotor(cl.compile_bivector(bd2), x.cuda())
        y2.backward(gy.cuda())
        assert rel_err(y2, y64) <= TOL
        assert rel_err(bd2.grad, gb64) <= TOL


def test_rotor_errors():
    cl = cc.CliffordAlgebra([1] * 6, device="cuda")
    with pytest.raises(ValueError, match="n >= 7"):
        cl.compile_bivector(torch.zeros(1, 15, device="cuda"))
    cl8 = cc.CliffordAlgebra([1] * 8, device="cuda")
    with pytest.raises(ValueError, match="first dim must be 1"):
        cl8.compile_bivector(torch.zeros(2, 28, device="cuda"))
    with pytest.raises(ValueError, match=r"cs must have shape \(28, 2\)"):
        cl8.apply_rotor(torch.zeros(5, device="cuda"), torch.zeros(2, 256, device="cuda"))
    cl13 = cc.CliffordAlgebra([1] * 13, device="cuda")
    with pytest.raises(ValueError, match="n <= 12"):
        cl13.compile_bivector(torch.zeros(1, 78, device="cuda"))


def _rotor_step(cl, biv, x, gy, need_biv=True, need_x=True):
    bd = biv.cuda().requires_grad_(need_biv)
    xd = x.cuda().requires_grad_(need_x)
    y = cl.apply_bivector(bd, xd)
    y.backward(gy.cuda())
    return y.detach(), (bd.grad if need_biv else None), (xd.grad if need_x else None)


@pytest.mark.parametrize("B", [1, 3, 16, 27, 1000, 40001])
def test_rotor8_matrix_path_matches_chain_and_oracle(B, clf_env):
    """n = 8 runs through the Cl(8,0) representation by default; the register
    chain (CLF_ROTOR_PATH=chain) and the oracle give the same values and
    gradients, for batches that leave partial row groups (rows past the end
    must not enter the bivector-gradient sums), and for the gx-only and
    bivector-only backward variants."""
    cl = cc.CliffordAlgebra([1] * 7 + [-1], device="cuda")
    g = torch.Generator().manual_seed(B)
    biv = 0.6 * torch.randn(1, 28, generator=g)
    x = torch.randn(B, 256, generator=g)
    gy = torch.randn(B, 256, generator=g)
    print(f"[case] rotor8 matrix vs chain B={B}", flush=True)
    ym, gbm, gxm = _rotor_step(cl, biv, x, gy)
    _, gb_only, _ = _rotor_step(cl, biv, x, gy, need_x=False)
    _, _, gx_only = _rotor_step(cl, biv, x, gy, need_biv=False)
    clf_env.setenv("CLF_ROTOR_PATH", "chain")
    yc, gbc, gxc = _rotor_step(cl, biv, x, gy)
    clf_env.delenv("CLF_ROTOR_PATH")
    assert rel_err(ym, yc) <= TOL
    assert rel_err(gxm, gxc) <= TOL
    assert rel_err(gbm, gbc) <= TOL
    assert torch.equal(gb_only, gbm)
    assert torch.equal(gx_only, gxm)
    if B <= 1000:
        rows = torch.arange(B)
        y64, gb64, gx64 = oracle_step(biv, x[rows], gy[rows], 8)
        assert rel_err(ym, y64) <= TOL
        assert rel_err(gxm, gx64) <= TOL
        assert rel_err(gbm, gb64) <= TOL


def test_rotor8_state_spin_block():
    """The n = 8 state ends with the 16 x 16 spin matrix U = phi(R): orthogonal,
    and unchanged in sign convention by large angles (c < 0 planes)."""
    cl = cc.CliffordAlgebra([1] * 8, device="cuda")
    for scale in (0.05, 1.0, 3.0):
        biv = scale * torch.randn(1, 28, generator=torch.Generator().manual_seed(11))
        state = cc.rotor._compile_fwd(biv.cuda().reshape(-1), 8)
        assert state.numel() == 8 * 8 + 56 + 256
        U = state[120:].double().view(16, 16).cpu()
        torch.testing.assert_close(U @ U.T, torch.eye(16, dtype=torch.float64), atol=2e-6, rtol=0)


@pytest.mark.parametrize("n,B", [(3, 5), (7, 333), (8, 1), (8, 40001), (9, 77), (12, 9)])
def test_bivector_apply_bwd_matches_two_call_backward(n, B):
    """clf_rotor_bivector_apply_bwd (one call: apply backward, batch sum and
    compile backward, fused into one launch for n <= 8) against
    clf_rotor_apply_bwd + clf_rotor_compile_bwd through the C ABI: gx bitwise,
    the bivector gradient to 1e-6 (the fused launch keeps dL/dQ in fp64
    instead of rounding it to fp32 between the two launches); then the
    oracle on small batches."""
    from cliffordcuda_amd import _lib, rotor
    lib = _lib.load()
    g = torch.Generator().manual_seed(n * 1000 + B)
    C = n * (n - 1) // 2
    biv = (0.6 * torch.randn(1, C, generator=g)).cuda()
    x = torch.randn(B, 1 << n, generator=g).cuda()
    gy = torch.randn(B, 1 << n, generator=g).cuda()
    state = rotor._compile_fwd(biv, n)
    s = _lib.stream_of(x)
    print(f"[case] bivector apply bwd n={n} B={B}", flush=True)
    ws_bytes = lib.clf_rotor_bivector_apply_ws_bytes(n, B)
    ws = torch.empty(ws_bytes // 4 + 64, device="cuda")
    gx1 = torch.empty_like(x)
    gb1 = torch.empty_like(biv)
    _lib.check(lib.clf_rotor_bivector_apply_bwd(n, biv.data_ptr(), state.data_ptr(), x.data_ptr(), gy.data_ptr(),
                                                1 << n, gx1.data_ptr(), gb1.data_ptr(), B, ws.data_ptr(), ws_bytes,
                                                s), "clf_rotor_bivector_apply_bwd")
    ws2_bytes = lib.clf_rotor_apply_ws_bytes(n, B)
    ws2 = torch.empty(ws2_bytes // 4 + 64, device="cuda")
    gx2 = torch.empty_like(x)
    gstate = torch.empty_like(state)
    gb2 = torch.empty_like(biv)
    _lib.check(lib.clf_rotor_apply_bwd(n, state.data_ptr(), x.data_ptr(), gy.data_ptr(), gx2.data_ptr(),
                                       gstate.data_ptr(), B, ws2.data_ptr(), ws2_bytes, s), "clf_rotor_apply_bwd")
    _lib.check(lib.clf_rotor_compile_bwd(n, biv.data_ptr(), gstate.data_ptr(), gb2.data_ptr(), s),
               "clf_rotor_compile_bwd")
    # gx only and g_biv only
    gx3 = torch.empty_like(x)
    gb3 = torch.empty_like(biv)
    _lib.check(lib.clf_rotor_bivector_apply_bwd(n, biv.data_ptr(), state.data_ptr(), x.data_ptr(), gy.data_ptr(),
                                                1 << n, gx3.data_ptr(), None, B, None, 0, s), "gx only")
    _lib.check(lib.clf_rotor_bivector_apply_bwd(n, biv.data_ptr(), state.data_ptr(), x.data_ptr(), gy.data_ptr(),
                                                1 << n, None, gb3.data_ptr(), B, ws.data_ptr(), ws_bytes, s),
               "g_biv only")
    torch.cuda.synchronize()
    assert torch.equal(gx1, gx2) and torch.equal(gx3, gx1)
    assert torch.equal(gb3, gb1)
    assert rel_err(gb1, gb2) <= 1e-6
    if B <= 400 and n <= 9:
        _, gb64, gx64 = oracle_step(biv.cpu(), x.cpu(), gy.cpu(), n)
        assert rel_err(gb1, gb64) <= TOL and rel_err(gx1, gx64) <= TOL
    # a workspace below the stated size is refused before any launch
    assert lib.clf_rotor_bivector_apply_bwd(n, biv.data_ptr(), state.data_ptr(), x.data_ptr(), gy.data_ptr(),
                                            1 << n, None, gb3.data_ptr(), B, ws.data_ptr(), ws_bytes - 4,
                                            s) == _lib.CLF_ERR_WORKSPACE
