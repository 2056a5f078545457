"""Pins the operator oracle (oracle/sph.py, oracle/neighbors.py) by mathematics:
kernel normalisation integrals, linear-field exactness of the corrected
gradient, invariances, two-particle closed forms, and autograd of the dense
brute force (oracle/bruteforce.py) for every backward formula."""
import math

import numpy as np
import pytest
import torch

import helpers as H
from oracle import binning, bruteforce as bf, neighbors as nb, sph


def _setup(x, gs, eps, periodic, mode="grid", maxp=16, queries=None):
    spec = nb.GridSpec(tuple(gs), eps, periodic, mode, maxp)
    inst = binning.instantiate(x, gs, eps, periodic, mode, maxp)
    B, N = x.shape[:2]
    s0 = np.zeros((B, N, 1), np.float32)
    m0 = np.ones((B, N), np.float32)
    xb, _, _ = binning.bin_particles(x, s0, m0, inst["permutation"])
    pairs = nb.candidate_pairs(xb, inst["bin_offsets"], spec, queries)
    return spec, inst, xb, sph.Context(pairs, spec)


def _lattice(dim, spacing, half_width):
    ax = np.arange(-half_width, half_width + 1) * spacing
    pts = np.stack(np.meshgrid(*([ax] * dim), indexing="ij"), -1).reshape(-1, dim)
    return pts


@pytest.mark.parametrize("dim", [2, 3])
def test_poly6_normalisation_integral(dim):
    """sum_j a^D c6 W(r_j) over a fine lattice -> integral of c6 W = 1."""
    h = 0.5
    a = h / (60 if dim == 2 else 24)
    pts = _lattice(dim, a, int(math.ceil(h / a)) + 1)
    x = np.zeros((1, pts.shape[0], 2 if dim == 2 else 4), np.float32)
    x[0, :, :dim] = pts
    ctr = np.argmin(np.sum(pts ** 2, 1))
    q = binning.instantiate(x, (16,) * dim, h, False, "grid", 16)["permutation"][0, ctr]
    _, _, _, ctx = _setup(x, (16,) * dim, h, False, queries=np.array([q]))
    m = np.full(pts.shape[0], a ** dim)
    rho, _ = sph.density(ctx, m)
    assert abs(rho[0] - 1.0) < 2e-3


@pytest.mark.parametrize("dim", [2, 3])
def test_spiky_moment_matrix_is_identity_on_lattice(dim):
    """cS * sum v r (x) K(r) over a unit-density lattice -> I (pins cS and K)."""
    h = 0.5
    a = h / (60 if dim == 2 else 24)
    pts = _lattice(dim, a, int(math.ceil(h / a)) + 1)
    x = np.zeros((1, pts.shape[0], 2 if dim == 2 else 4), np.float32)
    x[0, :, :dim] = pts
    ctr = np.argmin(np.sum(pts ** 2, 1))
    q = binning.instantiate(x, (16,) * dim, h, False, "grid", 16)["permutation"][0, ctr]
    _, _, xb, ctx = _setup(x, (16,) * dim, h, False, queries=np.array([q]))
    m = np.full(pts.shape[0], a ** dim)
    rho = np.ones(pts.shape[0])
    M, _ = sph.moment_matrix(ctx, m, rho)
    np.testing.assert_allclose(M[0], np.eye(dim), atol=3e-3)


def test_coefficients_follow_textbook_forms():
    for dim in (2, 3):
        for eps in (0.1, 0.0026222667656838894):
            spec = nb.GridSpec((8,) * dim, eps, False)
            c6, cs = spec.coefficients()
            h = float(np.float32(eps))
            e6 = 4 / (math.pi * h ** 8) if dim == 2 else 315 / (64 * math.pi * h ** 9)
            es = 10 / (math.pi * h ** 5) if dim == 2 else 15 / (math.pi * h ** 6)
            assert abs(c6 / e6 - 1) < 2e-6 and abs(cs / es - 1) < 2e-6


def test_two_particle_closed_forms():
    h = 0.3
    d = 0.1
    x = np.array([[[0.0, 0.0], [d, 0.0]]], np.float32)
    spec, inst, xb, ctx = _setup(x, (8, 8), h, False)
    c6, cs = spec.coefficients()
    m = np.array([1.0, 2.0])
    rho, _ = sph.density(ctx, m)
    hh = float(np.float32(h))
    dd = float(np.float32(d))
    W0, W1 = hh ** 6, (hh * hh - dd * dd) ** 3
    order = inst["permutation"][0]
    mb = np.empty(2)
    mb[order] = m
    exp = c6 * np.array([mb[0] * W0 + mb[1] * W1, mb[1] * W0 + mb[0] * W1])
    np.testing.assert_allclose(rho, exp, rtol=1e-12)
    g, _ = sph.density_gradient(ctx, mb)
    mag = 3 * (hh - dd) ** 2
    # particle 0 sits at the origin, its neighbour at +x: grad points to +x
    assert g[0, 0] > 0 and abs(g[0, 1]) == 0
    np.testing.assert_allclose(g[:, 0], cs * np.array([mb[1] * mag, -mb[0] * mag]), rtol=1e-6)


@pytest.mark.parametrize("dim", [2, 3])
def test_linear_field_is_recovered_exactly_by_corrected_gradient(dim):
    rng = np.random.default_rng(1)
    N = 700 if dim == 2 else 1500
    x = np.zeros((1, N, 2 if dim == 2 else 4), np.float32)
    x[0, :, :dim] = rng.random((N, dim)).astype(np.float32)
    h = 0.2 if dim == 2 else 0.3
    spec, inst, xb, ctx = _setup(x, (12,) * dim, h, False)
    A = rng.standard_normal((4, dim))
    s = xb[0, :, :dim].astype(np.float64) @ A.T + 0.7
    m = np.ones(N)
    rho, _ = sph.density(ctx, m)
    out, raw, *_ = sph.gradient_hybrid(ctx, m, rho, s, tol=1e-3)
    inner = np.all((xb[0, :, :dim] > h) & (xb[0, :, :dim] < 1 - h), axis=1)
    np.testing.assert_allclose(out[inner], np.broadcast_to(A, out[inner].shape), atol=1e-9)
    # constant field: zero raw gradient everywhere
    raw_c, _ = sph.gradient(ctx, m, rho, np.full((N, 3), 2.5))
    assert np.abs(raw_c).max() < 1e-9 * np.abs(raw).max()


def test_translation_invariance_periodic():
    rng = np.random.default_rng(2)
    N = 300
    x = (rng.random((1, N, 2)) - 0.5).astype(np.float32)
    s = rng.standard_normal((N, 3))
    gs, h = (10, 10), 0.1
    outs = []
    for shift in (0.0, 0.25):
        xs = (x + np.float32(shift)).astype(np.float32)
        spec, inst, xb, ctx = _setup(xs, gs, h, True)
        order = np.argsort(inst["permutation"][0])  # binned slot -> input index
        m = np.ones(N)
        rho, _ = sph.density(ctx, m)
        g, _ = sph.gradient(ctx, m, rho, s[order])
        cnt, _ = sph.count(ctx)
        back = np.empty_like(rho)
        back[order] = rho
        gb = np.empty_like(g)
        gb[order] = g
        outs.append((back, gb, np.sort(cnt)))
    np.testing.assert_allclose(outs[0][0], outs[1][0], rtol=1e-4)
    np.testing.assert_allclose(outs[0][1], outs[1][1], rtol=1e-3, atol=1e-3 * np.abs(outs[0][1]).max())


def test_pairs_match_all_pairs_scan():
    """The stencil traversal finds exactly the all-pairs in-radius set."""
    rng = np.random.default_rng(4)
    for dim, periodic in ((2, False), (2, True), (3, False), (3, True)):
        x = ((rng.random((2, 150, 2 if dim == 2 else 4)) - 0.5) * 1.6).astype(np.float32)
        gs = (8,) * dim
        spec, inst, xb, ctx = _setup(x, gs, 0.2, periodic)
        flat = xb.reshape(300, -1)
        got = set(zip(ctx.p.i.tolist(), ctx.p.j.tolist()))
        ref = set()
        for i in range(300):
            b = i // 150
            js = np.arange(b * 150, b * 150 + 150)
            r = nb.displacement_f32(flat[i][None], flat[js], spec)
            ok = nb.sqnorm_f32(r) < spec.eps2_f32()
            ref |= {(i, int(j)) for j in js[ok]}
        assert got == ref


def _dense_pins(dim, periodic, seed):
    rng = np.random.default_rng(seed)
    B, N, C = 2, 90, 4
    gs, eps = (8,) * dim, 0.2
    x = ((rng.random((B, N, 2 if dim == 2 else 4)) - 0.5) * 1.6).astype(np.float32)
    if dim == 3:
        x[..., 3] = 0
    s = rng.standard_normal((B, N, C)).astype(np.float32)
    m = (rng.random((B, N)) + 0.5).astype(np.float32)
    spec = nb.GridSpec(gs, eps, periodic)
    inst = binning.instantiate(x, gs, eps, periodic, "grid", 16)
    xb, sb, mb = binning.bin_particles(x, s, m, inst["permutation"])
    pairs = nb.candidate_pairs(xb, inst["bin_offsets"], spec)
    ctx = sph.Context(pairs, spec)
    r_val = np.zeros((B, N, N, dim))
    mask = np.zeros((B, N, N), bool)
    for b in range(B):
        for i in range(N):
            r_val[b, i] = nb.displacement_f32(xb[b, i][None], xb[b], spec)
    mask[pairs.i // N, pairs.i % N, pairs.j % N] = True
    return B, N, C, spec, ctx, xb, sb, mb, r_val, mask


@pytest.mark.parametrize("dim,periodic", [(2, False), (3, False), (2, True), (3, True)])
def test_backward_formulas_equal_autograd(dim, periodic):
    B, N, C, spec, ctx, xb, sb, mb, r_val, mask = _dense_pins(dim, periodic, 10 + dim)
    dt = torch.float64
    xt = torch.tensor(xb[..., :dim].astype(np.float64), requires_grad=True)
    L, _ = spec.box_f32()
    P = bf.Pairs(xt, float(np.float32(spec.eps)), periodic, torch.tensor(L.astype(np.float64)),
                 torch.tensor(r_val), torch.tensor(mask))
    c6, cs = spec.coefficients()
    mt = torch.tensor(mb.astype(np.float64))
    mf = mb.reshape(-1).astype(np.float64)
    sf = sb.reshape(-1, C).astype(np.float64)
    rho = sph.density(ctx, mf)[0]
    np.testing.assert_allclose(bf.density(P, mt, c6).detach().numpy().ravel(), rho, rtol=1e-12)
    st = torch.tensor(sf.reshape(B, N, C), requires_grad=True)
    rt = torch.tensor(rho.reshape(B, N), requires_grad=True)
    rng = np.random.default_rng(0)
    # the reference's backward uses x_i - x_j wrapped on its own; periodic
    # wrap rounding makes that differ from -(x_j - x_i) in the last fp32 bit
    tol = 1e-10 if not periodic else 3e-6
    cases = {
        "blur": (lambda: bf.blur(P, mt, rt, st, c6), (B, N, C), lambda g: sph.blur_backward(ctx, mf, rho, sf, g)),
        "gradient": (lambda: bf.gradient(P, mt, rt, st, cs), (B, N, C, dim),
                     lambda g: sph.gradient_backward(ctx, mf, rho, sf, g)),
        "density": (lambda: bf.density(P, mt, c6), (B, N), lambda g: [sph.density_backward(ctx, mf, g)]),
        "density_gradient": (lambda: bf.density_gradient(P, mt, cs), (B, N, dim),
                             lambda g: [sph.density_gradient_backward(ctx, mf, g)]),
        "moment": (lambda: bf.moment_matrix(P, mt, rt, cs), (B, N, dim, dim),
                   lambda g: (lambda r: [r[0], None, r[1]])(sph.moment_matrix_backward(ctx, mf, rho, g))),
    }
    for name, (fwd, shape, explicit) in cases.items():
        for t in (xt, st, rt):
            t.grad = None
        g = rng.standard_normal(shape)
        (fwd() * torch.tensor(g, dtype=dt)).sum().backward()
        got = explicit(g.reshape((B * N,) + shape[2:]))
        for res, t in zip(got, (xt, st, rt)):
            if res is None:
                continue
            ag = t.grad.numpy().reshape(res[0].shape)
            err = np.abs(ag - res[0]).max() / np.abs(ag).max()
            assert err < tol, f"{name}: {err}"


@pytest.mark.parametrize("dim,periodic", [(2, False), (3, False), (2, True), (3, True)])
def test_forwards_equal_bruteforce(dim, periodic):
    """The oracle's forward sums equal the dense all-pairs forwards of
    oracle/bruteforce.py on the same pair set, with non-uniform masses so that
    the volume m/rho differs between the two ends of a pair.  The brute force
    weights blur, gradient and moment_matrix by the neighbour's volume v_j
    (``torch_sph.py:289-290, 372-373, 460-461``); its forwards are the ones
    whose autograd equals the reference's gather-form backward
    (test_backward_formulas_equal_autograd), so a v_j -> v_i change in the
    oracle fails here."""
    B, N, C, spec, ctx, xb, sb, mb, r_val, mask = _dense_pins(dim, periodic, 20 + dim)
    L, _ = spec.box_f32()
    h = float(np.float32(spec.eps))
    xt = torch.tensor(xb[..., :dim].astype(np.float64))
    P = bf.Pairs(xt, h, periodic, torch.tensor(L.astype(np.float64)), torch.tensor(r_val), torch.tensor(mask))
    c6, cs = spec.coefficients()
    mf = mb.reshape(-1).astype(np.float64)
    sf = sb.reshape(-1, C).astype(np.float64)
    mt = torch.tensor(mb.astype(np.float64))
    st = torch.tensor(sf.reshape(B, N, C))
    rho = sph.density(ctx, mf)[0]
    rt = torch.tensor(rho.reshape(B, N))
    assert np.ptp(mf / rho) > 0.3 * np.mean(mf / rho)  # volumes really differ between particles
    cases = [
        ("count", sph.count(ctx)[0], bf.count(P)),
        ("density", rho, bf.density(P, mt, c6)),
        ("blur", sph.blur(ctx, mf, rho, sf)[0], bf.blur(P, mt, rt, st, c6)),
        ("gradient", sph.gradient(ctx, mf, rho, sf)[0], bf.gradient(P, mt, rt, st, cs)),
        ("density_gradient", sph.density_gradient(ctx, mf)[0], bf.density_gradient(P, mt, cs)),
        ("moment_matrix", sph.moment_matrix(ctx, mf, rho)[0], bf.moment_matrix(P, mt, rt, cs)),
    ]
    for name, got, ref in cases:
        ref = ref.numpy().reshape(got.shape)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err < 1e-12, f"{name}: {err}"


@pytest.mark.parametrize("dim", [2, 3])
def test_three_particle_closed_forms_with_unequal_volumes(dim):
    """blur, gradient and moment_matrix of three collinear particles with
    masses 1, 2, 5 written out by hand: each neighbour term carries the
    NEIGHBOUR's volume m_j / rho_j (poly6 W = (h^2 - d^2)^3, spiky
    K = 3 (h - d)^2 / d * r, r = x_j - x_i)."""
    h, d1, d2 = 0.3, 0.1, 0.17
    P = 2 if dim == 2 else 4
    x = np.zeros((1, 3, P), np.float32)
    x[0, 1, 0], x[0, 2, 0] = d1, -d2
    gs = (8,) * dim
    spec, inst, xb, ctx = _setup(x, gs, h, False)
    c6, cs = spec.coefficients()
    perm = inst["permutation"][0]           # input index -> binned slot
    m_in = np.array([1.0, 2.0, 5.0])
    s_in = np.array([[1.0, -2.0], [0.5, 3.0], [-1.5, 0.25]])
    mb = np.empty(3)
    mb[perm] = m_in
    sb = np.empty((3, 2))
    sb[perm] = s_in
    hh = float(np.float32(h))
    X = np.array([0.0, float(np.float32(d1)), float(np.float32(-d2))])
    rho_in = np.zeros(3)
    for i in range(3):
        for j in range(3):
            dd = abs(X[j] - X[i])
            if dd < hh:
                rho_in[i] += c6 * m_in[j] * (hh * hh - dd * dd) ** 3
    rho_b = np.empty(3)
    rho_b[perm] = rho_in
    v = m_in / rho_in
    blur_e = np.zeros((3, 2))
    grad_e = np.zeros((3, 2, dim))
    mom_e = np.zeros((3, dim, dim))
    for i in range(3):
        for j in range(3):
            r = X[j] - X[i]
            dd = abs(r)
            if dd >= hh:
                continue
            blur_e[i] += c6 * v[j] * (hh * hh - dd * dd) ** 3 * s_in[j]
            if dd > 0:
                K = 3.0 * (hh - dd) ** 2 / dd * r
                grad_e[i, :, 0] += cs * v[j] * (s_in[j] - s_in[i]) * K
                mom_e[i, 0, 0] += cs * v[j] * r * K
    rho, _ = sph.density(ctx, mb)
    np.testing.assert_allclose(rho[perm], rho_in, rtol=1e-6)
    np.testing.assert_allclose(sph.blur(ctx, mb, rho_b, sb)[0][perm], blur_e, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(sph.gradient(ctx, mb, rho_b, sb)[0][perm], grad_e, rtol=1e-6,
                               atol=1e-9 * np.abs(grad_e).max())
    np.testing.assert_allclose(sph.moment_matrix(ctx, mb, rho_b)[0][perm], mom_e, rtol=1e-6,
                               atol=1e-9 * np.abs(mom_e).max())


@pytest.mark.parametrize("dim", [2, 3])
def test_blur_of_constant_field_on_lattice(dim):
    """Shepard check: blur of a constant field, with rho from the density
    operator, returns the constant.  On a lattice every particle whose
    2h-neighbourhood is complete sees the same rho as its neighbours, so
    c6 sum_j (m / rho_j) W_ij = rho_i / rho = 1 up to rounding."""
    h = 0.5
    a = h / (10 if dim == 2 else 5)
    hw = int(math.ceil(2.5 * h / a)) + 1
    pts = _lattice(dim, a, hw)
    x = np.zeros((1, pts.shape[0], 2 if dim == 2 else 4), np.float32)
    x[0, :, :dim] = pts
    gs = (16,) * dim
    spec = nb.GridSpec(gs, h, False, "grid", 16)
    inst = binning.instantiate(x, gs, h, False, "grid", 16)
    xb, _, _ = binning.bin_particles(x, np.zeros((1, pts.shape[0], 1), np.float32),
                                     np.ones((1, pts.shape[0]), np.float32), inst["permutation"])
    box = np.max(np.abs(xb[0, :, :dim]), axis=1)
    near = np.flatnonzero(box < 1.5 * h + 1e-6)   # every neighbour of an inner point
    inner = np.flatnonzero(box < 0.5 * h + 1e-6)
    m = np.full(pts.shape[0], a ** dim)
    rho = np.full(pts.shape[0], np.nan)            # outside `near` never read
    rho[near] = sph.density(sph.Context(nb.candidate_pairs(xb, inst["bin_offsets"], spec, near), spec), m)[0]
    ctx = sph.Context(nb.candidate_pairs(xb, inst["bin_offsets"], spec, inner), spec)
    out, _ = sph.blur(ctx, m, rho, np.full((pts.shape[0], 2), 3.25))
    assert inner.size > 10 and np.isfinite(out).all()
    np.testing.assert_allclose(out, 3.25, rtol=1e-6)  # fp32 lattice positions


def test_gradcheck_small():
    """torch.autograd.gradcheck of the dense float64 forward (clamped 2D)."""
    B, N, C, spec, ctx, xb, sb, mb, r_val, mask = _dense_pins(2, False, 3)
    xt = torch.tensor(xb[..., :2].astype(np.float64), requires_grad=True)
    st = torch.tensor(sb.astype(np.float64), requires_grad=True)
    c6, cs = spec.coefficients()
    mt = torch.tensor(mb.astype(np.float64))
    mk = torch.tensor(mask)
    h = float(np.float32(spec.eps))

    def f(x, s):
        P = bf.Pairs(x, h, mask=mk)
        rho = bf.density(P, mt, c6)
        return bf.blur(P, mt, rho, s, c6).sum(-1), bf.gradient(P, mt, rho, s, cs).sum((-1, -2))

    assert torch.autograd.gradcheck(f, (xt, st), eps=1e-7, atol=1e-5, rtol=1e-4)


def test_safe_inverse():
    rng = np.random.default_rng(6)
    for dim in (2, 3):
        A = rng.standard_normal((200, dim, dim))
        M = A @ np.swapaxes(A, 1, 2) + 0.1 * np.eye(dim)
        L, det = sph.safe_inv_sym(M, 1e-3)
        big = np.abs(det) >= 1e-3
        np.testing.assert_allclose(np.einsum("qab,qbc->qac", M[big], L[big]),
                                   np.broadcast_to(np.eye(dim), M[big].shape), atol=1e-8)
        Z = np.zeros((3, dim, dim))
        Z[:, 0, 0] = 1e-4
        Li, _ = sph.safe_inv_sym(Z, 1e-3)
        np.testing.assert_array_equal(Li, np.broadcast_to(np.eye(dim), Li.shape))


def test_safe_inverse_indefinite():
    """The identity branch is taken on |det| < tol, not det < tol
    (sphops/sph_cuda.cu:3111, 3152): an indefinite matrix with det < -tol is
    inverted, one with -tol < det < 0 is replaced by the identity."""
    for dim in (2, 3):
        mats = H.indefinite_matrices(dim)
        big, small = mats["big"], mats["small"]
        dets = np.linalg.det(big)
        assert np.all(dets < -1e-3)
        L, det = sph.safe_inv_sym(big, 1e-3)
        np.testing.assert_allclose(det, dets, rtol=1e-10)
        np.testing.assert_allclose(L, np.linalg.inv(big), rtol=1e-9, atol=1e-9)
        dets = np.linalg.det(small)
        assert np.all((dets < 0) & (dets > -1e-3))
        L, det = sph.safe_inv_sym(small, 1e-3)
        np.testing.assert_allclose(det, dets, rtol=1e-9, atol=1e-15)
        np.testing.assert_array_equal(L, np.broadcast_to(np.eye(dim), L.shape))
