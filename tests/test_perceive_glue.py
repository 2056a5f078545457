"""The oracle of NPA.perceive's feature assembly (oracle/perceive.py) on the
CPU: the log-normalisation's closed form, gradcheck of the whole assembly, and
the closed-form Jacobian that the fused HIP backward applies
(npa_amd/csrc/perceive_glue.hip), checked against autograd."""
import numpy as np
import torch

from oracle import perceive as P


def test_log_normalize_closed_form():
    g = torch.Generator().manual_seed(3)
    v = torch.randn(200, 3, generator=g, dtype=torch.float64) * torch.logspace(-6, 3, 200, dtype=torch.float64)[:, None]
    out = P.log_normalize(v)
    n = v.norm(dim=-1)
    # log(1 + u) as the reference writes it: rounding 1 + u costs up to 1.2e-16 absolute
    assert torch.allclose(out.norm(dim=-1), torch.log1p(n), rtol=1e-12, atol=2e-16)
    cos = (out * v).sum(-1) / (out.norm(dim=-1) * n)
    assert torch.allclose(cos, torch.ones_like(cos), rtol=0, atol=1e-12)
    assert torch.equal(P.log_normalize(torch.zeros(4, 2, dtype=torch.float64)), torch.zeros(4, 2, dtype=torch.float64))


def test_features_layout_and_gradcheck():
    g = torch.Generator().manual_seed(5)
    B, N, C, D = 2, 5, 3, 2
    s, bl = (torch.randn(B, N, C, generator=g, dtype=torch.float64, requires_grad=True) for _ in range(2))
    gs = torch.randn(B, N, C, D, generator=g, dtype=torch.float64, requires_grad=True)
    gr = torch.randn(B, N, D, generator=g, dtype=torch.float64, requires_grad=True)
    z = P.features(s, bl, gs, gr, 0.05, 0.1)
    assert z.shape == (B, N, 2 * C + C * D + D)
    assert torch.equal(z[..., :C], s) and torch.equal(z[..., C:2 * C], bl)
    coef = float(np.float32(1.0) / np.float32(0.1) * np.float32(0.05))
    assert torch.allclose(z[..., 2 * C:2 * C + C * D], P.log_normalize(gs * coef).reshape(B, N, -1))
    assert torch.allclose(z[..., -D:], P.log_normalize(gr * coef ** (1 + D) / N))
    assert torch.autograd.gradcheck(lambda a, b, c, d: P.features(a, b, c, d, 0.05, 0.1), (s, bl, gs, gr))
    z2 = P.features(s, bl, None, gr, 0.05, 0.1, log_norm_density_grad=False)
    assert z2.shape == (B, N, 2 * C + D)
    assert torch.allclose(z2[..., -D:], gr * coef ** (1 + D) / N)


def _jt_closed_form(v, w, eps=1e-12):
    """J^T w of the log-normalisation at v, the form the HIP backward uses:
    (phi/m) w + (phi'/m - phi m'/m^2) (v.w) v / u, phi = log(1 + u),
    m = max(u, eps), m' = [u >= eps], and 0 for the second term at u = 0."""
    u = np.linalg.norm(v)
    m = max(u, eps)
    phi = np.log1p(u)
    a = phi / m
    b = 0.0
    if u > 0:
        dm = phi / (m * m) if u >= eps else 0.0
        b = (1.0 / ((1.0 + u) * m) - dm) / u
    return a * w + b * np.dot(v, w) * v


def test_log_normalize_jacobian_closed_form():
    rng = np.random.default_rng(7)
    for D in (2, 3):
        for scale in (1e-3, 0.3, 1.0, 40.0):
            v = rng.standard_normal(D) * scale
            w = rng.standard_normal(D)
            vt = torch.tensor(v, requires_grad=True)
            (P.log_normalize(vt[None])[0] * torch.tensor(w)).sum().backward()
            assert np.allclose(_jt_closed_form(v, w), vt.grad.numpy(), rtol=1e-12, atol=1e-15)
        vt = torch.zeros(D, dtype=torch.float64, requires_grad=True)
        (P.log_normalize(vt[None])[0] * torch.ones(D, dtype=torch.float64)).sum().backward()
        assert np.array_equal(vt.grad.numpy(), _jt_closed_form(np.zeros(D), np.ones(D)))


def test_euler_update_closed_forms_and_gradcheck():
    g = torch.Generator().manual_seed(11)
    B, N, C, D = 2, 6, 3, 3
    y = torch.randn(B, N, D + C, generator=g, dtype=torch.float64)
    y[0, 0, :D] = 0.0
    xb = torch.randn(B, N, 4, generator=g, dtype=torch.float64)
    sb = torch.randn(B, N, C, generator=g, dtype=torch.float64)
    mask = (torch.rand(B, N, 1, generator=g) < 0.5).double()
    x, s, dn = P.euler_update(y, xb, sb, mask, None, 1.5, 0.02, dt=0.5)
    u = y[..., :D].norm(dim=-1)
    assert torch.allclose(dn, 1.5 * 0.02 * u / (1 + u), rtol=1e-14, atol=0)
    dx = (x - xb)[..., :D]
    on = mask[..., 0] > 0
    # direction of a, length dt * |dx| for updated particles; others unchanged
    assert torch.allclose(dx[on].norm(dim=-1), 0.5 * dn[on], rtol=1e-12, atol=1e-15)
    assert torch.allclose((dx[on] * y[..., :D][on]).sum(-1), dx[on].norm(dim=-1) * u[on], rtol=1e-12, atol=1e-15)
    assert torch.equal(x[~on], xb[~on]) and torch.equal(s[~on], sb[~on])
    assert torch.equal(x[..., 3], xb[..., 3])
    assert torch.allclose(s[on], sb[on] + 0.5 * y[..., D:][on])
    ins = [t.clone().requires_grad_(True) for t in (y, xb, sb)]
    noise = torch.randn(B, N, 4, generator=g, dtype=torch.float64)
    y2 = ins[0].detach().clone()
    y2[0, 0, :D] = 0.3  # gradcheck away from the norm's kink at a = 0
    ins[0] = y2.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b, c: P.euler_update(a, b, c, mask, noise, 1.5, 0.02, 0.5, 0.1),
                                    tuple(ins))


def _euler_dy_closed_form(a, g_x, g_n, alpha, eps, dt, m):
    """dL/da of the kernel: g = dt m g_x + g_n dx/|dx|; kappa (g / (1 + u) -
    (a.g) a / (u (1 + u)^2)), both a-terms zero at a = 0."""
    kappa = alpha * eps
    u = np.linalg.norm(a)
    dx = kappa * a / (1 + u)
    dn = np.linalg.norm(dx)
    g = dt * m * g_x + (g_n * dx / dn if dn > 0 else 0.0)
    b = np.dot(a, g) / (u * (1 + u) ** 2) if u > 0 else 0.0
    return kappa * (g / (1 + u) - b * a)


def test_euler_update_gradient_closed_form():
    rng = np.random.default_rng(4)
    for D in (2, 3):
        for a in (rng.standard_normal(D) * 3, rng.standard_normal(D) * 1e-3, np.zeros(D)):
            g_x, g_n, m = rng.standard_normal(D), rng.standard_normal(), 1.0
            y = torch.tensor(np.concatenate([a, [0.7]]), requires_grad=True)
            xb = torch.zeros(1, 1, 4 if D == 3 else 2, dtype=torch.float64)
            x, s, dn = P.euler_update(y[None, None], xb, torch.zeros(1, 1, 1, dtype=torch.float64), None, None, 1.3,
                                      0.05, dt=0.8)
            gx = np.zeros(xb.shape[-1])
            gx[:D] = g_x
            ((x * torch.tensor(gx)).sum() + dn.sum() * g_n).backward()
            assert np.allclose(y.grad.numpy()[:D], _euler_dy_closed_form(a, g_x, g_n, 1.3, 0.05, 0.8, m),
                               rtol=1e-12, atol=1e-15)
