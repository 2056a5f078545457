"""float64 SPH perception operators on reference pair sets (oracle only).

Forward sums restate ``sphops/torch_sph.py:96-471`` (poly6 ``W = (h^2-|r|^2)^3``,
spiky ``K = 3 (h-|r|)^2 / |r| * r``) with the reference's fp32 coefficients
(``sphops/sph_cuda.cu:1862-1878``).  Backward sums are the reference's gather
formulas (``sphops/sph_cuda.cu:414-721`` particle mode; ``:1160-1375`` grid
mode), evaluated in float64 and pinned against torch.autograd of
``oracle.bruteforce``.

Every function returns ``(value, mag)``: ``mag`` is the same sum over absolute
pair terms, the scale against which fp32 summation error is judged.

Arrays are flat over binned particles: ``x`` (B*N, P), ``s`` (B*N, C),
``m``/``rho`` (B*N,).  Results are per query (``pairs.queries``).
"""
import numpy as np


def _seg_sum(vals, pairs):
    """Sum pair values per query (pairs are grouped by query)."""
    Q = pairs.queries.shape[0]
    out = np.zeros((Q,) + vals.shape[1:], dtype=np.float64)
    if vals.shape[0]:
        np.add.at(out, pairs.q, vals)
    return out


def _kernels(r, h):
    """poly6 value, spiky vector K(r), poly6 gradient and spiky Jacobian
    dK/dr = a I - b r r^T at float64 ``r``, plus the Jacobian's elementary
    magnitude |a| I + |b| |r| |r|^T: for |r| << h the two terms of a diagonal
    element are ~3 h^2 / |r| each and cancel to ~6 h, so fp32 rounding scales
    with them, not with the cancelled |J|."""
    r = np.asarray(r, dtype=np.float64)
    d2 = np.sum(r * r, axis=-1)
    d = np.sqrt(d2)
    h2 = h * h
    W = np.maximum(0.0, h2 - d2) ** 3
    inside = (d > 0) & (d < h)
    ds = np.where(inside, d, 1.0)
    mag = np.where(inside, 3.0 * (h - ds) ** 2 / ds, 0.0)
    K = mag[:, None] * r
    gW = np.where((d2 > 0) & (d2 < h2), -6.0 * np.maximum(0.0, h2 - d2) ** 2, 0.0)[:, None] * r
    D = r.shape[-1]
    eye = np.eye(D)[None]
    a = np.where(inside, 3.0 * (h - ds) ** 2 / ds, 0.0)[:, None, None]
    b = np.where(inside, 3.0 * (h2 - ds * ds) / ds ** 3, 0.0)[:, None, None]
    J = a * eye - b * (r[:, :, None] * r[:, None, :])
    Jmag = np.abs(a) * eye + np.abs(b) * (np.abs(r)[:, :, None] * np.abs(r)[:, None, :])
    return W, K, gW, J, Jmag


class Context:
    """Pair set plus per-pair kernel values for one grid snapshot."""

    def __init__(self, pairs, spec):
        self.p = pairs
        self.spec = spec
        self.h = float(np.float32(spec.eps))
        self.c6, self.cs = spec.coefficients()
        self.W, self.K, _, _, _ = _kernels(pairs.r, self.h)
        self.Wb, self.Kb, self.gWb, self.Jb, self.Jb_mag = _kernels(pairs.rb, self.h)


def count(ctx):
    v = _seg_sum(np.ones(ctx.p.i.shape[0]), ctx.p)
    return v, v


def density(ctx, m):
    t = ctx.c6 * m[ctx.p.j] * ctx.W
    return _seg_sum(t, ctx.p), _seg_sum(np.abs(t), ctx.p)


def blur(ctx, m, rho, s):
    v = (m / rho)[ctx.p.j]
    t = ctx.c6 * (v * ctx.W)[:, None] * s[ctx.p.j]
    return _seg_sum(t, ctx.p), _seg_sum(np.abs(t), ctx.p)


def gradient(ctx, m, rho, s):
    v = (m / rho)[ctx.p.j]
    ds = s[ctx.p.j] - s[ctx.p.i]
    t = ctx.cs * v[:, None, None] * ds[:, :, None] * ctx.K[:, None, :]
    return _seg_sum(t, ctx.p), _seg_sum(np.abs(t), ctx.p)


def density_gradient(ctx, m):
    t = ctx.cs * m[ctx.p.j][:, None] * ctx.K
    return _seg_sum(t, ctx.p), _seg_sum(np.abs(t), ctx.p)


def moment_matrix(ctx, m, rho):
    v = (m / rho)[ctx.p.j]
    r = np.asarray(ctx.p.r, dtype=np.float64)
    t = ctx.cs * v[:, None, None] * r[:, :, None] * ctx.K[:, None, :]
    return _seg_sum(t, ctx.p), _seg_sum(np.abs(t), ctx.p)


def safe_inv_sym(M, tol):
    """Adjugate inverse of symmetric 2x2/3x3 matrices; identity where
    ``|det| < tol`` (``sphops/sph_cuda.cu:3095-3179``).  Returns (inv, det)."""
    M = np.asarray(M, dtype=np.float64)
    D = M.shape[-1]
    if D == 2:
        a, b, d = M[..., 0, 0], M[..., 0, 1], M[..., 1, 1]
        det = a * d - b * b
        adj = np.stack([np.stack([d, -b], -1), np.stack([-b, a], -1)], -2)
    else:
        a, b, c = M[..., 0, 0], M[..., 0, 1], M[..., 0, 2]
        d, e, f = M[..., 1, 1], M[..., 1, 2], M[..., 2, 2]
        t1, t2, t3 = d * f - e * e, c * e - b * f, b * e - c * d
        det = a * t1 + b * t2 + c * t3
        r0 = np.stack([t1, t2, t3], -1)
        r1 = np.stack([t2, a * f - c * c, b * c - a * e], -1)
        r2 = np.stack([t3, b * c - a * e, a * d - b * b], -1)
        adj = np.stack([r0, r1, r2], -2)
    small = np.abs(det) < tol
    safe = np.where(small, 1.0, det)
    inv = adj / safe[..., None, None]
    inv = np.where(small[..., None, None], np.eye(D), inv)
    return inv, det


def gradient_hybrid(ctx, m, rho, s, tol=1e-3):
    """Forward value of ``gradient_hybrid`` (``sphops/sph.py:474-484``):
    ``raw @ safe_inv(M)``.  Returns (out, raw, raw_mag, M, M_mag, L, det)."""
    raw, raw_mag = gradient(ctx, m, rho, s)
    M, M_mag = moment_matrix(ctx, m, rho)
    L, det = safe_inv_sym(M, tol)
    return raw @ L, raw, raw_mag, M, M_mag, L, det


# ---------------------------------------------------------------- backward
#
# ``mag`` of a backward output sums the absolute values of the elementary
# products (pair x channel x component) the value is accumulated from, so it
# bounds the fp32 rounding of sums that cancel inside a pair as well as
# across pairs.

def density_backward(ctx, m, g):
    """dL/dx for upstream ``g`` = dL/drho (``sph_cuda.cu:1160-1184``)."""
    p = ctx.p
    coef = g[p.i] * m[p.j] + g[p.j] * m[p.i]
    acoef = np.abs(g[p.i] * m[p.j]) + np.abs(g[p.j] * m[p.i])
    t = ctx.c6 * coef[:, None] * ctx.gWb
    return _seg_sum(t, p), _seg_sum(ctx.c6 * acoef[:, None] * np.abs(ctx.gWb), p)


def blur_backward(ctx, m, rho, s, g):
    """(dx, ds, drho) for upstream ``g`` = dL/dblur (``sph_cuda.cu:1185-1235``)."""
    p = ctx.p
    v = m / rho
    vi, vj = v[p.i], v[p.j]
    W = ctx.Wb
    mr2 = m[p.i] / rho[p.i] ** 2
    t_s = ctx.c6 * (vi * W)[:, None] * g[p.j]
    B = np.sum(g[p.j] * s[p.i], axis=1)
    A = np.sum(g[p.i] * s[p.j], axis=1)
    aB = np.sum(np.abs(g[p.j] * s[p.i]), axis=1)
    aA = np.sum(np.abs(g[p.i] * s[p.j]), axis=1)
    t_r = -ctx.c6 * mr2 * W * B
    t_x = ctx.c6 * (A * vj + B * vi)[:, None] * ctx.gWb
    m_r = ctx.c6 * mr2 * np.abs(W) * aB
    m_x = ctx.c6 * (aA * np.abs(vj) + aB * np.abs(vi))[:, None] * np.abs(ctx.gWb)
    return [(_seg_sum(t_x, p), _seg_sum(m_x, p)), (_seg_sum(t_s, p), _seg_sum(np.abs(t_s), p)),
            (_seg_sum(t_r, p), _seg_sum(m_r, p))]


def gradient_backward(ctx, m, rho, s, g):
    """(dx, ds, drho) for upstream ``g`` (B*N, C, D) = dL/dgrad
    (``sph_cuda.cu:1265-1327``)."""
    p = ctx.p
    v = m / rho
    vi, vj = v[p.i], v[p.j]
    w = ctx.Kb
    gi, gj = g[p.i], g[p.j]
    mr2 = m[p.i] / rho[p.i] ** 2
    c = gj * vi[:, None, None] + gi * vj[:, None, None]
    ac = np.abs(gj * vi[:, None, None]) + np.abs(gi * vj[:, None, None])
    t_s = ctx.cs * np.sum(c * w[:, None, :], axis=2)
    m_s = ctx.cs * np.sum(ac * np.abs(w)[:, None, :], axis=2)
    delta = s[p.i] - s[p.j]
    t_r = -ctx.cs * mr2 * np.sum(gj * delta[:, :, None] * w[:, None, :], axis=(1, 2))
    m_r = ctx.cs * mr2 * np.sum(np.abs(gj * delta[:, :, None] * w[:, None, :]), axis=(1, 2))
    u = np.sum(delta[:, :, None] * c, axis=1)
    au = np.sum(np.abs(delta)[:, :, None] * ac, axis=1)
    t_x = ctx.cs * np.einsum("pab,pb->pa", ctx.Jb, u)
    m_x = ctx.cs * np.einsum("pab,pb->pa", ctx.Jb_mag, au)
    return [(_seg_sum(t_x, p), _seg_sum(m_x, p)), (_seg_sum(t_s, p), _seg_sum(m_s, p)),
            (_seg_sum(t_r, p), _seg_sum(m_r, p))]


def density_gradient_backward(ctx, m, g):
    """dL/dx for upstream ``g`` (B*N, D) = dL/d(grad rho) (``sph_cuda.cu:1236-1264``)."""
    p = ctx.p
    diff = g[p.j] * m[p.i][:, None] - g[p.i] * m[p.j][:, None]
    adiff = np.abs(g[p.j] * m[p.i][:, None]) + np.abs(g[p.i] * m[p.j][:, None])
    t = ctx.cs * np.einsum("pab,pb->pa", ctx.Jb, diff)
    mt = ctx.cs * np.einsum("pab,pb->pa", ctx.Jb_mag, adiff)
    return _seg_sum(t, p), _seg_sum(mt, p)


def moment_matrix_backward(ctx, m, rho, g):
    """(dx, drho) for upstream ``g`` (B*N, D, D) = dL/dM (``sph_cuda.cu:1328-1375``)."""
    p = ctx.p
    v = m / rho
    vi, vj = v[p.i], v[p.j]
    r = np.asarray(p.rb, dtype=np.float64)
    w = ctx.Kb
    gi, gj = g[p.i], g[p.j]
    mr2 = m[p.i] / rho[p.i] ** 2
    c = gi * vj[:, None, None] + gj * vi[:, None, None]
    ac = np.abs(gi * vj[:, None, None]) + np.abs(gj * vi[:, None, None])
    t_r = -ctx.cs * mr2 * np.einsum("pab,pa,pb->p", gj, r, w)
    m_r = ctx.cs * mr2 * np.einsum("pab,pa,pb->p", np.abs(gj), np.abs(r), np.abs(w))
    direct = np.einsum("pab,pb->pa", c, w)
    a_direct = np.einsum("pab,pb->pa", ac, np.abs(w))
    via_j = np.einsum("pcb,pab->pc", ctx.Jb, r[:, :, None] * c)
    a_via = np.einsum("pcb,pab->pc", ctx.Jb_mag, np.abs(r)[:, :, None] * ac)
    t_x = ctx.cs * (direct + via_j)
    m_x = ctx.cs * (a_direct + a_via)
    return [(_seg_sum(t_x, p), _seg_sum(m_x, p)), (_seg_sum(t_r, p), _seg_sum(m_r, p))]
