"""Dense all-pairs torch restatement of ``sphops/torch_sph.py`` (oracle only).

Two roles:
* float64 with autograd: pins the explicit gather-form backward of
  ``oracle.sph`` (``torch.autograd`` is the arbiter of what the derivative is);
* float32 on the host cores: the timed CPU baseline ("port" of the
  reference's CPU torch path, ``torch_sph.py:185-471``), run row-chunked.

Pair displacements are ``r = x_j - x_i`` (``torch_sph.py:25-53``).  A caller
may inject exact fp32 displacement values and a pair mask (the reference
grid's pair set), keeping ``dr/dx`` the identity.
"""
import math

import torch


def pairwise_displacement(x, periodic=False, box=None):
    """``torch_sph._pairwise_displacement``: (B,N,D) -> (B,N,N,D), ``x_j - x_i``,
    wrapped to ``[-L/2, L/2)`` per axis when periodic."""
    r = x.unsqueeze(1) - x.unsqueeze(2)
    if periodic:
        L = torch.as_tensor(box, dtype=x.dtype, device=x.device)
        r = torch.remainder(r + 0.5 * L, L) - 0.5 * L
    return r


def poly6_coef(h, dim):
    return 4.0 / (math.pi * h ** 8) if dim == 2 else 315.0 / (64.0 * math.pi * h ** 9)


def spiky_coef(h, dim):
    return 10.0 / (math.pi * h ** 5) if dim == 2 else 15.0 / (math.pi * h ** 6)


def poly6(r, h, mask):
    d2 = (r * r).sum(-1)
    return torch.where(mask, torch.clamp(h * h - d2, min=0.0) ** 3, torch.zeros_like(d2))


def spiky(r, h, mask):
    d2 = (r * r).sum(-1, keepdim=True)
    inside = mask.unsqueeze(-1) & (d2 > 0) & (d2 < h * h)
    d = torch.sqrt(torch.where(inside, d2, torch.ones_like(d2)))
    mag = torch.where(inside, 3.0 * torch.clamp(h - d, min=0.0) ** 2 / d, torch.zeros_like(d))
    return mag * r


class Pairs:
    """Displacements and mask for one batch of clouds.  ``r`` may be given
    exact values ``r_val`` while keeping autograd's identity Jacobian."""

    def __init__(self, x, h, periodic=False, box=None, r_val=None, mask=None):
        r = pairwise_displacement(x, periodic, box)
        if r_val is not None:
            r = r + (r_val.to(r.dtype) - r).detach()
        self.r = r
        self.mask = mask if mask is not None else ((r * r).sum(-1) < h * h)
        self.h = h


def density(P, m, c6):
    return c6 * (poly6(P.r, P.h, P.mask) * m.unsqueeze(1)).sum(2)


def count(P):
    return P.mask.to(P.r.dtype).sum(2)


def blur(P, m, rho, s, c6):
    v = m / rho
    w = poly6(P.r, P.h, P.mask) * v.unsqueeze(1)
    return c6 * torch.einsum("bij,bjf->bif", w, s)


def gradient(P, m, rho, s, cs):
    v = m / rho
    K = spiky(P.r, P.h, P.mask) * v.unsqueeze(1).unsqueeze(-1)
    dA = s.unsqueeze(1) - s.unsqueeze(2)
    return cs * (dA.unsqueeze(-1) * K.unsqueeze(3)).sum(2)


def density_gradient(P, m, cs):
    return cs * (spiky(P.r, P.h, P.mask) * m.unsqueeze(1).unsqueeze(-1)).sum(2)


def moment_matrix(P, m, rho, cs):
    v = m / rho
    K = spiky(P.r, P.h, P.mask) * v.unsqueeze(1).unsqueeze(-1)
    return cs * (P.r.unsqueeze(-1) * K.unsqueeze(-2)).sum(2)


def safe_inv_sym(M, tol):
    det = torch.linalg.det(M)
    inv = torch.linalg.inv(torch.where((det.abs() < tol)[..., None, None],
                                       torch.eye(M.shape[-1], dtype=M.dtype), M))
    return torch.where((det.abs() < tol)[..., None, None], torch.eye(M.shape[-1], dtype=M.dtype), inv)


def gradient_hybrid(P, m, rho, s, cs, tol=1e-3):
    """``sph.gradient_hybrid``: forward ``raw @ L``, straight-through backward."""
    with torch.no_grad():
        L = safe_inv_sym(moment_matrix(P, m, rho, cs), tol)
    raw = gradient(P, m, rho, s, cs)
    return raw + (raw @ L - raw).detach()


# ------------------------------------------------------------- CPU baseline

def _rows(x, a, rb, periodic, box):
    """Displacements x_j - x_i for rows i in [a, a+rb) against all j."""
    r = x.unsqueeze(1) - x[:, a:a + rb].unsqueeze(2)
    if periodic:
        L = torch.as_tensor(box, dtype=x.dtype)
        r = torch.remainder(r + 0.5 * L, L) - 0.5 * L
    return r


def row_block_step(x, s, h, a, rows, periodic=False, box=None, tol=1e-3, seed=7):
    """One row block of the perception fwd+bwd step on the host, in the
    reference's brute-force form (``torch_sph.py:185-471``): for rows
    ``[a, a+rows)`` against all N columns, pass A (density, density
    gradient), pass B (blur, moment matrix, safe inverse, gradient_hybrid) and
    the backward of ``sum(out * g)`` for seeded upstream ``g`` into x, s and
    rho (through the density rows too).  The full step is the sum of N/rows
    such blocks; each costs the same because every block spans all columns.
    Returns the number of in-radius pairs of the block."""
    B, N, D = x.shape
    C = s.shape[-1]
    rows = min(rows, N - a)
    c6, cs = poly6_coef(h, D), spiky_coef(h, D)
    gen = torch.Generator().manual_seed(seed)
    g_blur = torch.randn(B, rows, C, generator=gen, dtype=x.dtype)
    g_grad = torch.randn(B, rows, C, D, generator=gen, dtype=x.dtype)
    g_dg = torch.randn(B, rows, D, generator=gen, dtype=x.dtype)
    xr = x.detach().requires_grad_(True)
    sr = s.detach().requires_grad_(True)
    m = torch.ones(B, N, dtype=x.dtype)
    rho = torch.full((B, N), float(c6 * h ** (2 * D + 2)), dtype=x.dtype, requires_grad=True)
    r = _rows(xr, a, rows, periodic, box)
    mask = (r.detach() ** 2).sum(-1) < h * h
    W = poly6(r, h, mask)
    rho_rows = c6 * (W * m.unsqueeze(1)).sum(2)
    K = spiky(r, h, mask)
    vj = (m / rho).unsqueeze(1)
    blur_o = c6 * torch.einsum("bij,bjf->bif", W * vj, sr)
    dA = sr.unsqueeze(1) - sr[:, a:a + rows].unsqueeze(2)
    Kv = K * vj.unsqueeze(-1)
    raw = cs * (dA.unsqueeze(-1) * Kv.unsqueeze(3)).sum(2)
    with torch.no_grad():
        M = cs * (r.unsqueeze(-1) * Kv.unsqueeze(-2)).sum(2)
        L = safe_inv_sym(M, tol)
    gh = raw + (raw @ L - raw).detach()
    dg = cs * (K * m.unsqueeze(1).unsqueeze(-1)).sum(2)
    loss = (blur_o * g_blur).sum() + (gh * g_grad).sum() + (dg * g_dg).sum()
    loss.backward(retain_graph=True)
    (rho_rows * rho.grad[:, a:a + rows]).sum().backward()
    return int(mask.sum())
