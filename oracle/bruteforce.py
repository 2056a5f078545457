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

def perception_step_cpu(x, s, h, periodic=False, box=None, row_block=None, full=True, tol=1e-3):
    """One perception fwd+bwd step on the host in the input dtype: pass A
    (rho, grad rho), pass B (blur, moment matrix, safe inverse, gradient_hybrid)
    and the backward of ``sum(out * g)`` for fixed seeded upstream ``g``.

    Rows are processed in blocks of ``row_block`` particles against all
    columns (exact; per-block graphs).  Returns the number of in-radius pairs
    (including self) so throughput can be reported per pair."""
    B, N, D = x.shape
    C = s.shape[-1]
    c6, cs = poly6_coef(h, D), spiky_coef(h, D)
    rb = row_block or N
    gen = torch.Generator().manual_seed(7)
    g_blur = torch.randn(B, N, C, generator=gen, dtype=x.dtype)
    g_grad = torch.randn(B, N, C, D, generator=gen, dtype=x.dtype)
    g_dg = torch.randn(B, N, D, generator=gen, dtype=x.dtype)
    x = x.detach().requires_grad_(full)
    s = s.detach().requires_grad_(True)
    m = torch.ones(B, N, dtype=x.dtype)
    pairs = 0
    with torch.no_grad():
        rho_nd = torch.empty(B, N, dtype=x.dtype)
        for a in range(0, N, rb):
            r = pairwise_displacement(x, periodic, box)[:, a:a + rb] if rb == N else \
                _rows(x, a, rb, periodic, box)
            mask = (r * r).sum(-1) < h * h
            pairs += int(mask.sum())
            rho_nd[:, a:a + rb] = c6 * (poly6(r, h, mask) * m.unsqueeze(1)).sum(2)
    rho = rho_nd.clone().requires_grad_(full)
    drho_total = torch.zeros(B, N, dtype=x.dtype)
    for a in range(0, N, rb):
        r = _rows(x, a, rb, periodic, box)
        mask = (r.detach() ** 2).sum(-1) < h * h
        P = _RowPairs(r, mask, h)
        sl = slice(a, a + rb)
        vj = (m / rho).unsqueeze(1)
        Wm = poly6(P.r, h, mask)
        blur_o = c6 * torch.einsum("bij,bjf->bif", Wm * vj, s)
        K = spiky(P.r, h, mask)
        dA = s.unsqueeze(1) - s[:, sl].unsqueeze(2)
        raw = cs * (dA.unsqueeze(-1) * (K * vj.unsqueeze(-1)).unsqueeze(3)).sum(2)
        with torch.no_grad():
            M = cs * (P.r.unsqueeze(-1) * (K * vj.unsqueeze(-1)).unsqueeze(-2)).sum(2)
            L = safe_inv_sym(M, tol)
        gh = raw + (raw @ L - raw).detach()
        dg = cs * (K * m.unsqueeze(1).unsqueeze(-1)).sum(2)
        loss = (blur_o * g_blur[:, sl]).sum() + (gh * g_grad[:, sl]).sum()
        if full:
            loss = loss + (dg * g_dg[:, sl]).sum()
        loss.backward()
    if full and rho.grad is not None:
        # rho -> x through the density pass (pass A backward)
        for a in range(0, N, rb):
            r = _rows(x, a, rb, periodic, box)
            mask = (r.detach() ** 2).sum(-1) < h * h
            rr = c6 * (poly6(r, h, mask) * m.unsqueeze(1)).sum(2)
            (rr * rho.grad[:, a:a + rb]).sum().backward()
        drho_total += rho.grad
    return pairs


class _RowPairs:
    def __init__(self, r, mask, h):
        self.r, self.mask, self.h = r, mask, h


def _rows(x, a, rb, periodic, box):
    xi = x[:, a:a + rb]
    r = x.unsqueeze(1) - xi.unsqueeze(2)
    if periodic:
        L = torch.as_tensor(box, dtype=x.dtype)
        r = torch.remainder(r + 0.5 * L, L) - 0.5 * L
    return r
