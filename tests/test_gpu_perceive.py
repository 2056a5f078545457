"""Fused perception features (npa_amd.perceive) against the oracle restatement
of NPA.perceive's feature assembly (oracle/perceive.py, float64 on the CPU):
z and the gradients of z with respect to the operator outputs, over the
constructor flags, 2D and 3D; and perceive() end to end."""
import numpy as np
import pytest
import torch

import helpers as H
from oracle import perceive as P

pytestmark = pytest.mark.gpu

FLAGS = [
    dict(),
    dict(log_norm_grad=False),
    dict(log_norm_density_grad=False),
    dict(density_grad=False),
    dict(state_grad=False),
    dict(state_grad=False, density_grad=False),
]


def _close(name, got, ref, rtol=1e-5, atol=1e-6):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    err = np.abs(got - ref)
    bad = err > rtol * np.abs(ref) + atol * (rms + 1.0)
    assert not bad.any(), f"{name}: {bad.sum()} of {bad.size} off, max err {err.max():.3g}"


def _ops(dim, C, seed):
    import npa_amd.sphops as sp
    c = H.random_case(f"perceive{dim}d", 2, 300, C, dim, 10, 0.2, False, "grid", uniform=False, sigma=0.3,
                      seed=seed)
    grid = sp.HashGrid(dim=dim, boundary="clamped", mode="grid", grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=c.N, batch_size=c.B, max_particles_per_block=c.maxp)
    x, s = torch.from_numpy(c.x).cuda(), torch.from_numpy(c.s).cuda()
    snap = grid.instantiate(x)
    xb, sb = sp.bin_particles(x, s, snap)
    rho = sp.density(xb, snap)
    return grid, x, s, sb, sp.blur(xb, rho, sb, snap), sp.gradient_hybrid(xb, rho, sb, snap), \
        sp.density_gradient(xb, snap)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("fi", range(len(FLAGS)))
@pytest.mark.parametrize("C", [5, 16, 64])
def test_features_match_oracle(dim, fi, C):
    """C = 5 and 16 give tiles whose particle count does not divide N; C = 64
    is the widest row (the fewest particles per tile)."""
    from npa_amd import perceive as PF
    f = dict(state_grad=True, density_grad=True, log_norm_grad=True, log_norm_density_grad=True)
    f.update(FLAGS[fi])
    grid, _, _, sb, bl, gs, gr = _ops(dim, C, 100 + fi)
    eps, eps0 = grid.eps, 0.1
    coef = np.float32(np.float32(1.0) / np.float32(eps0)) * np.float32(eps)  # as the oracle and perceive()
    flags = ((PF.STATE_GRAD | (PF.LOG_NORM_GRAD if f["log_norm_grad"] else 0)) if f["state_grad"] else 0) | \
            ((PF.DENSITY_GRAD | (PF.LOG_NORM_DENSITY_GRAD if f["log_norm_density_grad"] else 0))
             if f["density_grad"] else 0)
    ins = [t.detach().clone().requires_grad_(True) for t in (sb, bl, gs, gr)]
    gs_in = ins[2] if f["state_grad"] else None
    gr_in = ins[3] if f["density_grad"] else None
    N = sb.shape[1]
    z = PF.PerceptionFeatures.apply(ins[0], ins[1], gs_in, gr_in, dim, float(coef),
                                    float(np.float32(coef ** np.float32(1 + dim))), float(N), flags)
    ref_in = [t.detach().cpu().double().requires_grad_(True) for t in (sb, bl, gs, gr)]
    zr = P.features(ref_in[0], ref_in[1], ref_in[2] if f["state_grad"] else None,
                    ref_in[3] if f["density_grad"] else None, eps, eps0, f["log_norm_grad"],
                    f["log_norm_density_grad"])
    assert z.shape == zr.shape
    _close("z", z.detach().cpu(), zr.detach())
    dz = torch.randn(z.shape, generator=torch.Generator().manual_seed(fi)).cuda()
    used = [i for i, t in enumerate([ins[0], ins[1], gs_in, gr_in]) if t is not None]
    got = torch.autograd.grad(z, [ins[i] for i in used], dz)
    ref = torch.autograd.grad(zr, [ref_in[i] for i in used], dz.cpu().double())
    for i, g, r in zip(used, got, ref):
        _close(f"grad {i}", g.cpu(), r)


@pytest.mark.parametrize("dim", [2, 3])
def test_perceive_end_to_end(dim):
    """perceive() gives the oracle's z of the separately computed operator
    outputs, and gradients to x (stopgrad_pos off) and s that match the
    reference's torch assembly backpropagated through the same operators."""
    import npa_amd.sphops as sp
    from npa_amd import perceive as PF
    grid, x, s, sb, bl, gs, gr = _ops(dim, 16, 7)
    xg, sg = x.clone().requires_grad_(True), s.clone().requires_grad_(True)
    z, xb, sb2, snap = PF.perceive(xg, sg, grid, eps0=0.1, stopgrad_pos=False)
    zr = P.features(sb.detach().cpu().double(), bl.detach().cpu().double(), gs.detach().cpu().double(),
                    gr.detach().cpu().double(), grid.eps, 0.1)
    # the operators inside perceive() run with position gradients on (another
    # kernel variant), so their fp32 outputs round differently from _ops'
    _close("z", z.detach().cpu(), zr, rtol=1e-4, atol=1e-5)
    dz = torch.randn(z.shape, generator=torch.Generator().manual_seed(1)).cuda()
    gx, gsv = torch.autograd.grad(z, [xg, sg], dz)
    # the same perception with the reference's torch assembly, on the GPU in fp32
    xh, sh = x.clone().requires_grad_(True), s.clone().requires_grad_(True)
    snap2 = grid.instantiate(xh.detach())
    xb2, sb3 = sp.bin_particles(xh, sh, snap2)
    rho = sp.density(xb2, snap2)
    zt = P.features(sb3, sp.blur(xb2, rho, sb3, snap2), sp.gradient_hybrid(xb2, rho, sb3, snap2),
                    sp.density_gradient(xb2, snap2), grid.eps, 0.1)
    hx, hs = torch.autograd.grad(zt, [xh, sh], dz)
    _close("dL/ds", gsv.cpu(), hs.cpu(), rtol=1e-4, atol=1e-5)
    _close("dL/dx", gx.cpu(), hx.cpu(), rtol=1e-4, atol=1e-5)
