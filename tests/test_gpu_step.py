"""Fused Euler update (npa_amd.step) against the oracle restatement of
NPA.forward's position-step scaling and step_euler's update
(oracle/perceive.py, float64 on the CPU); step_euler / step_euler_trace end to
end against the same step assembled from the sphops operators and torch ops."""
import numpy as np
import pytest
import torch

import helpers as H
from oracle import perceive as P

pytestmark = pytest.mark.gpu


def _close(name, got, ref, rtol=1e-5, atol=1e-6):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    err = np.abs(got - ref)
    bad = err > rtol * np.abs(ref) + atol * (rms + 1.0)
    assert not bad.any(), f"{name}: {bad.sum()} of {bad.size} off, max err {err.max():.3g}"


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("noisy", [False, True])
@pytest.mark.parametrize("C", [3, 16])
def test_euler_update_matches_oracle(dim, masked, noisy, C):
    from npa_amd.step import EulerUpdate
    g = torch.Generator().manual_seed(dim * 100 + C + 10 * masked + noisy)
    B, N, Pw = 2, 333, (2 if dim == 2 else 4)
    y = torch.randn(B, N, dim + C, generator=g)
    y[0, :5, :dim] = 0.0  # a = 0: the norm's zero-gradient branch
    xb, sb = torch.randn(B, N, Pw, generator=g), torch.randn(B, N, C, generator=g)
    mask = (torch.rand(B, N, 1, generator=g) < 0.5).float() if masked else None
    noise = torch.randn(B, N, Pw, generator=g) if noisy else None
    alpha, eps, dt, ns = 1.25, 0.03, 0.5, 0.2
    ins = [t.cuda().requires_grad_(True) for t in (y, xb, sb)]
    x, s, dn = EulerUpdate.apply(*ins, None if mask is None else mask.cuda(), None if noise is None else noise.cuda(),
                                 dim, alpha, eps, dt, ns)
    rin = [t.double().requires_grad_(True) for t in (y, xb, sb)]
    rx, rs, rdn = P.euler_update(*rin, None if mask is None else mask.double(),
                                 None if noise is None else noise.double(), alpha, eps, dt, ns)
    for nm, a, b in (("x", x, rx), ("s", s, rs), ("|dx|", dn, rdn)):
        _close(nm, a.detach().cpu(), b.detach())
    ups = [torch.randn(t.shape, generator=g) for t in (rx, rs, rdn)]
    got = torch.autograd.grad((x, s, dn), ins, [u.cuda() for u in ups])
    ref = torch.autograd.grad((rx, rs, rdn), rin, [u.double() for u in ups])
    for nm, a, b in zip(("dL/dy", "dL/dx_bin", "dL/ds_bin"), got, ref):
        _close(nm, a.cpu(), b)
    # only the position output used (no stats, state unused): NULL upstreams
    x, s, dn = EulerUpdate.apply(*ins, None, None, dim, alpha, eps, dt, 0.0)
    rx, _, _ = P.euler_update(*rin, None, None, alpha, eps, dt, 0.0)
    (gy,) = torch.autograd.grad(x, ins[0], ups[0].cuda())
    (ry,) = torch.autograd.grad(rx, rin[0], ups[0].double())
    _close("dL/dy (x only)", gy.cpu(), ry)


class _Model(torch.nn.Module):
    """The attributes of the reference's NPA (models/npa.py:15-63) that
    perception and step_euler read, with its MLP shape."""

    def __init__(self, D, C, hidden=32, **flags):
        super().__init__()
        self.spatial_dims, self.state_dims = D, C
        self.register_buffer("eps0", torch.tensor([0.1]))
        self.register_buffer("alpha", torch.tensor([1.0]))
        f = dict(state_grad=True, density_grad=True, log_norm_grad=True, log_norm_density_grad=True,
                 stopgrad_pos=True, stopgrad_state=False)
        f.update(flags)
        for k, v in f.items():
            setattr(self, k, v)
        width = 2 * C + (C * D if self.state_grad else 0) + (D if self.density_grad else 0)
        self.model = torch.nn.Sequential(torch.nn.Linear(width, hidden), torch.nn.ReLU(),
                                         torch.nn.Linear(hidden, D + C, bias=False))


def _reference_step(model, x, s, grid, dt, update_prob, noise_std):
    """step_euler assembled as the reference assembles it, from the sphops
    operators and torch ops (fp32 on the GPU)."""
    import npa_amd.sphops as sp
    B, N, C = s.shape
    with torch.no_grad():
        snap = grid.instantiate(x)
    xb, sb = sp.bin_particles(x, s, snap)
    xp = xb.detach()
    rho = sp.density(xp, snap)
    z = P.features(sb, sp.blur(xp, rho, sb, snap), sp.gradient_hybrid(xp, rho, sb, snap),
                   sp.density_gradient(xp, snap), grid.eps, 0.1)
    y = model.model(z)
    mask = (torch.rand(B, N, 1, device=x.device) < update_prob).float() if update_prob < 1.0 else None
    noise = torch.randn_like(x) if noise_std > 0 else None
    xn, sn, dn = P.euler_update(y, xb, sb, mask, noise, 1.0, grid.eps, dt, noise_std)
    return xn, sn, dn, snap


@pytest.mark.parametrize("dim", [2, 3])
def test_step_euler_end_to_end(dim):
    import npa_amd.sphops as sp
    from npa_amd import step as S
    C = 8
    c = H.random_case(f"step{dim}d", 2, 400, C, dim, 12, 0.15, False, "grid", uniform=False, sigma=0.3, seed=3)
    grid = sp.HashGrid(dim=dim, boundary="clamped", mode="grid", grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=c.N, batch_size=c.B, max_particles_per_block=c.maxp)
    torch.manual_seed(0)
    model = _Model(dim, C).cuda()
    x0, s0 = torch.from_numpy(c.x).cuda(), torch.from_numpy(c.s).cuda()
    results = []
    for fused in (True, False):
        s = s0.clone().requires_grad_(True)
        x = x0.clone()
        model.zero_grad()
        torch.manual_seed(123)
        total = 0.0
        for _ in range(2):
            if fused:
                x, s, stats = S.step_euler(model, x, s, grid, dt=1.0, update_prob=0.5, intermediate=True,
                                           noise_std=0.01)
                total = total + stats["dx_norm"]
            else:
                x, s, dn, _ = _reference_step(model, x, s, grid, 1.0, 0.5, 0.01)
                total = total + dn.mean()
        loss = (s ** 2).mean() + (x ** 2).mean() + total
        loss.backward()
        results.append((x.detach().cpu(), s.detach().cpu(), float(total.detach()),
                        [p.grad.detach().cpu().clone() for p in model.model.parameters()]))
    (xf, sf, tf, gf), (xr, sr, tr, gr) = results
    _close("x", xf, xr, rtol=1e-4, atol=1e-5)
    _close("s", sf, sr, rtol=1e-4, atol=1e-5)
    assert abs(tf - tr) <= 1e-4 * abs(tr)
    for i, (a, b) in enumerate(zip(gf, gr)):
        _close(f"MLP grad {i}", a, b, rtol=1e-3, atol=1e-4)


def test_step_euler_trace_order():
    """step_euler_trace returns particles in the input order: unbinning the
    binned update with the step's snapshot."""
    import npa_amd.sphops as sp
    from npa_amd import step as S
    C, dim = 8, 3
    c = H.random_case("trace3d", 1, 300, C, dim, 10, 0.2, False, "grid", uniform=False, sigma=0.3, seed=5)
    grid = sp.HashGrid(dim=dim, boundary="clamped", mode="grid", grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=c.N, batch_size=c.B, max_particles_per_block=c.maxp)
    torch.manual_seed(0)
    model = _Model(dim, C).cuda()
    x, s = torch.from_numpy(c.x).cuda(), torch.from_numpy(c.s).cuda()
    torch.manual_seed(9)
    xb, sb, _ = S.step_euler(model, x, s, grid, update_prob=1.0)
    torch.manual_seed(9)
    xt, st, dxt, dst = S.step_euler_trace(model, x, s, grid, update_prob=1.0, return_aux=True)
    perm = model.last_snapshot.permutation.long()
    assert torch.equal(xt, xb[0][perm[0]][None]) and torch.equal(st, sb[0][perm[0]][None])
    _close("x = x0 + dx", xt.cpu(), (x + dxt).cpu())
    _close("s = s0 + ds", st.cpu(), (s + dst).cpu())


def test_step_euler_static_matches_torch_assembly():
    """The state-only model's step (models/static_npa.py:24-38) with fused
    perception against the same step over the torch feature assembly."""
    import npa_amd.sphops as sp
    from npa_amd import step as S
    C, dim = 8, 2
    c = H.random_case("static2d", 2, 400, C, dim, 12, 0.15, False, "grid", uniform=False, sigma=0.3, seed=6)
    grid = sp.HashGrid(dim=dim, boundary="clamped", mode="grid", grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=c.N, batch_size=c.B, max_particles_per_block=c.maxp)
    torch.manual_seed(0)
    model = _Model(dim, C).cuda()
    model.model[2] = torch.nn.Linear(32, C, bias=False).cuda()  # ds only
    x, s0 = torch.from_numpy(c.x).cuda(), torch.from_numpy(c.s).cuda()
    cmask = (torch.arange(C, device="cuda") % 2).float()
    out = []
    for fused in (True, False):
        s = s0.clone().requires_grad_(True)
        model.zero_grad()
        torch.manual_seed(4)
        if fused:
            xn, sn = S.step_euler_static(model, x, s, grid, dt=0.5, update_prob=0.5, channel_mask=cmask)
        else:
            with torch.no_grad():
                snap = grid.instantiate(x)
            xb, sb = sp.bin_particles(x, s, snap)
            xp = xb.detach()
            rho = sp.density(xp, snap)
            z = P.features(sb, sp.blur(xp, rho, sb, snap), sp.gradient_hybrid(xp, rho, sb, snap),
                           sp.density_gradient(xp, snap), grid.eps, 0.1)
            ds = model.model(z) * cmask
            m = (torch.rand(2, 400, 1, device="cuda") < 0.5).float()
            xn, sn = xb + 0, sb + 0.5 * ds * m
        (sn ** 2).sum().backward()
        out.append((xn.detach().cpu(), sn.detach().cpu(), s.grad.cpu(), model.model[0].weight.grad.cpu()))
    (xf, sf, gf, wf), (xr, sr, gr, wr) = out
    assert torch.equal(xf, xr)
    _close("s", sf, sr, rtol=1e-4, atol=1e-5)
    _close("dL/ds", gf, gr, rtol=1e-4, atol=1e-5)
    _close("dL/dW", wf, wr, rtol=1e-3, atol=1e-4)
