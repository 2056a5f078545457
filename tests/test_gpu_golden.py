"""The HIP path against the committed golden fixtures (tests/golden/), plus
the two API helpers around binning: wrap_positions and the Permute backward."""
import os

import numpy as np
import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def grid_for(d, dim):
    import npa_amd.sphops as sp
    grid = [int(v) for v in d["grid"]]
    B, N = d["x"].shape[:2]
    boundary = "periodic" if bool(d["periodic"]) else "clamped"
    return sp.HashGrid(dim=dim, boundary=boundary, mode="grid", grid_size=grid, eps=float(d["eps"]),
                       num_particles=N, batch_size=B, max_particles_per_block=64)


@pytest.mark.parametrize("name", ["ref2d_clamped", "ref2d_periodic"])
def test_fixture(name):
    import npa_amd.sphops as sp
    d = np.load(os.path.join(HERE, f"{name}.npz"))
    print(f"[case] golden {name}", flush=True)
    grid = grid_for(d, 2)
    x, s, m = dev(d["x"]), dev(d["s"]), dev(d["m"])
    snap = grid.instantiate(x)
    np.testing.assert_array_equal(snap.permutation.cpu().numpy(), d["permutation"])
    np.testing.assert_array_equal(snap.bin_offsets.cpu().numpy(), d["bin_offsets"])
    np.testing.assert_array_equal(snap.block_info.cpu().numpy(), d["block_info"])
    assert int(snap.total_blocks.item()) == int(d["total_blocks"])
    xb, sb, mb = sp.bin_particles(x, s, snap, m)
    np.testing.assert_array_equal(xb.cpu().numpy(), d["xb"])
    np.testing.assert_array_equal(sb.cpu().numpy(), d["sb"])
    with torch.no_grad():
        np.testing.assert_array_equal(sp.count(xb, snap).cpu().numpy().reshape(-1), d["count"])
        rho = sp.density(xb, snap, mb)
        H.assert_close(f"{name}:rho", rho.cpu().numpy().reshape(-1), d["rho"], d["rho_mag"])
        dg = sp.density_gradient(xb, snap, mb)
        H.assert_close(f"{name}:dgrad", dg.cpu().numpy().reshape(-1, 2), d["dgrad"], d["dgrad_mag"])
        bl = sp.blur(xb, rho, sb, snap, mb)
        H.assert_close(f"{name}:blur", bl.cpu().numpy().reshape(-1, 4), d["blur"], d["blur_mag"])
        gr = sp.gradient(xb, rho, sb, snap, mb)
        H.assert_close(f"{name}:grad", gr.cpu().numpy().reshape(-1, 4, 2), d["grad"], d["grad_mag"])

    def grads(fn, up, need):
        X = xb.detach().clone().requires_grad_("x" in need)
        S = sb.detach().clone().requires_grad_("s" in need)
        R = rho.detach().clone().requires_grad_("rho" in need)
        fn(X, S, R).backward(dev(up))
        return X.grad, S.grad, R.grad

    gx, _, _ = grads(lambda X, S, R: sp.density(X, snap, mb), d["g_rho"], ("x",))
    H.assert_close(f"{name}:density.dx", gx.cpu().numpy().reshape(-1, 2), d["b_density_dx"], d["b_density_dx_mag"])
    gx, _, _ = grads(lambda X, S, R: sp.density_gradient(X, snap, mb), d["g_dg"], ("x",))
    H.assert_close(f"{name}:dgrad.dx", gx.cpu().numpy().reshape(-1, 2), d["b_dgrad_dx"], d["b_dgrad_dx_mag"])
    for key, fn, up in (("b_blur", lambda X, S, R: sp.blur(X, R, S, snap, mb), d["g_blur"]),
                        ("b_grad", lambda X, S, R: sp.gradient(X, R, S, snap, mb), d["g_grad"])):
        gx, gs, gr = grads(fn, up, ("x", "s", "rho"))
        H.assert_close(f"{name}:{key}.dx", gx.cpu().numpy().reshape(-1, 2), d[f"{key}_dx"], d[f"{key}_dx_mag"])
        H.assert_close(f"{name}:{key}.ds", gs.cpu().numpy().reshape(-1, 4), d[f"{key}_ds"], d[f"{key}_ds_mag"])
        H.assert_close(f"{name}:{key}.drho", gr.cpu().numpy().reshape(-1), d[f"{key}_drho"],
                       d[f"{key}_drho_mag"])


def test_pair3d_closed_form():
    import npa_amd.sphops as sp
    d = np.load(os.path.join(HERE, "pair3d.npz"))
    grid = [int(v) for v in d["grid"]]
    g = sp.HashGrid(dim=3, boundary="clamped", mode="grid", grid_size=grid, eps=float(d["h"]), num_particles=2,
                    batch_size=1, max_particles_per_block=64)
    x, m = dev(d["x"]), dev(d["m"])
    snap = g.instantiate(x)
    xb, _, mb = sp.bin_particles(x, torch.zeros(1, 2, 1, device="cuda"), snap, m)
    perm = snap.permutation.cpu().numpy()[0]
    with torch.no_grad():
        rho = sp.density(xb, snap, mb).cpu().numpy()[0][perm]
        dg = sp.density_gradient(xb, snap, mb).cpu().numpy()[0][perm]
    np.testing.assert_allclose(rho, d["rho"], rtol=1e-5)
    np.testing.assert_allclose(dg, d["dgrad"], rtol=1e-5)


@pytest.mark.parametrize("boundary", ["periodic", "clamped"])
def test_wrap_positions(boundary):
    """HashGrid.wrap_positions (sphops/sph.py:107-123) against the oracle:
    each axis wrapped into [-L/2, L/2) with L = grid_size * eps (periodic),
    unchanged (clamped)."""
    import npa_amd.sphops as sp
    from oracle import binning
    grid = sp.HashGrid(dim=3, boundary=boundary, mode="grid", grid_size=[8, 6, 10], eps=0.125, num_particles=500,
                       batch_size=2)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((2, 500, 3)) * 2.0).astype(np.float32)
    out = grid.wrap_positions(dev(x)).cpu().numpy()
    ref = binning.wrap_positions(x, (8, 6, 10), 0.125, boundary == "periodic")
    if boundary == "periodic":
        L = np.array([8, 6, 10]) * 0.125
        diff = np.mod(out.astype(np.float64) - ref + L / 2, L) - L / 2   # equal modulo the box
        assert np.abs(diff).max() < 2e-6
        assert np.all(out >= -L / 2 - 1e-6) and np.all(out <= L / 2 + 1e-6)
    else:
        np.testing.assert_array_equal(out, ref)


@pytest.mark.parametrize("mass_grad", [True, False])
def test_permute_backward_is_a_gather(mass_grad):
    """bin_particles' backward returns upstream[b, perm[b, i]] for x, s and
    mass (sphops/sph.py:148-175), bit for bit; a mass that needs no gradient
    gets none, and its rows are not moved (both mass pointers NULL), while a
    single NULL mass pointer is refused."""
    import ctypes
    import npa_amd.sphops as sp
    from npa_amd.sphops import _native
    c = H.random_case("perm", 2, 300, 5, 3, 8, 0.25, False, "grid", sigma=0.8)
    grid = sp.HashGrid(dim=3, boundary="clamped", mode="grid", grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=c.N, batch_size=c.B)
    x, s = (dev(a).requires_grad_(True) for a in (c.x, c.s))
    m = dev(c.m).requires_grad_(mass_grad)
    snap = grid.instantiate(x.detach())
    xb, sb, mb = sp.bin_particles(x, s, snap, m)
    rng = np.random.default_rng(4)
    ux, us, um = (rng.standard_normal(t.shape).astype(np.float32) for t in (xb, sb, mb))
    loss = (xb * dev(ux)).sum() + (sb * dev(us)).sum()
    if mass_grad:
        loss = loss + (mb * dev(um)).sum()
    loss.backward()
    perm = snap.permutation.cpu().numpy()
    b = np.arange(c.B)[:, None]
    np.testing.assert_array_equal(x.grad.cpu().numpy(), ux[b, perm])
    np.testing.assert_array_equal(s.grad.cpu().numpy(), us[b, perm])
    if mass_grad:
        np.testing.assert_array_equal(m.grad.cpu().numpy(), um[b, perm])
    else:
        assert m.grad is None
        lib, hg = _native.lib, grid.hashgrid
        p = lambda t: ctypes.c_void_p(t.data_ptr())
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        gx, gs, gm = torch.empty_like(xb), torch.empty_like(sb), torch.full_like(mb, 7.0)
        assert lib.sphops_backward_bin_particles(hg._h, p(xb), p(sb), ctypes.c_void_p(), p(snap.permutation), p(gx),
                                                 p(gs), p(gm), 5, st) != 0
        assert b"both or neither" in lib.sphops_last_error()
        assert lib.sphops_backward_bin_particles(hg._h, p(xb), p(sb), ctypes.c_void_p(), p(snap.permutation), p(gx),
                                                 p(gs), ctypes.c_void_p(), 5, st) == 0
        torch.cuda.synchronize()
        assert torch.equal(gx, x.detach()) and torch.equal(gs, s.detach())
        assert bool((gm == 7.0).all())


@pytest.mark.parametrize("dim", [2, 3])
def test_safe_inverse_indefinite(dim):
    """safe_inv_sym_mat (sphops/sph.py:467-471, sph_cuda.cu:3095-3179) on
    symmetric indefinite matrices: det < -tol is inverted, -tol < det < 0
    gives the identity (the |det| < tol branch, sph_cuda.cu:3111, 3152), as
    the oracle does; positive definite ones are covered by the parity cases."""
    import npa_amd.sphops as sp
    from oracle import sph
    mats = H.indefinite_matrices(dim)
    M = np.concatenate([mats["big"], mats["small"]]).astype(np.float32)
    got = sp.safe_inv_sym_mat(dev(M[None]), 1e-3).cpu().numpy()[0]   # (B, N, D, D) as in the reference
    ref, det = sph.safe_inv_sym(M.astype(np.float64), 1e-3)
    n = len(mats["big"])
    assert np.all(det[:n] < -1e-3) and np.all((det[n:] < 0) & (det[n:] > -1e-3))
    np.testing.assert_array_equal(got[n:], np.broadcast_to(np.eye(dim, dtype=np.float32), got[n:].shape))
    scale = np.abs(ref) + np.einsum("qab,qbc,qcd->qad", np.abs(ref), np.abs(M), np.abs(ref))
    H.assert_close(f"safe_inv_indefinite{dim}", got[:n], ref[:n], scale[:n])
