"""Edge cases of the full path on the GPU: clouds with no particles run every
stage (binning, the neighbour list, forward and backward of every operator)
and return empty or zero outputs, as the reference's kernels launch nothing
for them; cell bounds on grids of more than 2^22 cells."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim,boundary,mode", [(2, "periodic", "grid"), (3, "clamped", "grid"),
                                               (3, "clamped", "particle")])
def test_empty_cloud(dim, boundary, mode):
    import npa_amd.sphops as sp
    print(f"[case] empty dim={dim} {boundary} {mode}", flush=True)
    gs = [8] * dim
    grid = sp.HashGrid(dim=dim, boundary=boundary, mode=mode, grid_size=gs, eps=0.25, num_particles=0,
                       batch_size=2, max_particles_per_block=16)
    P = 2 if dim == 2 else 4
    x = torch.zeros(2, 0, P, device="cuda", requires_grad=True)
    s = torch.zeros(2, 0, 16, device="cuda", requires_grad=True)
    snap = grid.instantiate(x.detach())
    assert snap.permutation.shape == (2, 0)
    assert int(snap.bin_offsets.abs().sum().item()) == 0 and snap.bin_offsets.numel() == 2 * 8 ** dim + 1
    xb, sb = sp.bin_particles(x, s, snap)
    rho = sp.density(xb, snap)
    outs = [rho, sp.blur(xb, rho, sb, snap), sp.gradient_hybrid(xb, rho, sb, snap), sp.density_gradient(xb, snap),
            sp.gradient(xb, rho, sb, snap), sp.moment_matrix(xb, rho, snap)]
    assert [tuple(o.shape[:2]) for o in outs] == [(2, 0)] * len(outs)
    loss = sum(o.sum() for o in outs)
    loss.backward()
    torch.cuda.synchronize()
    assert x.grad.shape == x.shape and s.grad.shape == s.shape
    assert int(sp.count(xb.detach(), snap).numel()) == 0


def _binning_case(name, x, grid_size, eps, maxp, B=1):
    import helpers as H
    import numpy as np
    N = x.shape[1]
    return H.Case(name, H.pack_pos(x), np.zeros((B, N, 4), np.float32), np.ones((B, N), np.float32),
                  tuple(grid_size), eps, False, "grid", maxp)


@pytest.mark.parametrize("layout", ["one-cell", "ends", "mixed"])
def test_large_grid_cell_bounds(layout):
    """Above 2^22 cells the permutation and block rows find each cell's
    first and last sorted position by searching the sorted keys instead of
    loading bin_offsets.  Runs that reach the first or the last sorted
    position, a cell holding every particle of a cloud, and single-particle
    cells, on a 2 x 160 x 128 x 128 grid (2 clouds, 5.2 M cells): permutation,
    bin_offsets, block_info and total_blocks bit-exact against the oracle."""
    import numpy as np
    import helpers as H
    import npa_amd.sphops as sp
    rng = np.random.default_rng(23)
    gs, eps, B, N = (160, 128, 128), 0.01, 2, 3000
    half = np.array(gs) * eps / 2
    if layout == "one-cell":
        x = np.broadcast_to(0.0025 + rng.random((1, N, 3)) * 0.005, (B, N, 3)).copy()   # cell (80, 64, 64)
    elif layout == "ends":
        lo = -half + 0.002 + rng.random((N // 2, 3)) * 0.006        # the first cell
        hi = half - 0.008 + rng.random((N - N // 2, 3)) * 0.006     # the last cell
        x = np.stack([np.concatenate([lo, hi]), np.concatenate([hi, lo])])
    else:
        x = np.concatenate([rng.normal(0, 0.02, (B, N // 2, 3)),
                            (rng.random((B, N - N // 2, 3)) - 0.5) * 2 * (half - 1e-3)], axis=1)
    c = _binning_case(f"cells-{layout}", x, gs, eps, 16, B)
    print(f"[case] large-grid cell bounds {layout}", flush=True)
    grid = sp.HashGrid(dim=3, boundary="clamped", mode="grid", grid_size=list(gs), eps=eps, num_particles=N,
                       batch_size=B, max_particles_per_block=16)
    snap = grid.instantiate(torch.from_numpy(c.x).cuda())
    ref = H.oracle_binning(c)
    np.testing.assert_array_equal(snap.permutation.cpu().numpy(), ref["permutation"])
    np.testing.assert_array_equal(snap.bin_offsets.cpu().numpy(), ref["bin_offsets"])
    np.testing.assert_array_equal(snap.block_info.cpu().numpy(), ref["block_info"])
    assert int(snap.total_blocks.item()) == ref["total_blocks"]


def test_large_grid_many_particles():
    """Above 2^22 cells the permutation runs inside the bin_offsets launch,
    one permutation workgroup after every few chunk workgroups; here the
    permutation's workgroups outnumber the chunks' (300,000 particles on
    4.35 M cells), the case where the interleave takes one chunk workgroup per
    permutation workgroup and the launch grows to cover them all: every
    binning output bit-exact against the oracle."""
    import numpy as np
    import helpers as H
    import npa_amd.sphops as sp
    rng = np.random.default_rng(29)
    gs, eps, B, N = (170, 160, 160), 0.01, 1, 300_000
    half = np.array(gs) * eps / 2
    x = (rng.random((B, N, 3)) - 0.5) * 2 * (half - 1e-3)
    c = _binning_case("cells-many", x, gs, eps, 16, B)
    print("[case] large-grid many particles", flush=True)
    grid = sp.HashGrid(dim=3, boundary="clamped", mode="grid", grid_size=list(gs), eps=eps, num_particles=N,
                       batch_size=B, max_particles_per_block=16)
    snap = grid.instantiate(torch.from_numpy(c.x).cuda())
    ref = H.oracle_binning(c)
    np.testing.assert_array_equal(snap.permutation.cpu().numpy(), ref["permutation"])
    np.testing.assert_array_equal(snap.bin_offsets.cpu().numpy(), ref["bin_offsets"])
    np.testing.assert_array_equal(snap.block_info.cpu().numpy(), ref["block_info"])
    assert int(snap.total_blocks.item()) == ref["total_blocks"]
