"""Edge cases of the full path on the GPU: clouds with no particles run every
stage (binning, the neighbour list, forward and backward of every operator)
and return empty or zero outputs, as the reference's kernels launch nothing
for them."""
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
