"""A whole perception step (instantiate, bin, density, blur, gradient_hybrid,
density_gradient, full backward) captured in a HIP graph with
torch.cuda.graph, in the grid's capture mode (neighbour lists with a fixed
capacity and device-side wave counts): every replay, on new positions and
states, gives bit-for-bit the eager step's outputs and gradients."""
import numpy as np
import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu


def _step(sp, grid, x, s, ups):
    xr = x.detach().requires_grad_(True)
    sr = s.detach().requires_grad_(True)
    with torch.no_grad():
        snap = grid.instantiate(xr)
    xb, sb = sp.bin_particles(xr, sr, snap)
    rho = sp.density(xb, snap)
    outs = [sp.blur(xb, rho, sb, snap), sp.gradient_hybrid(xb, rho, sb, snap), sp.density_gradient(xb, snap)]
    torch.autograd.backward(outs, ups)
    return outs + [rho, xr.grad, sr.grad]


@pytest.mark.parametrize("dim,periodic,mode", [(2, True, "grid"), (3, False, "grid"), (3, False, "particle")])
def test_captured_step_replays_match_eager(dim, periodic, mode):
    import npa_amd.sphops as sp
    B, N, C = 2, 3000, 16
    cases = [H.random_case(f"graph{dim}d", B, N, C, dim, 16, 0.06, periodic, mode, uniform=True, sigma=0.45,
                           seed=seed) for seed in (1, 2, 3, 4)]
    c0 = cases[0]
    grid = sp.HashGrid(dim=dim, boundary="periodic" if periodic else "clamped", mode=mode,
                       grid_size=list(c0.grid_size), eps=c0.eps, num_particles=N, batch_size=B,
                       max_particles_per_block=c0.maxp)
    gen = torch.Generator(device="cuda").manual_seed(0)
    P = c0.x.shape[-1]
    ups = [torch.randn(B, N, C, device="cuda", generator=gen), torch.randn(B, N, C, dim, device="cuda", generator=gen),
           torch.randn(B, N, dim, device="cuda", generator=gen)]
    xs = [torch.from_numpy(c.x).cuda() for c in cases]
    ss = [torch.from_numpy(c.s).cuda() for c in cases]
    # the first step teaches the grid which operators pair up (later snapshots
    # run them fused, which rounds differently), so it is not a reference
    _step(sp, grid, xs[0], ss[0], ups)
    eager = [[t.clone() for t in _step(sp, grid, x, s, ups)] for x, s in zip(xs, ss)]
    cap = 2 * grid.list_capacity_hint()
    assert cap > 0
    grid.set_capture_capacity(cap)
    static_x, static_s = xs[0].clone(), ss[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(sp, grid, static_x, static_s, ups)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(sp, grid, static_x, static_s, ups)
    names = ["blur", "gradient_hybrid", "density_gradient", "rho", "dL/dx", "dL/ds"]
    for k in (1, 2, 3, 1):
        static_x.copy_(xs[k])
        static_s.copy_(ss[k])
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(names, outs, eager[k]):
            assert torch.equal(got, ref), f"replay on case {k}: {name} differs"
        # eager work between replays, as a caller would do
        again = _step(sp, grid, xs[0], ss[0], ups)
        torch.cuda.synchronize()
        assert torch.equal(again[0], eager[0][0])
    assert not grid.list_overflow()
    grid.set_capture_capacity(0)
