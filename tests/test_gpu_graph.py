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


def test_capture_below_the_sizes_still_correct():
    """Capture mode with sizes far below the step's needs: an index buffer of
    64 entries (almost every row is walked on the stencil instead) and pair
    launches sized for a twentieth of the waves (the kernels loop over the
    true device counts).  Replays still give the eager results, within fp32
    summation-order differences, and list_overflow reports the small buffer."""
    import npa_amd.sphops as sp
    B, N, C, dim = 2, 3000, 16, 3
    cases = [H.random_case("graph-small", B, N, C, dim, 16, 0.06, False, "grid", uniform=True, sigma=0.45,
                           seed=seed) for seed in (5, 6)]
    c0 = cases[0]
    grid = sp.HashGrid(dim=dim, boundary="clamped", mode="grid", grid_size=list(c0.grid_size), eps=c0.eps,
                       num_particles=N, batch_size=B, max_particles_per_block=c0.maxp)
    gen = torch.Generator(device="cuda").manual_seed(1)
    ups = [torch.randn(B, N, C, device="cuda", generator=gen), torch.randn(B, N, C, dim, device="cuda", generator=gen),
           torch.randn(B, N, dim, device="cuda", generator=gen)]
    xs = [torch.from_numpy(c.x).cuda() for c in cases]
    ss = [torch.from_numpy(c.s).cuda() for c in cases]
    _step(sp, grid, xs[0], ss[0], ups)
    eager = [[t.clone() for t in _step(sp, grid, x, s, ups)] for x, s in zip(xs, ss)]
    grid.hashgrid.set_capture_capacity(64, wave_margin=0.05)
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
    for k in (1, 0):
        static_x.copy_(xs[k])
        static_s.copy_(ss[k])
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(names, outs, eager[k]):
            err = (got - ref).abs().max().item()
            assert err <= 1e-4 * ref.abs().max().item() + 1e-6, f"replay on case {k}: {name} off by {err}"
    assert grid.list_overflow()
    grid.set_capture_capacity(0)


class _TinyNPA(torch.nn.Module):
    """The NPA attributes step_euler reads (models/npa.py:15-63), small MLP."""

    def __init__(self, D, C):
        super().__init__()
        self.spatial_dims = D
        self.register_buffer("eps0", torch.tensor([0.1]))
        self.register_buffer("alpha", torch.tensor([1.0]))
        self.state_grad = self.density_grad = self.log_norm_grad = self.log_norm_density_grad = True
        self.stopgrad_pos, self.stopgrad_state = True, False
        self.model = torch.nn.Sequential(torch.nn.Linear(2 * C + C * D + D, 32), torch.nn.ReLU(),
                                         torch.nn.Linear(32, D + C, bias=False))


def test_captured_rollout_matches_eager():
    """A 3-step step_euler rollout with its backward (train.py:227-237 without
    the random mask) captured as one graph: replays on new states match the
    eager rollout."""
    import npa_amd.sphops as sp
    from npa_amd import step as S
    B, N, C, D, K = 2, 1500, 8, 2, 3
    cases = [H.random_case("rollout", B, N, C, D, 16, 0.06, False, "grid", uniform=False, sigma=0.3, seed=seed)
             for seed in (11, 12, 13)]
    c0 = cases[0]
    grid = sp.HashGrid(dim=D, boundary="clamped", mode="grid", grid_size=list(c0.grid_size), eps=c0.eps,
                       num_particles=N, batch_size=B, max_particles_per_block=c0.maxp)
    torch.manual_seed(0)
    model = _TinyNPA(D, C).cuda()
    gen = torch.Generator(device="cuda").manual_seed(2)
    up_x = torch.randn(B, N, c0.x.shape[-1], device="cuda", generator=gen)
    up_s = torch.randn(B, N, C, device="cuda", generator=gen)

    def run(x0, s0):
        leaf = s0.detach().requires_grad_(True)
        x, s = leaf_rollout(x0, leaf)
        torch.autograd.backward([x, s], [up_x, up_s])
        return [x.detach(), s.detach(), leaf.grad] + [p.grad for p in model.parameters()]

    def leaf_rollout(x0, leaf):
        x, s = x0, leaf
        for _ in range(K):
            x, s, _ = S.step_euler(model, x, s, grid, update_prob=1.0)
        return x, s

    xs = [torch.from_numpy(c.x).cuda() for c in cases]
    ss = [torch.from_numpy(c.s).cuda() for c in cases]
    for p in model.parameters():
        p.grad = torch.zeros_like(p)
    run(xs[0], ss[0])  # teaches the grid its fused passes
    eager = []
    for x0, s0 in zip(xs, ss):
        for p in model.parameters():
            p.grad.zero_()
        eager.append([t.clone() for t in run(x0, s0)])
    grid.set_capture_capacity(2 * grid.list_capacity_hint())
    static_x, static_s = xs[0].clone(), ss[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for p in model.parameters():
                p.grad.zero_()
            run(static_x, static_s)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    for p in model.parameters():
        p.grad.zero_()
    with torch.cuda.graph(graph):
        outs = run(static_x, static_s)
    names = ["x", "s", "dL/ds0"] + [f"dL/dW{i}" for i in range(len(list(model.parameters())))]
    for k in (1, 2, 0):
        static_x.copy_(xs[k])
        static_s.copy_(ss[k])
        for p in model.parameters():
            p.grad.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(names, outs, eager[k]):
            assert torch.allclose(got, ref, rtol=1e-6, atol=1e-7), f"replay {k}: {name}"
    assert not grid.list_overflow()
    grid.set_capture_capacity(0)
