"""Timings of the paths around the perception operators, each beside the
reference's own torch formulation of the same computation on the same GPU
(``python bench.py --extras``; one JSON line per measurement):

* ``perceive``: NPA.perceive forward + backward (models/npa.py:87-137) with
  the fused feature kernels, against the reference's torch feature assembly
  over the same sphops operators;
* ``step_euler``: perception, an NPA-shaped MLP (128 hidden units), the Euler
  update and a loss on x, s and the |dx| stats, forward + backward
  (models/npa.py:123-204), fused update against the reference's torch ops;
* ``mlp``: the NPA MLP forward + backward over 2^20 rows, torch's autograd
  against npa_amd.mlp's row-chunked weight gradients;
* ``splat``: splat_particles_batch forward + backward (utils/splatting.py),
  against the reference's torch scatter_add_ formulation;
* ``rollout``: an 8-step step_euler rollout with its backward at the
  reference's growing-config shape, eager and replayed from one HIP graph;
* ``graph``: the bench's perception step eager and replayed from a HIP graph
  (the grid's capture mode), for every BASELINE configuration.

The reference's torch formulations are restated in oracle/torch_ref.py (test
and measurement infrastructure, never called by the library); this file
imports them only inside the baseline leg of each measurement.
"""
import json
import os
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import npa_amd.sphops as sp
from npa_amd import perceive as fused_perceive
from npa_amd import splatting, step, workloads


def _time(fn, iters, warmup=3):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def _baseline():
    """The reference's torch formulations: the baseline leg only."""
    from oracle import torch_ref
    return torch_ref


def _grid(wl):
    return sp.HashGrid(dim=wl.dim, boundary="periodic" if wl.periodic else "clamped", mode=wl.mode,
                       grid_size=list(wl.grid_size), eps=wl.h, num_particles=wl.N, batch_size=wl.B,
                       max_particles_per_block=wl.maxp)


class _NPA(torch.nn.Module):
    """The attributes of the reference's NPA that perception and step_euler
    read (models/npa.py:15-63), with its MLP shape."""

    def __init__(self, D, C, hidden=128):
        super().__init__()
        self.spatial_dims = D
        self.register_buffer("eps0", torch.tensor([0.1]))
        self.register_buffer("alpha", torch.tensor([1.0]))
        self.state_grad = self.density_grad = self.log_norm_grad = self.log_norm_density_grad = True
        self.stopgrad_pos, self.stopgrad_state = True, False
        self.model = torch.nn.Sequential(torch.nn.Linear(2 * C + C * D + D, hidden), torch.nn.ReLU(),
                                         torch.nn.Linear(hidden, D + C, bias=False))


# ---- measurements

def bench_perceive(cfg="cfg5", iters=20):
    wl = workloads.make(cfg)
    dev = torch.device("cuda", 0)
    x, s = torch.from_numpy(wl.x).to(dev), torch.from_numpy(wl.s).to(dev)
    grid = _grid(wl)
    W = 2 * wl.C + wl.C * wl.dim + wl.dim
    dz = torch.randn(wl.B, wl.N, W, device=dev, generator=torch.Generator(device=dev).manual_seed(0))

    def run(fused):
        sr = s.detach().requires_grad_(True)
        z = fused_perceive.perceive(x, sr, grid, eps0=0.1)[0] if fused else _baseline().perceive(x, sr, grid)[0]
        z.backward(dz)

    return {"bench": "perceive", "config": cfg, "what": "NPA.perceive forward + backward (stopgrad_pos)",
            "fused_ms": _time(lambda: run(True), iters), "reference_torch_ms": _time(lambda: run(False), iters)}


def bench_step(cfg="cfg5", iters=10):
    wl = workloads.make(cfg)
    dev = torch.device("cuda", 0)
    x, s = torch.from_numpy(wl.x).to(dev), torch.from_numpy(wl.s).to(dev)
    grid = _grid(wl)
    torch.manual_seed(0)
    model = _NPA(wl.dim, wl.C).to(dev)

    def run(fused):
        sr = s.detach().requires_grad_(True)
        if fused:
            xn, sn, st = step.step_euler(model, x, sr, grid, update_prob=0.5, intermediate=True)
            dn = st["dx_norm"]
        else:  # the reference's step: torch feature assembly, torch MLP, torch update
            ref = _baseline()
            z, xb, sb, _ = ref.perceive(x, sr, grid)
            xn, sn, dn = ref.euler(model.model(z), xb, sb, wl.dim, model.alpha, grid.eps, 0.5)
        ((sn ** 2).mean() + (xn ** 2).mean() + dn).backward()

    return {"bench": "step_euler", "config": cfg,
            "what": "perception + MLP(128) + Euler update + loss, forward + backward",
            "fused_ms": _time(lambda: run(True), iters), "reference_torch_ms": _time(lambda: run(False), iters)}


def bench_splat(images=8, particles=4096, img_size=256, pixel_size=2.0 / 64, iters=10):
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    x = (torch.rand(images, particles, 2, device=dev, generator=g) - 0.5) * 1.6
    c = torch.rand(images, particles, 8, device=dev, generator=g)
    up = torch.randn(images, img_size, img_size, 4, device=dev, generator=g)
    kw = dict(img_size=img_size, sigma=1.0, lo=-1.0, hi=1.0, y_up=True, pixel_size=pixel_size)

    def run(fused):
        xg, cg = x.clone().requires_grad_(True), c.clone().requires_grad_(True)
        if fused:
            img = splatting.splat_particles_batch(xg, cg, **kw)
        else:
            img = torch.stack([_baseline().splat(xg[b], cg[b], **kw) for b in range(images)])
        img.backward(up)

    return {"bench": "splat", "config": f"{images} images x {particles} particles, {img_size}^2, sigma 1.0, "
            f"pixel_size {pixel_size:.5g} ({img_size * pixel_size / 2:.1f} px)",
            "what": "splat_particles_batch forward + backward",
            "fused_ms": _time(lambda: run(True), iters), "reference_torch_ms": _time(lambda: run(False), iters)}


def bench_graph(cfg, iters=20):
    wl = workloads.make(cfg)
    dev = torch.device("cuda", 0)
    B, N, C, D = wl.B, wl.N, wl.C, wl.dim
    x, s = torch.from_numpy(wl.x).to(dev), torch.from_numpy(wl.s).to(dev)
    gen = torch.Generator(device=dev).manual_seed(1)
    ups = [torch.randn(B, N, C, device=dev, generator=gen), torch.randn(B, N, C, D, device=dev, generator=gen),
           torch.randn(B, N, D, device=dev, generator=gen)]
    grid = _grid(wl)

    def one(xx, ss):
        xr, sr = xx.detach().requires_grad_(True), ss.detach().requires_grad_(True)
        with torch.no_grad():
            snap = grid.instantiate(xr)
        xb, sb = sp.bin_particles(xr, sr, snap)
        rho = sp.density(xb, snap)
        torch.autograd.backward([sp.blur(xb, rho, sb, snap), sp.gradient_hybrid(xb, rho, sb, snap),
                                 sp.density_gradient(xb, snap)], ups)

    eager = _time(lambda: one(x, s), iters)
    grid.set_capture_capacity(int(grid.list_capacity_hint() * 1.25))
    sx, ss_ = x.clone(), s.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            one(sx, ss_)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        one(sx, ss_)
    replay = _time(graph.replay, iters)
    overflow = grid.list_overflow()
    grid.set_capture_capacity(0)
    return {"bench": "graph", "config": cfg, "what": "the bench's perception step, fwd + full bwd",
            "eager_ms": eager, "graph_replay_ms": replay, "list_overflow": overflow}


def bench_mlp(rows=1 << 20, iters=10):
    """The NPA MLP (83 -> 128 -> ReLU -> 19, the 3D C = 16 shape) forward +
    backward over one row per particle: torch's own autograd against
    npa_amd.mlp (row-chunked weight gradients)."""
    from npa_amd import mlp as M
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    net = torch.nn.Sequential(torch.nn.Linear(83, 128), torch.nn.ReLU(), torch.nn.Linear(128, 19, bias=False)).to(dev)
    z = torch.randn(rows, 83, device=dev)
    up = torch.randn(rows, 19, device=dev)

    def run(fused):
        zz = z.detach().requires_grad_(True)
        (M.mlp(net, zz) if fused else net(zz)).backward(up)

    return {"bench": "mlp", "config": f"{rows} rows, 83 -> 128 -> 19", "what": "MLP forward + backward",
            "fused_ms": _time(lambda: run(True), iters), "reference_torch_ms": _time(lambda: run(False), iters)}


def bench_rollout(K=8, B=8, N=4096, C=16, iters=5):
    """A K-step step_euler rollout with its backward, the shape of the
    reference's training loop (train.py:227-237; growing config: batch 8 of
    4096 2D particles, 16 channels), eager and replayed from one captured
    graph.  No update mask (update_prob = 1): the mask's random draws would
    need a graph-safe generator."""
    from npa_amd import workloads as W
    dev = torch.device("cuda", 0)
    wl = W.make("cfg1")
    rng = torch.Generator(device=dev).manual_seed(0)
    x0 = torch.zeros(B, N, 2, device=dev)
    r = torch.sqrt(torch.rand(B, N, device=dev, generator=rng)) * 0.5
    th = torch.rand(B, N, device=dev, generator=rng) * 6.283185307179586
    x0[..., 0], x0[..., 1] = r * torch.cos(th), r * torch.sin(th)
    s0 = torch.randn(B, N, C, device=dev, generator=rng) * 0.1
    grid = sp.HashGrid(dim=2, boundary="clamped", mode="grid", grid_size=list(wl.grid_size), eps=wl.h,
                       num_particles=N, batch_size=B, max_particles_per_block=wl.maxp)
    torch.manual_seed(0)
    model = _NPA(2, C).to(dev)
    up_x, up_s = torch.randn_like(x0), torch.randn_like(s0)

    def run(xi, si):
        x, s = xi, si.detach().requires_grad_(True)
        for _ in range(K):
            x, s, _ = step.step_euler(model, x, s, grid, update_prob=1.0)
        torch.autograd.backward([x, s], [up_x, up_s])

    for p in model.parameters():
        p.grad = torch.zeros_like(p)
    eager = _time(lambda: run(x0, s0), iters)
    grid.set_capture_capacity(2 * grid.list_capacity_hint())
    sx, ss_ = x0.clone(), s0.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run(sx, ss_)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(sx, ss_)
    replay = _time(graph.replay, iters)
    overflow = grid.list_overflow()
    grid.set_capture_capacity(0)
    return {"bench": "rollout", "config": f"{K} steps, batch {B} x {N} 2D particles, C = {C}, MLP 128",
            "what": "step_euler rollout + backward", "eager_ms": eager, "graph_replay_ms": replay,
            "list_overflow": overflow}


def run_all():
    torch.cuda.set_device(0)
    results = [bench_perceive(), bench_step(), bench_mlp(), bench_splat(), bench_rollout()]
    results += [bench_graph(c) for c in ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5")]
    for r in results:
        print(json.dumps(r), flush=True)
    return results


if __name__ == "__main__":
    # python bench_extras.py [perceive|step|mlp|splat|rollout ...]: the
    # named measurements only (all of them with no argument)
    import sys
    names = sys.argv[1:]
    if not names:
        run_all()
    else:
        torch.cuda.set_device(0)
        table = {"perceive": bench_perceive, "step": bench_step, "mlp": bench_mlp, "splat": bench_splat,
                 "rollout": bench_rollout}
        for n in names:
            print(json.dumps(table[n]()), flush=True)
