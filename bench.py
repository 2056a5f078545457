"""Benchmark: fwd+bwd SPH perception pair-interactions/s on one MI355X.

One step is the drop-in path NPA's perception takes (models/npa.py:87-137 of
the reference) with the full backward (stopgrad_pos=False):
  instantiate (rebin) -> bin_particles -> density -> blur -> gradient_hybrid
  -> density_gradient -> backward of all three outputs with fixed upstream
  gradients (through density and the permutation).
Workload: BASELINE.json config 5 (3D stress): N = 1,048,576 particles from 8
Gaussians, C = 16, h calibrated to 32 mean neighbours, clamped grid, inputs
resident in HBM before timing.

Printed: one JSON line (metric, value = pair-interactions/s, ...) with
``roofline`` for the dominant kernel (its algorithmic bytes per launch over
its HIP-event-timed average duration) and ``cpu_baseline`` (the reference's
brute-force torch CPU path, restated in oracle/bruteforce.py, timed on a
bounded row sample of the same workload and extrapolated).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg5")
    ap.add_argument("--variant", default="full", choices=["full", "npa"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=10)
    return ap.parse_args()


def per_particle_bytes(C, D, P):
    """Algorithmic HBM bytes per particle for each native kernel (each input
    row read once, each output row written once; neighbour re-reads are
    served from cache and not counted)."""
    f = 4
    x, m, rho = P * f, f, f
    s, g_s, g_cd = C * f, C * f, C * D * f
    return {
        "density_fwd": x + m + f,
        "density_gradient_fwd": x + m + D * f,
        "blur_fwd": x + m + rho + s + C * f,
        "gradient_hybrid_fwd": x + m + rho + s + C * D * f,
        "blur_bwd": x + m + rho + s + g_s + P * f + C * f + f,
        "gradient_bwd": x + m + rho + s + g_cd + P * f + C * f + f,
        "density_gradient_bwd": x + m + D * f + P * f,
        "density_bwd": x + m + f + P * f,
    }


def step_bytes(C, D, P, cells):
    """Algorithmic bytes of one full step: the kernels above plus binning
    (key pass, sort, permutation, bin_offsets write), bin and unbin moves."""
    k = per_particle_bytes(C, D, P)
    f = 4
    binning = P * f + 4 * f + f        # read x, keys+values out, permutation out
    move = 2 * (P * f + C * f + f) + f  # bin_particles read+write, perm read
    unmove = 2 * (P * f + C * f + f) + f
    per_particle = binning + move + unmove + sum(k.values())
    return per_particle, 4 * cells


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(multi-GPU sharding is a design note, not implemented)"}))
        sys.exit(2)
    import numpy as np
    import torch

    import npa_amd.sphops as sp
    from npa_amd import workloads

    torch.cuda.set_device(0)
    t0 = time.time()
    wl = workloads.make(args.config)
    B, N, C, D = wl.B, wl.N, wl.C, wl.dim
    P = wl.x.shape[-1]
    cells = int(np.prod(wl.grid_size)) * B
    print(f"[bench] workload {wl.name}: B={B} N={N} C={C} D={D} h={wl.h:.6g} grid={wl.grid_size} "
          f"({cells / 1e6:.1f} M cells), built in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    dev = torch.device("cuda", 0)
    x = torch.from_numpy(wl.x).to(dev)
    s = torch.from_numpy(wl.s).to(dev)
    gen = torch.Generator(device=dev).manual_seed(1)
    g_blur = torch.randn(B, N, C, device=dev, generator=gen)
    g_hyb = torch.randn(B, N, C, D, device=dev, generator=gen)
    g_dg = torch.randn(B, N, D, device=dev, generator=gen)
    grid = sp.HashGrid(dim=D, boundary="periodic" if wl.periodic else "clamped", mode="grid",
                       grid_size=list(wl.grid_size), eps=wl.h, num_particles=N, batch_size=B,
                       max_particles_per_block=wl.maxp)
    full = args.variant == "full"

    def step():
        xr = x.detach().requires_grad_(full)
        sr = s.detach().requires_grad_(True)
        with torch.no_grad():
            snap = grid.instantiate(xr)
        xb, sb = sp.bin_particles(xr, sr, snap)
        xp = xb if full else xb.detach()
        rho = sp.density(xp, snap)
        bl = sp.blur(xp, rho, sb, snap)
        gh = sp.gradient_hybrid(xp, rho, sb, snap)
        outs, grads = [bl, gh], [g_blur, g_hyb]
        if full:
            outs.append(sp.density_gradient(xp, snap))
            grads.append(g_dg)
        torch.autograd.backward(outs, grads)
        return snap, xb

    # pair-interactions per step (ordered pairs |r| < h incl. self), counted once
    snap0, xb0 = step()
    with torch.no_grad():
        pairs = float(sp.count(xb0.detach(), snap0).sum().item())
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    print(f"[bench] {args.steps} steps: {ms:.3f} ms/step, {pairs / (ms * 1e-3) / 1e9:.3f} G pairs/s",
          file=sys.stderr, flush=True)

    # ---- per-kernel timing (HIP events on the launch stream)
    kt = kernel_times(sp, grid, x, s, g_blur, g_hyb, g_dg, full, args.kernel_reps)
    ppb = per_particle_bytes(C, D, P)
    dom = max((k for k in kt if k in ppb), key=lambda k: kt[k])
    dom_ms = kt[dom]
    alg = ppb[dom] * B * N
    achieved = alg / (dom_ms * 1e-3) / 1e9
    pp, cell_bytes = step_bytes(C, D, P, cells)
    step_alg = pp * B * N + cell_bytes
    print("[bench] kernel ms: " + ", ".join(f"{k}={v:.3f}" for k, v in sorted(kt.items(), key=lambda t: -t[1])),
          file=sys.stderr, flush=True)

    cpu = None if args.no_cpu_baseline else cpu_baseline(wl, pairs)

    line = {
        "metric": "fwd+bwd perception pair-interactions/sec at 1 GPU; % of HBM roofline",
        "value": pairs / (ms * 1e-3),
        "unit": "pair-interactions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{wl.name}: 3D stress, B={B} N={N} particles from 8 Gaussians (log sigma U[0.01,0.2]), "
                        f"C={C} fp32, h={wl.h:.6g} (32 mean neighbours), clamped grid "
                        f"{'x'.join(map(str, wl.grid_size))}, rebin every step, "
                        f"{'full backward' if full else 'NPA-default backward (stopgrad_pos)'}",
            "particles_per_step": B * N,
            "pairs_per_step": pairs,
            "particles_per_s": B * N / (ms * 1e-3),
            "step_alg_bytes": step_alg,
            "step_roofline_frac": step_alg / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
            "kernel_ms": kt,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
            "alg_bytes_per_launch": alg,
            "avg_launch_ms": dom_ms,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def kernel_times(sp, grid, x, s, g_blur, g_hyb, g_dg, full, reps):
    """Average duration of each native operator call on the path the step
    takes (generic entry points with the snapshot's neighbour list), by HIP
    events on the current stream around `reps` back-to-back calls.  An
    operator call is one packing kernel plus one pair kernel."""
    import torch
    from npa_amd.sphops import _native as O
    from npa_amd.sphops.sph import _plan
    hg = grid.hashgrid
    out = {}

    def timed(name, fn, n=reps):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        out[name] = a.elapsed_time(b) / n

    timed("instantiate", lambda: grid.instantiate(x))
    snap = grid.instantiate(x)
    xb, sb = sp.bin_particles(x, s, snap)
    timed("bin_particles", lambda: sp.bin_particles(x, s, snap))
    timed("neighbor_list", lambda: hg.neighbor_list(xb, snap.bin_offsets))
    nbr = _plan(snap, xb)
    rho = sp.density(xb, snap)
    m = torch.ones_like(rho)
    B, N, C = s.shape
    D = grid.dim
    bo = snap.bin_offsets
    bufs = dict(rho=torch.empty_like(rho), blur=torch.empty_like(sb), dg=torch.empty(B, N, D, device=x.device),
                gh=torch.empty(B, N, C, D, device=x.device), gx=torch.empty_like(xb), gs=torch.empty_like(sb),
                gr=torch.empty_like(rho))
    calls = {
        "density_fwd": lambda: hg.op_forward(O.OP_DENSITY, xb, bufs["rho"], bo, mass=m, nbr=nbr),
        "density_gradient_fwd": lambda: hg.op_forward(O.OP_DENSITY_GRADIENT, xb, bufs["dg"], bo, mass=m, nbr=nbr),
        "blur_fwd": lambda: hg.op_forward(O.OP_BLUR, xb, bufs["blur"], bo, mass=m, rho=rho, state=sb, nbr=nbr),
        "gradient_hybrid_fwd": lambda: hg.op_forward(O.OP_GRADIENT_HYBRID, xb, bufs["gh"], bo, mass=m, rho=rho,
                                                     state=sb, nbr=nbr),
        "blur_bwd": lambda: hg.op_backward(O.OP_BLUR, xb, g_blur, bo, m, rho=rho, state=sb, grad_x=bufs["gx"],
                                           grad_state=bufs["gs"], grad_rho=bufs["gr"], dLdx=full, dLds=True,
                                           dLdrho=full, nbr=nbr),
        "gradient_bwd": lambda: hg.op_backward(O.OP_GRADIENT, xb, g_hyb, bo, m, rho=rho, state=sb, grad_x=bufs["gx"],
                                               grad_state=bufs["gs"], grad_rho=bufs["gr"], dLdx=full, dLds=True,
                                               dLdrho=full, nbr=nbr),
    }
    if full:
        calls["density_gradient_bwd"] = lambda: hg.op_backward(O.OP_DENSITY_GRADIENT, xb, g_dg, bo, m,
                                                               grad_x=bufs["gx"], nbr=nbr)
        calls["density_bwd"] = lambda: hg.op_backward(O.OP_DENSITY, xb, rho, bo, m, grad_x=bufs["gx"], nbr=nbr)
    for name, fn in calls.items():
        timed(name, fn)
    return out


def cpu_baseline(wl, pairs_per_step):
    """The reference's CPU path (brute-force all-pairs torch, restated in
    oracle/bruteforce.py, fp32, autograd backward) on the host cores: a
    bounded sample of row blocks of the same cloud, extrapolated linearly to
    all N rows (the all-pairs cost is the same for every row block)."""
    import numpy as np
    import torch
    from oracle import bruteforce

    threads = torch.get_num_threads()
    x = torch.from_numpy(wl.x[..., :wl.dim].astype(np.float32))
    s = torch.from_numpy(wl.s)
    N = wl.N
    rows = 8 if N > 200000 else 64
    box = None
    if wl.periodic:
        box = [g * wl.h for g in wl.grid_size]
    # warm-up block, then time blocks until ~15 s of work
    bruteforce.row_block_step(x, s, wl.h, 0, rows, wl.periodic, box)
    t_total, nblk = 0.0, 0
    while t_total < 15.0 and nblk < 64:
        a = (nblk * 7919 * rows) % max(1, N - rows)
        t = time.perf_counter()
        bruteforce.row_block_step(x, s, wl.h, a, rows, wl.periodic, box)
        t_total += time.perf_counter() - t
        nblk += 1
    per_row = t_total / (nblk * rows)
    t_step = per_row * N * wl.B
    return {
        "value": pairs_per_step / t_step,
        "unit": "pair-interactions/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{nblk} blocks of {rows} rows x all {N} columns of the same cloud, fp32 torch CPU "
                  f"fwd+bwd; {t_total:.1f}s measured, extrapolated linearly to {N} rows "
                  f"(step estimate {t_step:.3g}s)",
    }


if __name__ == "__main__":
    main()
