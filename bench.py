"""Benchmark: fwd+bwd SPH perception pair-interactions/s on one MI355X.

One step is the drop-in path NPA's perception takes (models/npa.py:87-137 of
the reference) with the full backward (stopgrad_pos=False):
  instantiate (rebin) -> bin_particles -> density -> blur -> gradient_hybrid
  -> density_gradient -> backward of all three outputs with fixed upstream
  gradients (through density and the permutation).
The calls are the reference's public functions; the library evaluates
density + density_gradient and blur + gradient_hybrid as two fused passes
once the grid has seen them called together (the warm-up step does that).
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
    ap.add_argument("--mode", default="grid", choices=["grid", "particle"],
                    help="the reference's HashGrid mode (particle: Morton order, cubic power-of-two grid)")
    ap.add_argument("--tiles", action="store_true",
                    help="use the opt-in cell-tiled pass-B backward (sphops_neighbor_tiles)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 FETCH_SIZE / WRITE_SIZE runs that fill roofline.traffic")
    ap.add_argument("--extras", action="store_true",
                    help="instead of the step: time the fused perceive glue, step_euler update, splatting and "
                         "graph replay beside the reference's torch formulations (one JSON line each)")
    ap.add_argument("--pmc-child", default=None, help=argparse.SUPPRESS)
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
        # fused passes: pass A = density + density_gradient, pass B = blur + gradient_hybrid
        "pass_a_fwd": x + m + f + D * f,
        "pass_b_fwd": x + m + rho + s + C * f + C * D * f,
        "pass_a_bwd": x + m + f + D * f + P * f,
        "pass_b_bwd": x + m + rho + s + g_s + g_cd + P * f + C * f + f,
        "pass_b_bwd_ds": x + m + rho + g_s + g_cd + C * f,
    }


# pair kernels the timed step launches (with pass fusion), one launch each,
# per variant
STEP_KERNELS = {
    "full": ("pass_a_fwd", "pass_b_fwd", "pass_a_bwd", "pass_b_bwd"),
    "npa": ("density_fwd", "pass_b_fwd", "pass_b_bwd_ds"),
}
DOMINANT = {"full": "pass_b_bwd", "npa": "pass_b_bwd_ds"}

def pair_kernel(name, D, periodic, C):
    """rocprofv3 kernel-name fragment of the pair kernel an operator call of
    the step launches (the call also launches a packing kernel), or None."""
    p = "true" if periodic else "false"
    split = C in (16, 32)  # blur + gradient_hybrid on the lane-split kernels
    names = {
        "pass_a_fwd": f"OpDensityPair<{D}, {p}>",
        "pass_a_bwd": f"OpDensityPairBwd<{D}, {p}>",
        "pass_b_fwd": f"k_blur_hybrid_fwd_quad<{D}, {p}, {C // 4}," if split else None,
        "pass_b_bwd": f"k_blur_hybrid_bwd_quad<{D}, {p}, {C // 4}, true," if split else None,
        "pass_b_bwd_ds": f"k_blur_hybrid_bwd_quad<{D}, {p}, {C // 4}, false," if split else None,
    }
    return names.get(name)


COPY_BYTES = 256 << 20
CUS, XCDS = 256, 8  # MI355X


def step_bytes(C, D, P, full=True):
    """Minimal compulsory HBM bytes of one step per particle (each tensor of
    the step read or written once per pass: hash + sort, permute, pass A,
    pass B, their backward, permute backward) and per cell (the bin_offsets
    write): full backward 48P + 36C + 8CD + 8D + 68, NPA default
    (stopgrad_pos, no density gradient) 32P + 32C + 8CD + 4D + 56."""
    if full:
        return 48 * P + 36 * C + 8 * C * D + 8 * D + 68, 4
    return 32 * P + 32 * C + 8 * C * D + 4 * D + 56, 4


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(multi-GPU sharding is a design note, not implemented)"}))
        sys.exit(2)
    if args.pmc_child:
        return pmc_child(args)
    if args.extras:
        import bench_extras
        bench_extras.run_all()
        return
    # counter runs first, in child processes, before this process touches the GPU
    pmc = None
    if not args.no_traffic:
        pmc = measure_traffic(args, DOMINANT[args.variant])
    import numpy as np
    import torch

    import npa_amd.sphops as sp
    from npa_amd import workloads

    torch.cuda.set_device(0)
    t0 = time.time()
    wl = workloads.make(args.config, mode=args.mode)
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
    grid = sp.HashGrid(dim=D, boundary="periodic" if wl.periodic else "clamped", mode=wl.mode,
                       grid_size=list(wl.grid_size), eps=wl.h, num_particles=N, batch_size=B,
                       max_particles_per_block=wl.maxp)
    full = args.variant == "full"
    grid.hashgrid.tiles_enabled = args.tiles

    def step(full=full):
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
    def timed_steps(variant_full):
        for _ in range(args.warmup):
            step(variant_full)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            step(variant_full)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    ms = timed_steps(full)
    print(f"[bench] {args.steps} steps ({args.variant}): {ms:.3f} ms/step, {pairs / (ms * 1e-3) / 1e9:.3f} G pairs/s",
          file=sys.stderr, flush=True)
    # the other backward variant of the same step, reported alongside
    other = "npa" if full else "full"
    ms_other = timed_steps(not full)
    print(f"[bench] {args.steps} steps ({other}): {ms_other:.3f} ms/step", file=sys.stderr, flush=True)

    # ---- per-kernel timing (HIP events on the launch stream)
    kt = kernel_times(sp, grid, x, s, g_blur, g_hyb, g_dg, True, args.kernel_reps)
    ppb = per_particle_bytes(C, D, P)
    dom = max(STEP_KERNELS[args.variant], key=lambda k: kt[k])
    dom_ms = kt[dom]
    alg = ppb[dom] * B * N
    achieved = alg / (dom_ms * 1e-3) / 1e9
    pp, pc = step_bytes(C, D, P, full)
    step_alg = pp * B * N + pc * cells
    po, pco = step_bytes(C, D, P, not full)
    other_alg = po * B * N + pco * cells
    other_dom = max(STEP_KERNELS[other], key=lambda k: kt[k])
    traffic = None
    if pmc is not None and pmc.get("kernel") == dom:
        traffic = pmc["bytes_per_launch"]
    copy_gbs = measured_copy_gbs()
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
            "workload": f"{wl.name}: {workloads.DESCRIPTIONS[wl.name]}; B={B} N={N} C={C} fp32, h={wl.h:.6g} "
                        f"({workloads.TARGETS[wl.name]:g} mean neighbours), "
                        f"{'periodic' if wl.periodic else 'clamped'} {wl.mode}-mode grid "
                        f"{'x'.join(map(str, wl.grid_size))}, "
                        f"rebin every step, {'full backward' if full else 'NPA-default backward (stopgrad_pos)'}",
            "particles_per_step": B * N,
            "pairs_per_step": pairs,
            "particles_per_s": B * N / (ms * 1e-3),
            "step_alg_bytes": step_alg,
            "step_roofline_frac": step_alg / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
            "kernel_ms": kt,
            "other_variant": {
                "variant": "npa-default (stopgrad_pos: dL/ds only, no density gradient; models/npa.py:28,95-96)"
                           if full else "full backward",
                "ms_per_step": ms_other,
                "pairs_per_s": pairs / (ms_other * 1e-3),
                "particles_per_s": B * N / (ms_other * 1e-3),
                "step_alg_bytes": other_alg,
                "step_roofline_frac": other_alg / (ms_other * 1e-3) / (HBM_PEAK_GBS * 1e9),
                "dominant_kernel": other_dom,
                "dominant_kernel_ms": kt[other_dom],
            },
        },
        "roofline": {
            # the roofline the fraction is reported against (the path is a
            # sparse gather with no dense contraction: HBM, not MFMA); what the
            # counters show limits the kernel is `limiter`
            "bound": "hbm",
            "limiter": limiter(pmc, traffic, dom_ms) if pmc is not None and pmc.get("kernel") == dom else None,
            "kernel": dom,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "alg_bytes_per_launch": alg,
            "avg_launch_ms": dom_ms,
            "pair_kernel": pair_kernel(dom, D, wl.periodic, C),
            "valu_busy": pmc.get("valu_busy") if pmc is not None and pmc.get("kernel") == dom else None,
            "ta_busy": pmc.get("ta_busy") if pmc is not None and pmc.get("kernel") == dom else None,
            "td_busy": pmc.get("td_busy") if pmc is not None and pmc.get("kernel") == dom else None,
            "measured_copy_gbs": copy_gbs,
            "pmc": pmc,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def limiter(pmc, traffic, dom_ms):
    """What bounds the dominant kernel, from its counters: the busiest of the
    VALU issue (valu_busy), the vector-memory address/data path that carries
    neighbour rows from L2 (TA / TD busy) and HBM (measured traffic over time
    against the 8 TB/s peak)."""
    util = {"valu": pmc.get("valu_busy"), "vmem-l2 (TA/TD)": max(pmc.get("ta_busy") or 0.0, pmc.get("td_busy") or 0.0),
            "hbm": traffic / (dom_ms * 1e-3) / (HBM_PEAK_GBS * 1e9) if traffic else None}
    util = {k: v for k, v in util.items() if v is not None}
    if not util:
        return None
    name = max(util, key=util.get)
    return {"name": name, "utilisation": util}


def measured_copy_gbs(nbytes=COPY_BYTES, reps=20):
    """Device copy bandwidth on this GPU (read + write bytes over time, HIP
    events): the practical ceiling next to the 8 TB/s spec figure."""
    import torch
    src = torch.ones(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    return 2 * nbytes / (e0.elapsed_time(e1) / reps * 1e-3) / 1e9


def kernel_times(sp, grid, x, s, g_blur, g_hyb, g_dg, full, reps, only=None):
    """Average duration of each native operator call on the path the step
    takes (generic entry points with the snapshot's neighbour list), by HIP
    events on the current stream around `reps` back-to-back calls.  A
    forward call is one packing kernel plus one pair kernel; a backward call
    reads the records its forward packed (as in the step) and is the pair
    kernel alone."""
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

    if only is None:
        timed("instantiate", lambda: grid.instantiate(x))
    snap = grid.instantiate(x)
    xb, sb = sp.bin_particles(x, s, snap)
    if only is None:
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
    # the (x, weight) records a forward packs for its backward (mass and
    # volume weights): backward calls read them, as in the step
    pk_m = torch.empty(B * N, 4, device=x.device)
    pk_v = torch.empty(B * N, 4, device=x.device)
    hg.op_forward(O.OP_DENSITY_PAIR, xb, bufs["rho"], bo, mass=m, nbr=nbr, out2=bufs["dg"], packed=pk_m)
    hg.op_forward(O.OP_BLUR_GRADIENT_HYBRID, xb, bufs["blur"], bo, mass=m, rho=rho, state=sb, nbr=nbr,
                  out2=bufs["gh"], packed=pk_v)
    calls = {
        "density_fwd": lambda: hg.op_forward(O.OP_DENSITY, xb, bufs["rho"], bo, mass=m, nbr=nbr),
        "density_gradient_fwd": lambda: hg.op_forward(O.OP_DENSITY_GRADIENT, xb, bufs["dg"], bo, mass=m, nbr=nbr),
        "blur_fwd": lambda: hg.op_forward(O.OP_BLUR, xb, bufs["blur"], bo, mass=m, rho=rho, state=sb, nbr=nbr),
        "gradient_hybrid_fwd": lambda: hg.op_forward(O.OP_GRADIENT_HYBRID, xb, bufs["gh"], bo, mass=m, rho=rho,
                                                     state=sb, nbr=nbr),
        "blur_bwd": lambda: hg.op_backward(O.OP_BLUR, xb, g_blur, bo, m, rho=rho, state=sb, grad_x=bufs["gx"],
                                           grad_state=bufs["gs"], grad_rho=bufs["gr"], dLdx=full, dLds=True,
                                           dLdrho=full, nbr=nbr, packed=pk_v),
        "gradient_bwd": lambda: hg.op_backward(O.OP_GRADIENT, xb, g_hyb, bo, m, rho=rho, state=sb, grad_x=bufs["gx"],
                                               grad_state=bufs["gs"], grad_rho=bufs["gr"], dLdx=full, dLds=True,
                                               dLdrho=full, nbr=nbr, packed=pk_v),
    }
    if full:
        calls["density_gradient_bwd"] = lambda: hg.op_backward(O.OP_DENSITY_GRADIENT, xb, g_dg, bo, m,
                                                               grad_x=bufs["gx"], nbr=nbr, packed=pk_m)
        calls["density_bwd"] = lambda: hg.op_backward(O.OP_DENSITY, xb, rho, bo, m, grad_x=bufs["gx"], nbr=nbr,
                                                      packed=pk_m)
    calls["pass_a_fwd"] = lambda: hg.op_forward(O.OP_DENSITY_PAIR, xb, bufs["rho"], bo, mass=m, nbr=nbr,
                                                out2=bufs["dg"])
    calls["pass_b_fwd"] = lambda: hg.op_forward(O.OP_BLUR_GRADIENT_HYBRID, xb, bufs["blur"], bo, mass=m, rho=rho,
                                                state=sb, nbr=nbr, out2=bufs["gh"])
    calls["pass_a_bwd"] = lambda: hg.op_backward(O.OP_DENSITY_PAIR, xb, rho, bo, m, grad_x=bufs["gx"], nbr=nbr,
                                                 upstream2=g_dg, packed=pk_m)
    calls["pass_b_bwd"] = lambda: hg.op_backward(O.OP_BLUR_GRADIENT_HYBRID, xb, g_blur, bo, m, rho=rho, state=sb,
                                                 grad_x=bufs["gx"], grad_state=bufs["gs"], grad_rho=bufs["gr"],
                                                 nbr=nbr, upstream2=g_hyb, packed=pk_v)
    calls["pass_b_bwd_ds"] = lambda: hg.op_backward(O.OP_BLUR_GRADIENT_HYBRID, xb, g_blur, bo, m, rho=rho,
                                                    state=sb, grad_state=bufs["gs"], dLdx=False, dLdrho=False,
                                                    nbr=nbr, upstream2=g_hyb, packed=pk_v)
    for name, fn in calls.items():
        if only is None or name == only:
            timed(name, fn)
    return out


def pmc_child(args):
    """Runs under rocprofv3 --pmc: a plain copy of COPY_BYTES (the counter
    calibration), then three calls of one timed operator on the workload."""
    import torch
    import npa_amd.sphops as sp
    from npa_amd import workloads
    torch.cuda.set_device(0)
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    wl = workloads.make(args.config, mode=args.mode)
    B, N, C, D = wl.B, wl.N, wl.C, wl.dim
    dev = torch.device("cuda", 0)
    x = torch.from_numpy(wl.x).to(dev)
    s = torch.from_numpy(wl.s).to(dev)
    gen = torch.Generator(device=dev).manual_seed(1)
    g_blur = torch.randn(B, N, C, device=dev, generator=gen)
    g_hyb = torch.randn(B, N, C, D, device=dev, generator=gen)
    g_dg = torch.randn(B, N, D, device=dev, generator=gen)
    grid = sp.HashGrid(dim=D, boundary="periodic" if wl.periodic else "clamped", mode=wl.mode,
                       grid_size=list(wl.grid_size), eps=wl.h, num_particles=N, batch_size=B,
                       max_particles_per_block=wl.maxp)
    grid.hashgrid.tiles_enabled = args.tiles
    kernel_times(sp, grid, x, s, g_blur, g_hyb, g_dg, args.variant == "full", 3, only=args.pmc_child)
    torch.cuda.synchronize()
    print(f"[pmc-child] {args.pmc_child} done", flush=True)


def _pmc_run(counter, kernel, frag, args):
    """One rocprofv3 --pmc run of the child for one or more counters
    (space-separated, all in one pass); returns (copy, kernel) mean values
    per dispatch, or dicts of them by counter name when several."""
    import csv
    import shutil
    import subprocess
    import tempfile
    prof = shutil.which("rocprofv3")
    if prof is None:
        raise RuntimeError("rocprofv3 not on PATH")
    out = tempfile.mkdtemp(prefix="npa_pmc_", dir="/tmp")
    names = counter.split()
    cmd = [prof, "--pmc", *names, "--output-format", "csv", "-d", out, "-o", "run", "--",
           sys.executable, os.path.abspath(__file__), "--pmc-child", kernel, "--config", args.config,
           "--variant", args.variant, "--mode", args.mode] + (["--tiles"] if args.tiles else [])
    env = dict(os.environ, TMPDIR="/tmp")
    r = subprocess.run(cmd, cwd="/tmp", env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=240)
    if r.returncode != 0 or b"[pmc-child]" not in r.stdout:
        raise RuntimeError(f"rocprofv3 --pmc {counter} exited {r.returncode}: {r.stdout[-400:]!r}")
    path = None
    for root, _, files in os.walk(out):
        for f in files:
            if f.endswith("counter_collection.csv"):
                path = os.path.join(root, f)
    if path is None:
        raise RuntimeError("no counter_collection.csv")
    per_dispatch = {}
    with open(path) as fh:
        for row in csv.DictReader(fh):
            if row["Counter_Name"] not in names:
                continue
            key = (row["Counter_Name"], row["Dispatch_Id"], row["Kernel_Name"])
            per_dispatch[key] = per_dispatch.get(key, 0.0) + float(row["Counter_Value"])
    shutil.rmtree(out, ignore_errors=True)
    res = {}
    for cn in names:
        copy, target = [], []
        for (c, _, name), v in per_dispatch.items():
            if c != cn:
                continue
            if "copy" in name.lower():
                copy.append(v)
            elif frag in name:
                target.append(v)
        if not copy or not target:
            raise RuntimeError(f"{cn}: kernels not found in the counter output")
        # the largest copy dispatches are the calibration copies
        copy = sorted(copy)[-3:]
        res[cn] = (sum(copy) / len(copy), sum(target) / len(target))
    return res[names[0]] if len(names) == 1 else res


def measure_traffic(args, kernel):
    """HBM bytes per launch of `kernel`'s pair kernel: FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch), each scaled by what the same counter reads
    for a plain copy of COPY_BYTES (which must fetch and write COPY_BYTES)."""
    try:
        from npa_amd import workloads
        wl = workloads.make(args.config, mode=args.mode)
        frag = pair_kernel(kernel, wl.dim, wl.periodic, wl.C)
        if frag is None:
            raise RuntimeError(f"no single pair kernel for {kernel} at C = {wl.C}")
        res = {"kernel": kernel, "copy_bytes": COPY_BYTES}
        total = 0.0
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            c, t = _pmc_run(counter, kernel, frag, args)
            scale = COPY_BYTES / (c * 1024.0)
            res[counter] = {"copy_kib": c, "kernel_kib": t, "scale": scale, "kernel_bytes": t * 1024.0 * scale}
            total += t * 1024.0 * scale
        res["bytes_per_launch"] = total
        # VALU utilisation: VALU issue cycles per CU (one wave instruction per
        # CU and clock at most) over the active clock of an XCD
        # and the vector-memory path: TA / TD busy cycles summed over the 256
        # instances (one per CU) over the same clock
        busy = _pmc_run("SQ_ACTIVE_INST_VALU TA_TA_BUSY_sum TD_TD_BUSY_sum GRBM_GUI_ACTIVE", kernel, frag, args)
        gui = busy["GRBM_GUI_ACTIVE"][1] / XCDS
        if gui > 0:
            res["valu_busy"] = busy["SQ_ACTIVE_INST_VALU"][1] / CUS / gui
            res["ta_busy"] = busy["TA_TA_BUSY_sum"][1] / CUS / gui
            res["td_busy"] = busy["TD_TD_BUSY_sum"][1] / CUS / gui
        print(f"[bench] traffic of {kernel}: {total / 1e6:.1f} MB per launch "
              f"(fetch {res['FETCH_SIZE']['kernel_bytes'] / 1e6:.1f}, write {res['WRITE_SIZE']['kernel_bytes'] / 1e6:.1f})",
              file=sys.stderr, flush=True)
        return res
    except Exception as e:  # the counters are a report, not part of the measurement
        print(f"[bench] traffic not measured: {e}", file=sys.stderr, flush=True)
        return None


def cpu_baseline(wl, pairs_per_step):
    """The reference's CPU path (brute-force all-pairs torch, restated in
    oracle/bruteforce.py, fp32, autograd backward) on the host cores: a
    bounded sample of row blocks of the same cloud, extrapolated linearly to
    all N rows (the all-pairs cost is the same for every row block)."""
    import numpy as np
    import torch
    from oracle import bruteforce

    threads = torch.get_num_threads()
    affinity = len(os.sched_getaffinity(0))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
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
        "affinity_cores": affinity,
        "cpu_model": model,
        "kind": "port",
        "sample": f"{nblk} blocks of {rows} rows x all {N} columns of the same cloud, fp32 torch CPU "
                  f"fwd+bwd; {t_total:.1f}s measured, extrapolated linearly to {N} rows "
                  f"(step estimate {t_step:.3g}s)",
    }


if __name__ == "__main__":
    main()
