"""Synthetic particle clouds for the five benchmark configurations.

Each configuration fixes the cloud generator, the channel count C, the
boundary, the block size and a smoothing radius h calibrated so that the mean
neighbour count (pairs with |r| < h, self included) hits the target.  The
calibrated radii are stored in ``CALIBRATED_H`` (produced by
``python -m npa_amd.workloads --calibrate``, which bisects h on the seeded
sample with a KD-tree).  Grids are centred on the origin (the reference's
``floor(x/h) + G/2`` cell index) and sized to the data's extent.

Configurations (BASELINE.json ``configs``):
  cfg1  2D growing morphology: B=1, N=4096 uniform in the unit disk, C=16,
        ~20 neighbours, clamped grid, 32 particles per block.
  cfg2  2D texture: B=4, N=16384 uniform in [0,1)^2, C=12, ~24 neighbours,
        periodic box of side 1 (47 x 47 cells, h = 1/47), 32 per block.
  cfg3  2D point-cloud classification: B=64 clouds x 512 points on 3-6 random
        segments with N(0, 0.02^2) jitter, C=32, ~16 neighbours, clamped, 64.
  cfg4  3D Gaussian-splat growth: N=65536 from 4 isotropic Gaussians
        (sigma ~ U[0.05, 0.2], means ~ U[-0.5, 0.5]^3), C=32, ~30 neighbours.
  cfg5  3D stress: N=1,048,576 from 8 Gaussians (log sigma ~ U[log 0.01,
        log 0.2]), C=16, ~32 neighbours, clamped, rebinned every step.
The kernels are the reference's poly6/spiky pair (its only kernels); 3D
positions are float4 with w = 0.
"""
import math
from dataclasses import dataclass

import numpy as np

SEED = 42


@dataclass
class Workload:
    name: str
    x: np.ndarray          # (B, N, P) float32, P = 2 or 4
    s: np.ndarray          # (B, N, C) float32
    h: float
    grid_size: tuple
    periodic: bool
    maxp: int
    mode: str = "grid"

    @property
    def dim(self):
        return len(self.grid_size)

    @property
    def B(self):
        return self.x.shape[0]

    @property
    def N(self):
        return self.x.shape[1]

    @property
    def C(self):
        return self.s.shape[2]


TARGETS = {"cfg1": 20.0, "cfg2": 24.0, "cfg3": 16.0, "cfg4": 30.0, "cfg5": 32.0}

# One-line description of each configuration's cloud generator.
DESCRIPTIONS = {
    "cfg1": "2D growing morphology, positions uniform in the unit disk",
    "cfg2": "2D texture, positions uniform in the periodic unit box",
    "cfg3": "2D point-cloud classification, points on 3-6 random segments with N(0, 0.02^2) jitter",
    "cfg4": "3D Gaussian-splat growth, mixture of 4 isotropic Gaussians (sigma U[0.05, 0.2])",
    "cfg5": "3D stress, mixture of 8 Gaussians (log sigma U[log 0.01, log 0.2])",
}

# Mean-neighbour-calibrated radii for the seeded full-size clouds.
CALIBRATED_H = {
    "cfg1": 0.06921905279159546,
    "cfg2": 1.0 / 47.0,  # periodic: h must tile the unit box (calibrated 0.02115)
    "cfg3": 0.06505652517080307,
    "cfg4": 0.028674138709902763,
    "cfg5": 0.0026222667656838894,
}


def _disk(rng, n):
    r = np.sqrt(rng.random(n))
    t = 2 * np.pi * rng.random(n)
    return np.stack([r * np.cos(t), r * np.sin(t)], -1)


def _segments(rng, n):
    k = int(rng.integers(3, 7))
    a = rng.uniform(-1, 1, (k, 2))
    b = rng.uniform(-1, 1, (k, 2))
    lens = np.linalg.norm(b - a, axis=1)
    u = rng.random(n) * lens.sum()
    edges = np.cumsum(lens)
    seg = np.minimum(np.searchsorted(edges, u, side="right"), k - 1)
    t = (u - (edges[seg] - lens[seg])) / np.maximum(lens[seg], 1e-12)
    pts = a[seg] + t[:, None] * (b[seg] - a[seg])
    return pts + rng.normal(0.0, 0.02, (n, 2))


def _gmm(rng, n, k, sig_lo, sig_hi, log_sigma):
    means = rng.uniform(-0.5, 0.5, (k, 3))
    if log_sigma:
        sig = np.exp(rng.uniform(math.log(sig_lo), math.log(sig_hi), k))
    else:
        sig = rng.uniform(sig_lo, sig_hi, k)
    comp = np.repeat(np.arange(k), n // k)
    comp = np.concatenate([comp, rng.integers(0, k, n - comp.size)])
    rng.shuffle(comp)
    return means[comp] + rng.normal(0.0, 1.0, (n, 3)) * sig[comp][:, None]


def raw_points(name, scale=1.0, seed=SEED):
    """Positions (B, N, D) float64 and (B, N, C) states for a configuration.
    ``scale`` < 1 shrinks N (tests use reduced clouds of the same shape)."""
    rng = np.random.default_rng(seed)
    if name == "cfg1":
        B, N, C = 1, max(16, int(4096 * scale)), 16
        x = _disk(rng, N)[None]
    elif name == "cfg2":
        B, N, C = 4, max(16, int(16384 * scale)), 12
        x = rng.random((B, N, 2))
    elif name == "cfg3":
        B, N, C = max(1, int(64 * min(1.0, scale * 4))), 512, 32
        x = np.stack([_segments(rng, N) for _ in range(B)])
    elif name == "cfg4":
        B, N, C = 1, max(64, int(65536 * scale)), 32
        x = _gmm(rng, N, 4, 0.05, 0.2, False)[None]
    elif name == "cfg5":
        B, N, C = 1, max(64, int(1048576 * scale)), 16
        x = _gmm(rng, N, 8, 0.01, 0.2, True)[None]
    else:
        raise KeyError(name)
    s = rng.standard_normal((B, N, C))
    return x, s


def _pack(x):
    B, N, D = x.shape
    if D == 2:
        return x.astype(np.float32)
    out = np.zeros((B, N, 4), dtype=np.float32)
    out[..., :3] = x
    return out


def grid_for(x, h, periodic_side=None):
    """Cells per axis.  Periodic: the box side over h.  Clamped: the
    origin-centred grid covering the 99.9th percentile of |x| per axis; the
    remaining outliers are clamped into border cells, which keeps every pair
    closer than h in adjacent cells, so results are unchanged."""
    D = x.shape[-1]
    if periodic_side is not None:
        g = int(round(periodic_side / h))
        return (g,) * D
    ext = np.quantile(np.abs(x).reshape(-1, D), 0.999, axis=0)
    return tuple(int(2 * math.ceil(e / h) + 2) for e in ext)


def mean_neighbours(x, h, periodic_side=None):
    """Mean count of pairs with |r| < h (self included) over all clouds."""
    from scipy.spatial import cKDTree
    tot, n = 0, 0
    for cloud in x:
        pts = cloud
        if periodic_side is not None:
            pts = np.mod(cloud, periodic_side)
            tree = cKDTree(pts, boxsize=periodic_side)
        else:
            tree = cKDTree(pts)
        r = np.nextafter(h, 0)
        tot += tree.count_neighbors(tree, r)
        n += cloud.shape[0]
    return tot / n


def calibrate(name, scale=1.0, iters=40):
    x, _ = raw_points(name, scale)
    side = 1.0 if name == "cfg2" else None
    target = TARGETS[name]
    lo, hi = 1e-5, 1.0
    for _ in range(iters):
        mid = math.sqrt(lo * hi)
        if mean_neighbours(x, mid, side) < target:
            lo = mid
        else:
            hi = mid
    return float(np.float32(hi))


def make(name, scale=1.0, seed=SEED, h=None, mode="grid"):
    """Build a :class:`Workload`.  ``h`` defaults to the calibrated radius for
    full-size clouds; reduced clouds get h scaled to keep the neighbour count.
    ``mode="particle"`` gives the reference's particle (Morton) mode, whose
    grid must be cubic with a power-of-two side of at most 1024 cells
    (sphops/sph.py:69-71): the grid-mode extent rounded up (clamped clouds
    only; a periodic box fixes its side)."""
    x, s = raw_points(name, scale, seed)
    D = x.shape[-1]
    if h is None:
        h = CALIBRATED_H[name]
        if h is None:
            h = calibrate(name, 1.0)
        N = x.shape[1]
        full = {"cfg1": 4096, "cfg2": 16384, "cfg3": 512, "cfg4": 65536, "cfg5": 1048576}[name]
        if name == "cfg2":
            # the periodic unit box must hold a whole number of cells of side h:
            # fewer particles get fewer, wider cells at the same mean count
            if N != full:
                h = 1.0 / max(3, round(47 * math.sqrt(N / full)))
        else:
            h = float(np.float32(h * (full / N) ** (1.0 / D)))
    periodic = name == "cfg2"
    gs = grid_for(x, h, 1.0 if periodic else None)
    maxp = 32 if name in ("cfg1", "cfg2") else 64
    if mode == "particle":
        if periodic:
            raise ValueError(f"{name}: particle mode needs a power-of-two periodic box; not generated")
        side = 1
        while side < max(gs):
            side *= 2
        if side > 1024:
            raise ValueError(f"{name}: particle mode needs at most 1024 cells per axis, the cloud needs {max(gs)}")
        gs = (side,) * D
    elif mode != "grid":
        raise ValueError(f"unknown mode {mode!r}")
    return Workload(name, _pack(x), s.astype(np.float32), h, gs, periodic, maxp, mode)


if __name__ == "__main__":
    import sys
    if "--calibrate" in sys.argv:
        for nm in ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5"):
            hh = calibrate(nm)
            x, _ = raw_points(nm)
            side = 1.0 if nm == "cfg2" else None
            print(nm, repr(hh), "mean", mean_neighbours(x, hh, side), "grid", grid_for(x, hh, side), flush=True)
