"""Writes the golden fixtures in tests/golden/ (run: python tests/golden/make_golden.py).

The reference holds no stored vectors for sphops: its test.py draws random
data at run time and compares the CUDA path with torch_sph (sphops/test.py:
88-154, 595-627).  These fixtures freeze small cases of that validation
matrix, so the GPU tests can check against stored values without rerunning
the oracle, and the CPU tests check that the oracle still reproduces them.

* ``ref2d_clamped.npz`` / ``ref2d_periodic.npz``: the test.py input recipe at
  small size (B = 1, N = 96, C = 4, 2D, 16 x 16 cells, eps = 0.1, positions
  U[-1, 1)^2 overflowing the clamped grid, masses rand + 1e-3, states and
  upstream gradients N(0, 1)).  Stored: the inputs, the binning (bit-exact
  integers), and, on the oracle's binned arrays, float64 operator values and
  gradients with their magnitude sums (the tolerance scale).
* ``pair3d.npz``: two particles in 3D at distance d < h, with density,
  density gradient and spiky values from the closed forms
  W = (h^2 - d^2)^3 and grad W_spiky = 3 (h - d)^2 / d * r, evaluated here in
  float64 from the textbook normalisations 315 / (64 pi h^9), 15 / (pi h^6).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import binning, neighbors, sph  # noqa: E402


def pack2d(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def ref2d(periodic, seed):
    """Inputs and oracle outputs of one small reference-style case."""
    rng = np.random.default_rng(seed)
    B, N, C, D, G, eps = 1, 96, 4, 2, 16, 0.1
    x = pack2d((rng.random((B, N, D)) - 0.5) * 2.0)
    s = rng.standard_normal((B, N, C)).astype(np.float32)
    m = (rng.random((B, N)) + 1e-3).astype(np.float32)
    up = {
        "g_rho": rng.standard_normal((B, N)).astype(np.float32),
        "g_blur": rng.standard_normal((B, N, C)).astype(np.float32),
        "g_grad": rng.standard_normal((B, N, C, D)).astype(np.float32),
        "g_dg": rng.standard_normal((B, N, D)).astype(np.float32),
    }
    grid = (G, G)
    ob = binning.instantiate(x, grid, eps, periodic, "grid", 64)
    xb, sb, mb = binning.bin_particles(x, s, m, ob["permutation"])
    spec = neighbors.GridSpec(grid, eps, periodic, "grid", 64)
    ctx = sph.Context(neighbors.candidate_pairs(xb, ob["bin_offsets"], spec), spec)
    mf = mb.reshape(-1).astype(np.float64)
    sf = sb.reshape(-1, C).astype(np.float64)
    rho, rho_mag = sph.density(ctx, mf)
    out = dict(x=x, s=s, m=m, grid=np.array(grid), eps=np.float64(eps), periodic=np.bool_(periodic),
               permutation=ob["permutation"], bin_offsets=ob["bin_offsets"], block_info=ob["block_info"],
               total_blocks=np.int64(ob["total_blocks"]), xb=xb, sb=sb, mb=mb, **up)
    out["count"] = sph.count(ctx)[0]
    out["rho"], out["rho_mag"] = rho, rho_mag
    out["dgrad"], out["dgrad_mag"] = sph.density_gradient(ctx, mf)
    out["blur"], out["blur_mag"] = sph.blur(ctx, mf, rho, sf)
    out["grad"], out["grad_mag"] = sph.gradient(ctx, mf, rho, sf)
    (out["b_density_dx"], out["b_density_dx_mag"]) = sph.density_backward(
        ctx, mf, up["g_rho"].reshape(-1).astype(np.float64))
    (out["b_dgrad_dx"], out["b_dgrad_dx_mag"]) = sph.density_gradient_backward(
        ctx, mf, up["g_dg"].reshape(-1, D).astype(np.float64))
    for name, fn, g in (("b_blur", sph.blur_backward, up["g_blur"].reshape(-1, C)),
                        ("b_grad", sph.gradient_backward, up["g_grad"].reshape(-1, C, D))):
        (dx, dxm), (ds, dsm), (dr, drm) = fn(ctx, mf, rho, sf, g.astype(np.float64))
        out.update({f"{name}_dx": dx, f"{name}_dx_mag": dxm, f"{name}_ds": ds, f"{name}_ds_mag": dsm,
                    f"{name}_drho": dr, f"{name}_drho_mag": drm})
    return out


def pair3d():
    """Two particles, closed forms only (no oracle code)."""
    h = 0.25
    d = 0.1
    direction = np.array([2.0, -1.0, 2.0]) / 3.0
    x0 = np.array([0.01, 0.02, -0.03])
    x1 = x0 + d * direction
    m = np.array([0.7, 1.3])
    c6 = 315.0 / (64.0 * np.pi * h ** 9)
    cs = 15.0 / (np.pi * h ** 6)
    W0 = h ** 6                       # self term (h^2 - 0)^3
    W = (h * h - d * d) ** 3
    rho = c6 * np.array([m[0] * W0 + m[1] * W, m[1] * W0 + m[0] * W])
    k = 3.0 * (h - d) ** 2 / d        # spiky magnitude per unit displacement
    r01 = x1 - x0                     # x_j - x_i for i = 0
    dgrad = cs * np.stack([m[1] * k * r01, m[0] * k * (-r01)])
    x = np.zeros((1, 2, 4), np.float32)
    x[0, :, :3] = np.stack([x0, x1]).astype(np.float32)
    return dict(x=x, m=m.astype(np.float32)[None], h=np.float64(h), rho=rho, dgrad=dgrad, grid=np.array([8, 8, 8]))


def main():
    np.savez_compressed(os.path.join(HERE, "ref2d_clamped.npz"), **ref2d(False, 20240611))
    np.savez_compressed(os.path.join(HERE, "ref2d_periodic.npz"), **ref2d(True, 20240612))
    np.savez_compressed(os.path.join(HERE, "pair3d.npz"), **pair3d())
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
