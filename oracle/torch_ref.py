"""The reference's torch formulations of the paths around the perception
operators (oracle only: test and measurement infrastructure).

These restate, statement for statement, what the reference computes with torch
ops, so that bench_extras.py can time its fused kernels beside them on the same
GPU (the baseline leg of each measurement); the library never calls them:
* ``log_normalize``, ``perceive`` -- NPA.perceive's feature assembly
  (models/npa.py:83-137), all feature flags on, stopgrad_pos;
* ``euler`` -- NPA.forward's position-step scaling and step_euler's update
  (models/npa.py:125-133, 178-200);
* ``splat`` -- splat_particles (utils/splatting.py:6-92), torch scatter_add_.
The float64 CPU restatements the tests check against are oracle/perceive.py
and oracle/splatting.py.
"""
import math

import torch

import npa_amd.sphops as sp


def log_normalize(v):  # models/npa.py:83-85
    return torch.log(1.0 + v.norm(dim=-1, keepdim=True)) * torch.nn.functional.normalize(v, dim=-1)


def perceive(x, s, grid, eps0=0.1):  # models/npa.py:87-137, all flags on, stopgrad_pos
    B, N, C = s.shape
    eps = grid.eps
    with torch.no_grad():
        snap = grid.instantiate(x)
    x_bin, s_bin = sp.bin_particles(x, s, snap)
    xp = x_bin.detach()
    rho = sp.density(xp, snap)
    z = [s_bin, sp.blur(xp, rho, s_bin, snap)]
    coef = torch.tensor([eps], device=x.device) / torch.tensor([eps0], device=x.device)
    g = log_normalize(sp.gradient_hybrid(xp, rho, s_bin, snap) * coef)
    z.append(g.reshape(B, N, -1))
    gr = sp.density_gradient(xp, snap) * (coef ** (1 + grid.dim)) / N
    z.append(log_normalize(gr))
    return torch.cat(z, dim=-1), x_bin, s_bin, snap


def euler(y, x_bin, s_bin, D, alpha, eps, update_prob, dt=1.0):  # models/npa.py:125-133, 178-200
    B, N, _ = s_bin.shape
    dx = y[..., :D]
    dx = alpha * dx * eps / (1.0 + dx.norm(dim=-1, keepdim=True))
    ds = y[..., D:]
    dn = dx.norm(dim=-1).mean()
    m = (torch.rand(B, N, 1, device=y.device) < update_prob).float()
    if dx.shape[-1] != x_bin.shape[-1]:
        dx = torch.cat([dx, torch.zeros(B, N, 1, device=y.device)], dim=-1).contiguous()
    return x_bin + dt * dx * m, s_bin + dt * ds * m, dn


def splat(x, color, img_size, sigma, lo, hi, y_up, pixel_size):  # utils/splatting.py:6-92
    dev = x.device
    pos = (x - lo) / (hi - lo) * (img_size - 1)
    if y_up:
        pos = torch.stack([pos[:, 0], (img_size - 1) - pos[:, 1]], dim=1)
    sigma = sigma * img_size * pixel_size / (hi - lo)
    r = max(1, math.ceil(5 * float(sigma)))
    offs = torch.arange(-r, r + 1, device=dev, dtype=torch.int64)
    yy, xx = torch.meshgrid(offs, offs, indexing="ij")
    dx, dy = xx.reshape(-1), yy.reshape(-1)
    base = torch.floor(pos)
    cx, cy = base[:, 0].long(), base[:, 1].long()
    frac = pos - base
    x_idx = cx[:, None] + dx[None, :]
    y_idx = cy[:, None] + dy[None, :]
    mask = (x_idx >= 0) & (x_idx < img_size) & (y_idx >= 0) & (y_idx < img_size)
    g = torch.exp(-((dx[None, :] - frac[:, 0:1]) ** 2 + (dy[None, :] - frac[:, 1:2]) ** 2) / (2 * sigma * sigma))
    g = g / (1e-8 + torch.sum(g, dim=-1, keepdim=True))
    g = g * (img_size * pixel_size / (hi - lo)) ** 2.0
    flat = (y_idx * img_size + x_idx)[mask]
    w = g[mask]
    c = color[..., -3:][:, None, :].expand(-1, dx.numel(), -1)[mask, :]
    density = torch.zeros(img_size * img_size, 1, device=dev)
    rgb = torch.zeros(img_size * img_size, 3, device=dev)
    density.scatter_add_(0, flat[:, None], w[:, None])
    rgb.scatter_add_(0, flat[:, None].expand(-1, 3), c * w[:, None])
    return torch.cat([rgb, density], dim=1).view(img_size, img_size, 4)
