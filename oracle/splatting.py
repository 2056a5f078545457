"""2D Gaussian splatting, restated in torch (TEST INFRASTRUCTURE ONLY).

``splat`` follows ``utils/splatting.py:6-92`` (``splat_particles``): pixel
coordinates pos = (x - lo) / (hi - lo) * (img_size - 1) (y flipped with
y_up), sigma converted to pixels when normalize_color, a (2r+1)^2 patch with
r = max(1, ceil(5 sigma)) around floor(pos), weights exp(-|offset - frac|^2 /
(2 sigma^2)) normalised to sum to (img_size * pixel_size / (hi - lo))^2 over
the whole patch, and the in-image pixels accumulated as [w * rgb, w] with rgb
the last three colour channels.  It accumulates with ``index_add_`` on the
CPU, which is deterministic.  Works in any dtype (the tests use float64) and
is differentiable with torch.autograd.

``splat_pixel_major`` computes the same image the other way round, per pixel
over all particles, with no patch indexing or scatter: the independent check
of the restatement's index arithmetic.
"""
import math

import torch


def _setup(x, img_size, sigma, lo, hi, normalize_color, y_up, pixel_size):
    pos = (x - lo) / (hi - lo) * (img_size - 1)
    if y_up:
        pos = torch.stack([pos[:, 0], (img_size - 1) - pos[:, 1]], dim=1)
    if normalize_color:
        sigma = sigma * img_size * pixel_size / (hi - lo)
    radius = max(1, math.ceil(5 * float(sigma)))
    return pos, sigma, radius


def splat(x, color, img_size=256, sigma=2.0, lo=-1.0, hi=1.0, normalize_color=True, y_up=False,
          pixel_size=2.0 / 128.0):
    """(img_size, img_size, 4) image [r, g, b, density] of particles x (N, 2)
    with colours color (N, >= 3) (utils/splatting.py:6-92)."""
    pos, sigma, r = _setup(x, img_size, sigma, lo, hi, normalize_color, y_up, pixel_size)
    offs = torch.arange(-r, r + 1, dtype=torch.int64)
    oy, ox = torch.meshgrid(offs, offs, indexing="ij")
    ox, oy = ox.reshape(-1), oy.reshape(-1)
    base = torch.floor(pos)
    frac = pos - base
    cx, cy = base[:, 0].long(), base[:, 1].long()
    ix = cx[:, None] + ox[None, :]
    iy = cy[:, None] + oy[None, :]
    inside = (ix >= 0) & (ix < img_size) & (iy >= 0) & (iy < img_size)
    ax = ox[None, :] - frac[:, 0:1]
    ay = oy[None, :] - frac[:, 1:2]
    g = torch.exp(-(ax ** 2 + ay ** 2) / (2 * sigma * sigma))
    if normalize_color:
        g = g / (1e-8 + g.sum(dim=-1, keepdim=True))
        g = g * (img_size * pixel_size / (hi - lo)) ** 2.0
    rgb = color[..., -3:]
    flat = (iy * img_size + ix)[inside]
    w = g[inside]
    c = rgb[:, None, :].expand(-1, ox.numel(), -1)[inside]
    out = torch.zeros(img_size * img_size, 4, dtype=x.dtype)
    out = out.index_add(0, flat, torch.cat([c * w[:, None], w[:, None]], dim=1))
    return out.view(img_size, img_size, 4)


def splat_pixel_major(x, color, img_size=256, sigma=2.0, lo=-1.0, hi=1.0, normalize_color=True, y_up=False,
                      pixel_size=2.0 / 128.0):
    """The same image, pixel by pixel: pixel (row i, column j) sums over the
    particles whose patch square around floor(pos) contains it."""
    pos, sigma, r = _setup(x, img_size, sigma, lo, hi, normalize_color, y_up, pixel_size)
    base = torch.floor(pos)
    frac = pos - base
    two_s2 = 2 * sigma * sigma
    # each particle's full-patch weight total, as a separable product
    d = torch.arange(-r, r + 1, dtype=x.dtype)
    sx = torch.exp(-((d[None, :] - frac[:, 0:1]) ** 2) / two_s2).sum(-1)
    sy = torch.exp(-((d[None, :] - frac[:, 1:2]) ** 2) / two_s2).sum(-1)
    kk = (img_size * pixel_size / (hi - lo)) ** 2.0
    norm = (1e-8 + sx * sy) / kk if normalize_color else torch.ones_like(sx)
    cols = torch.arange(img_size, dtype=x.dtype)
    out = torch.zeros(img_size, img_size, 4, dtype=x.dtype)
    rgb = color[..., -3:]
    for i in range(img_size):
        oy = i - base[:, 1]
        ok_y = (oy >= -r) & (oy <= r)
        if not bool(ok_y.any()):
            continue
        ox = cols[None, :] - base[ok_y, 0:1]
        ok = (ox >= -r) & (ox <= r)
        gy = (oy[ok_y] - frac[ok_y, 1])[:, None]
        gx = ox - frac[ok_y, 0:1]
        w = torch.where(ok, torch.exp(-(gx ** 2 + gy ** 2) / two_s2), torch.zeros((), dtype=x.dtype))
        w = w / norm[ok_y, None]
        out[i, :, :3] = (w[:, :, None] * rgb[ok_y][:, None, :]).sum(0)
        out[i, :, 3] = w.sum(0)
    return out
