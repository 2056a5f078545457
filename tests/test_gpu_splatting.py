"""Splatting kernels (npa_amd.splatting) against the oracle restatement of
utils/splatting.py (oracle/splatting.py, float64 on the CPU): images and the
gradients with respect to positions and colours, for single images,
batches and ragged sections (with an empty one), normalised or not, y_up,
particles partly outside the image; and run-to-run determinism."""
import math

import numpy as np
import pytest
import torch

from oracle import splatting as S
from test_oracle_splatting import particles

pytestmark = pytest.mark.gpu

CASES = [
    dict(img_size=64, sigma=1.0, pixel_size=2.0 / 32, normalize_color=True, y_up=False),
    dict(img_size=256, sigma=2.0, normalize_color=True, y_up=True),  # the reference's defaults, y flipped: r = 20
    dict(img_size=50, sigma=1.5, normalize_color=False, y_up=False, lo=-1.5, hi=2.0),
    dict(img_size=17, sigma=1.0, pixel_size=2.0 / 8, normalize_color=True, y_up=True),  # tiles cut by the edge
    dict(img_size=32, sigma=0.1, normalize_color=False, y_up=True),  # the smallest patch, r = 1
    dict(img_size=96, sigma=12.0, normalize_color=False, y_up=False),  # r = 60: patches wider than tiles
    dict(img_size=64, sigma=3.0, pixel_size=2.0 / 64, normalize_color=True, y_up=False, lo=-3.0, hi=1.0),
]
PARTICLES = {5: 200}  # fewer particles where the patch is large (the float64 oracle is dense)
# sigma = 0.1 px: the exponent -|offset - frac|^2 / (2 sigma^2) reaches -50 within a
# pixel, so fp32 rounding of the position (about 2e-6 px at 30 px) moves a weight by
# up to 1e-4 of itself, in the reference's fp32 arithmetic as much as here
IMAGE_ATOL = {4: 2e-5}


def _radius(kw):
    span = kw.get("hi", 1.0) - kw.get("lo", -1.0)
    s = kw["sigma"] * kw["img_size"] * kw.get("pixel_size", 2.0 / 128.0) / span if kw["normalize_color"] else \
        kw["sigma"]
    return max(1, math.ceil(5 * s))


def _close(name, got, ref, rtol=2e-5, atol=1e-6):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    err = np.abs(got - ref)
    bad = err > rtol * np.abs(ref) + atol * (scale + 1e-30)
    assert not bad.any(), f"{name}: {bad.sum()} of {bad.size} off, max err {err.max():.3g} (max |ref| {scale:.3g})"


def _check(images_fn, oracle_images, x, c, seed, image_atol=1e-6):
    xg = x.float().cuda().requires_grad_(True)
    cg = c.float().cuda().requires_grad_(True)
    img = images_fn(xg, cg)
    xr = xg.detach().double().cpu().requires_grad_(True)
    cr = cg.detach().double().cpu().requires_grad_(True)
    ref = oracle_images(xr, cr)
    assert img.shape == ref.shape
    _close("image", img.detach().cpu(), ref.detach(), atol=image_atol)
    up = torch.randn(ref.shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    gx, gc = torch.autograd.grad(img, (xg, cg), up.float().cuda())
    rx, rc = torch.autograd.grad(ref, (xr, cr), up)
    _close("dL/dx", gx.cpu(), rx, rtol=1e-4, atol=1e-5)
    _close("dL/dcolor", gc.cpu(), rc, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_single_image(ci):
    from npa_amd import splatting as SP
    kw = CASES[ci]
    x, c = particles(PARTICLES.get(ci, 700), kw["img_size"], _radius(kw), kw.get("lo", -1.0), kw.get("hi", 1.0),
                     seed=ci, ncolor=3 + ci % 5)
    _check(lambda a, b: SP.splat_particles(a, b, **kw), lambda a, b: S.splat(a, b, **kw), x, c, ci,
           image_atol=IMAGE_ATOL.get(ci, 1e-6))


def test_batch_and_sections():
    from npa_amd import splatting as SP
    kw = CASES[0]
    r = _radius(kw)
    x, c = particles(3 * 300, kw["img_size"], r, -1.0, 1.0, seed=11, ncolor=3)
    _check(lambda a, b: SP.splat_particles_batch(a.view(3, 300, 2), b.view(3, 300, 3), **kw),
           lambda a, b: torch.stack([S.splat(a[i * 300:(i + 1) * 300], b[i * 300:(i + 1) * 300], **kw)
                                     for i in range(3)]), x, c, 1)
    sections = [250, 0, 650]
    bounds = np.cumsum([0] + sections)
    _check(lambda a, b: SP.splat_particles_sections(a, b, sections, **kw),
           lambda a, b: torch.stack([S.splat(a[bounds[i]:bounds[i + 1]], b[bounds[i]:bounds[i + 1]], **kw)
                                     for i in range(3)]), x, c, 2)
    # one block size, the last block shorter (torch.split semantics)
    _check(lambda a, b: SP.splat_particles_sections(a, b, 400, **kw),
           lambda a, b: torch.stack([S.splat(a[i:i + 400], b[i:i + 400], **kw) for i in (0, 400, 800)]), x, c, 3)


def test_deterministic_and_empty():
    from npa_amd import splatting as SP
    kw = CASES[1]
    x, c = particles(5000, kw["img_size"], _radius(kw), -1.0, 1.0, seed=5)
    xg, cg = x.float().cuda(), c.float().cuda()
    a = SP.splat_particles(xg, cg, **kw)
    b = SP.splat_particles(xg, cg, **kw)
    assert torch.equal(a, b)
    far = torch.full((10, 2), 50.0, device="cuda")  # every patch off the image
    assert torch.count_nonzero(SP.splat_particles(far, cg[:10], **kw)) == 0
    assert torch.count_nonzero(SP.splat_particles(far[:0], cg[:0], **kw)) == 0
