"""Pins of the splatting oracle (oracle/splatting.py) on the CPU: the
particle-major restatement of utils/splatting.py against an independent
pixel-major evaluation, weight conservation, the symmetry of a centred
splat, the y_up mirror, and gradcheck."""
import math

import numpy as np
import pytest
import torch

from oracle import splatting as S


def particles(n, img_size, r, lo, hi, seed, ncolor=3, margin=3):
    """Positions whose pixel coordinates have fractional parts in [0.05,
    0.95] (floor is stable under rounding), some outside the image."""
    rng = np.random.default_rng(seed)
    cell = rng.integers(-r - margin, img_size + r + margin, size=(n, 2))
    pos = cell + rng.uniform(0.05, 0.95, size=(n, 2))
    x = pos / (img_size - 1) * (hi - lo) + lo
    color = rng.uniform(0, 1, size=(n, ncolor))
    return torch.tensor(x), torch.tensor(color)


CASES = [
    dict(img_size=32, sigma=1.0, pixel_size=2.0 / 16, normalize_color=True, y_up=False),
    dict(img_size=40, sigma=1.0, pixel_size=2.0 / 20, normalize_color=True, y_up=True),
    dict(img_size=24, sigma=1.3, normalize_color=False, y_up=False),
]


def _radius(kw):
    s = kw["sigma"] * kw["img_size"] * kw.get("pixel_size", 2.0 / 128.0) / 2.0 if kw["normalize_color"] else \
        kw["sigma"]
    return max(1, math.ceil(5 * s))


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_particle_major_equals_pixel_major(ci):
    kw = CASES[ci]
    x, c = particles(60, kw["img_size"], _radius(kw), -1.0, 1.0, seed=ci, ncolor=5)
    a = S.splat(x, c, **kw)
    b = S.splat_pixel_major(x, c, **kw)
    assert torch.allclose(a, b, rtol=1e-12, atol=1e-15)
    assert a[..., 3].sum() > 0


def test_weight_conservation():
    kw = dict(img_size=48, sigma=1.0, pixel_size=2.0 / 24, normalize_color=True)
    r = _radius(kw)
    rng = np.random.default_rng(2)
    pos = rng.uniform(r + 1, 48 - r - 2, size=(30, 2))  # every patch inside the image
    x = torch.tensor(pos / 47 * 2.0 - 1.0)
    c = torch.tensor(rng.uniform(0, 1, size=(30, 3)))
    img = S.splat(x, c, **kw)
    K = (48 * (2.0 / 24) / 2.0) ** 2
    assert abs(float(img[..., 3].sum()) - 30 * K) < 1e-6 * 30 * K
    assert torch.allclose(img[..., :3].sum(dim=(0, 1)), K * c.sum(0), rtol=1e-7)


def test_centred_particle_symmetry_and_peak():
    H, kw = 33, dict(sigma=1.0, pixel_size=2.0 / 16, normalize_color=True, lo=0.0, hi=32.0)
    x = torch.tensor([[16.0, 16.0]], dtype=torch.float64)  # pos = x exactly: pixel 16, frac 0
    img = S.splat(x, torch.ones(1, 3, dtype=torch.float64), img_size=H, **kw)[..., 3]
    assert torch.allclose(img, img.T, rtol=0, atol=1e-15)
    assert torch.allclose(img, img.flip(0), rtol=0, atol=1e-15)
    assert torch.allclose(img, img.flip(1), rtol=0, atol=1e-15)
    sig = 1.0 * H * (2.0 / 16) / 32.0
    r = max(1, math.ceil(5 * sig))
    d = torch.arange(-r, r + 1, dtype=torch.float64)
    S1 = torch.exp(-d ** 2 / (2 * sig * sig)).sum()
    K = (H * (2.0 / 16) / 32.0) ** 2
    assert abs(float(img[16, 16]) - K / (1e-8 + float(S1) ** 2)) < 1e-12


def test_y_up_mirrors_rows():
    H, kw = 65, dict(sigma=0.9, normalize_color=False, lo=0.0, hi=64.0)
    rng = np.random.default_rng(8)
    x = torch.tensor(rng.integers(0, 65, size=(20, 2)).astype(np.float64))  # integer pixel positions
    c = torch.tensor(rng.uniform(0, 1, size=(20, 3)))
    up = S.splat(x, c, img_size=H, y_up=True, **kw)
    down = S.splat(x, c, img_size=H, y_up=False, **kw)
    assert torch.allclose(up, down.flip(0), rtol=0, atol=1e-15)


def test_gradcheck():
    kw = CASES[0]
    x, c = particles(6, kw["img_size"], _radius(kw), -1.0, 1.0, seed=9, ncolor=4)
    x.requires_grad_(True)
    c.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: S.splat(a, b, **kw), (x, c))
