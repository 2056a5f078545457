"""Differentiable 2D Gaussian splatting (utils/splatting.py:6-117 of the
reference) on the HIP kernels of libsphops_hip.so.

``splat_particles``, ``splat_particles_batch`` and ``splat_particles_sections``
take the reference's arguments and return its images ((H, W, 4) or
(images, H, W, 4), channels [r, g, b, density]).  All images of a call are
one launch.  The forward gathers per 16 x 16 tile in ascending particle order
and the backward sums per particle, so results are deterministic (the
reference's scatter_add_ is not).  Positions and colours are float32 on the
GPU; only the last three colour channels receive a gradient, as in the
reference.
"""
import ctypes

import torch

from .sphops import _native

_lib = _native.lib


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


class Splat(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, color, starts, img_size, sigma, lo, hi, normalize_color, y_up, pixel_size):
        if x.dtype != torch.float32 or color.dtype != torch.float32:
            raise TypeError("splatting takes float32 positions and colours")
        if not x.is_cuda or x.device != color.device or starts.device != x.device:
            raise TypeError("x, color and the section starts must be on one GPU")
        if x.dim() != 2 or x.shape[1] != 2 or color.dim() != 2 or color.shape[0] != x.shape[0]:
            raise RuntimeError(f"x must be (N, 2) and color (N, >= 3); got {tuple(x.shape)}, {tuple(color.shape)}")
        x, color = x.contiguous(), color.contiguous()
        images = starts.numel() - 1
        out = torch.empty(images, img_size, img_size, 4, device=x.device)
        args = (x.shape[0], color.shape[1], img_size, float(sigma), float(lo), float(hi), int(bool(normalize_color)),
                int(bool(y_up)), float(pixel_size))
        work = torch.empty(max(1, _lib.sphops_splat_workspace_bytes(x.shape[0])), dtype=torch.uint8, device=x.device)
        st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(x.device.index))
        _native.check(_lib.sphops_splat_forward(_ptr(x), _ptr(color), _ptr(starts), images, *args, _ptr(out),
                                                _ptr(work), st))
        ctx.save_for_backward(x, color, starts)
        ctx.args = args
        return out

    @staticmethod
    def backward(ctx, d_out):
        x, color, starts = ctx.saved_tensors
        d_out = d_out.contiguous()
        d_x = torch.empty_like(x)
        d_color = torch.empty_like(color)
        st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(x.device.index))
        _native.check(_lib.sphops_splat_backward(_ptr(x), _ptr(color), _ptr(starts), starts.numel() - 1, *ctx.args,
                                                 _ptr(d_out), _ptr(d_x), _ptr(d_color), st))
        return d_x, d_color, None, None, None, None, None, None, None, None


def _starts(sizes, device):
    s = torch.zeros(len(sizes) + 1, dtype=torch.int64)
    s[1:] = torch.cumsum(torch.as_tensor(sizes, dtype=torch.int64), 0)
    return s.to(device=device, dtype=torch.int32)


def _kw(img_size=256, sigma=2.0, lo=-1.0, hi=1.0, normalize_color=True, y_up=False, pixel_size=2.0 / 128.0):
    return img_size, sigma, lo, hi, normalize_color, y_up, pixel_size


def splat_particles(x, color, img_size=256, sigma=2.0, lo=-1.0, hi=1.0, normalize_color=True, y_up=False,
                    pixel_size=2.0 / 128.0):
    """(img_size, img_size, 4) image of particles x (N, 2) with colours
    color (N, >= 3) (utils/splatting.py:6-92)."""
    starts = _starts([x.shape[0]], x.device)
    return Splat.apply(x, color, starts, *_kw(img_size, sigma, lo, hi, normalize_color, y_up, pixel_size))[0]


def splat_particles_batch(x, color, **kwargs):
    """(B, H, W, 4) images of x (B, P, 2), color (B, P, >= 3)
    (utils/splatting.py:95-103)."""
    B, P, _ = x.shape
    assert color.shape[:2] == (B, P)
    starts = _starts([P] * B, x.device)
    return Splat.apply(x.reshape(B * P, 2), color.reshape(B * P, -1), starts, *_kw(**kwargs))


def splat_particles_sections(x, color, sections, **kwargs):
    """One (H, W, 4) image per block of rows of x (N, 2) and color (N, >= 3),
    blocks as torch.split(x, sections) makes them (utils/splatting.py:106-110):
    a list of sizes, or one block size (the last block may be shorter)."""
    N = x.shape[0]
    if isinstance(sections, int):
        if sections <= 0:
            raise RuntimeError("split size must be positive")
        sizes = [sections] * (N // sections) + ([N % sections] if N % sections else [])
    else:
        sizes = [int(s) for s in sections]
        if sum(sizes) != N:
            raise RuntimeError("sections must add up to the number of particles")
    starts = _starts(sizes, x.device)
    return Splat.apply(x, color, starts, *_kw(**kwargs))
