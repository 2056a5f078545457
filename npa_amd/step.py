"""NPA.forward and step_euler / step_euler_trace with fused kernels
(models/npa.py:123-241 of the reference).

``step_euler(model, x, s, grid, dt, update_prob, intermediate, noise_std)``
returns what the reference's ``step_euler`` returns for an ``NPA`` model:
perception through ``npa_amd.perceive.perceive`` (fused features), the
model's own MLP (``model.model``; its weight gradients through
``npa_amd.mlp``'s row-chunked kernel), then one HIP kernel
for the position-step scaling of NPA.forward, the update mask, the zero
padding of 3D positions, the Euler update, the optional noise and the
per-particle |dx| of the ``intermediate`` stats; one kernel maps the
gradient back to the MLP output.  Random numbers are drawn as the reference
draws them (``torch.rand(B, N, 1)`` for the mask, then ``torch.randn_like(x)``
for the noise), so a seeded run draws the same mask and noise.

``model`` is the reference's ``NPA`` module (or any module with its
attributes: spatial_dims, eps0, alpha, model, the four perception flags,
stopgrad_pos, stopgrad_state); ``model.last_snapshot`` is set as
NPA.forward sets it.
"""
import ctypes
import math

import torch

from .mlp import mlp
from .perceive import buffer_value, perceive
from .sphops import _native, unbin_particles

_lib = _native.lib


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _check(t, what):
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise TypeError(f"{what} must be a contiguous float32 tensor")


class EulerUpdate(torch.autograd.Function):
    """(x_out, s_out, dx_norm) from the MLP output y and the binned x, s
    (models/npa.py:125-133 and 189-200)."""

    @staticmethod
    def forward(ctx, y, x_bin, s_bin, mask, noise, dim, alpha, eps, dt, noise_std):
        B, N, P = x_bin.shape
        C = s_bin.shape[-1]
        for t, what in ((y, "y"), (x_bin, "x_bin"), (s_bin, "s_bin")):
            _check(t, what)
        if y.shape != (B, N, dim + C):
            raise RuntimeError(f"y must have shape {(B, N, dim + C)}, got {tuple(y.shape)}")
        for t, shape, what in ((mask, (B, N, 1), "mask"), (noise, (B, N, P), "noise")):
            if t is not None:
                _check(t, what)
                if t.shape != shape:
                    raise RuntimeError(f"{what} must have shape {shape}, got {tuple(t.shape)}")
        x_out = torch.empty_like(x_bin)
        s_out = torch.empty_like(s_bin)
        dx_norm = torch.empty(B, N, device=y.device)
        st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(y.device.index))
        _native.check(_lib.sphops_euler_update_forward(
            dim, P, _ptr(y), _ptr(x_bin), _ptr(s_bin), _ptr(mask), _ptr(noise), _ptr(x_out), _ptr(s_out),
            _ptr(dx_norm), B * N, C, alpha, eps, dt, noise_std, math.sqrt(dt), st))
        ctx.save_for_backward(y, mask)
        ctx.args = (dim, P, C, alpha, eps, dt)
        return x_out, s_out, dx_norm

    @staticmethod
    def backward(ctx, d_x, d_s, d_n):
        y, mask = ctx.saved_tensors
        dim, P, C, alpha, eps, dt = ctx.args
        B, N = y.shape[:2]
        d_y = None
        if ctx.needs_input_grad[0]:
            d_x = d_x.contiguous() if d_x is not None else None
            d_s = d_s.contiguous() if d_s is not None else None
            d_n = d_n.contiguous() if d_n is not None else None
            d_y = torch.empty_like(y)
            st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(y.device.index))
            _native.check(_lib.sphops_euler_update_backward(
                dim, P, _ptr(y), _ptr(mask), _ptr(d_x), _ptr(d_s), _ptr(d_n), _ptr(d_y), B * N, C, alpha, eps, dt,
                st))
        return d_y, d_x, d_s, None, None, None, None, None, None, None


def _perceive(model, x, s, grid):
    return perceive(x, s, grid, model.eps0, model.state_grad, model.density_grad, model.log_norm_grad,
                    model.log_norm_density_grad, model.stopgrad_pos, model.stopgrad_state)


def _draws(x, update_prob, noise_std):
    B, N = x.shape[:2]
    mask = None
    if update_prob < 1.0:
        mask = (torch.rand(B, N, 1, device=x.device) < update_prob).float()
    noise = torch.randn_like(x) if noise_std > 0 else None
    return mask, noise


def _step(model, x, s, grid, dt, update_prob, noise_std):
    z, x_bin, s_bin, snapshot = _perceive(model, x, s, grid)
    model.last_snapshot = snapshot
    y = mlp(model.model, z).contiguous()
    mask, noise = _draws(x, update_prob, noise_std)
    alpha = buffer_value(model.alpha)
    x_new, s_new, dx_norm = EulerUpdate.apply(y, x_bin.contiguous(), s_bin.contiguous(), mask, noise,
                                              model.spatial_dims, alpha, float(grid.eps), float(dt),
                                              float(noise_std))
    return x_new, s_new, dx_norm, y, alpha


def step_euler(model, x, s, grid, dt=1.0, update_prob=0.5, intermediate=False, noise_std=0.0):
    """step_euler (models/npa.py:154-204): returns (x, s, stats) in binned
    order; stats = {"dx_norm": mean |dx|} when intermediate, else None."""
    x_new, s_new, dx_norm, _, _ = _step(model, x, s, grid, dt, update_prob, noise_std)
    stats = {"dx_norm": dx_norm.mean()} if intermediate else None
    return x_new, s_new, stats


def step_euler_trace(model, x, s, grid, dt=1.0, update_prob=0.5, noise_std=0.0, return_aux=False):
    """step_euler_trace (models/npa.py:207-241): the updated particles in the
    input order; with return_aux also dx and ds of NPA.forward, unbinned."""
    x_new, s_new, _, y, alpha = _step(model, x, s, grid, dt, update_prob, noise_std)
    x_trace, s_trace = unbin_particles(x_new, s_new, model.last_snapshot)
    if not return_aux:
        return x_trace, s_trace
    D = model.spatial_dims
    a = y[..., :D]
    dx_bin = alpha * a * float(grid.eps) / (1.0 + a.norm(dim=-1, keepdim=True))
    if dx_bin.shape[-1] != x.shape[-1]:
        dx_bin = torch.cat([dx_bin, torch.zeros_like(dx_bin[..., :1])], dim=-1)
    dx_trace, ds_trace = unbin_particles(dx_bin.contiguous(), y[..., D:].contiguous(), model.last_snapshot)
    return x_trace, s_trace, dx_trace, ds_trace


def step_euler_static(model, x, s, grid, dt=1.0, update_prob=0.5, channel_mask=None):
    """step_euler of the state-only model (models/static_npa.py:15-38):
    fused perception, the model's MLP giving ds only, positions unchanged
    (x_bin + 0), s = s_bin + dt * ds * mask; returns (x, s) in binned order.
    The update is a single elementwise expression, left to torch."""
    B, N, C = s.shape
    z, x_bin, s_bin, snapshot = _perceive(model, x, s, grid)
    model.last_snapshot = snapshot
    ds = mlp(model.model, z)
    mask = 1.0
    if update_prob < 1.0:
        mask = (torch.rand(B, N, 1, device=x.device) < update_prob).float()
    if channel_mask is not None:
        ds = ds * channel_mask
    return x_bin + 0, s_bin + dt * ds * mask
