"""NPA.perceive with fused perception features (models/npa.py:87-137 of the
reference).

``perceive(x, s, grid, ...)`` returns what ``NPA.perceive`` returns,
``(z, x_bin, s_bin, snapshot)``, for the same flags.  The perception operators
are the drop-in ``npa_amd.sphops`` ones, called in the reference's order (so
their pass fusion applies); the features the reference then assembles with
torch elementwise ops and ``torch.cat`` (the eps/eps0 scaling, the
log-normalisation of models/npa.py:83-85, the density-gradient scaling by
coef^(1+D)/N) are built by one HIP kernel, and their gradient by another
(``sphops_perception_features_forward`` / ``_backward``).

Difference from the reference: its density-gradient branch uses ``coef``,
which it defines only in the state-gradient branch (models/npa.py:121-127), so
``state_grad=False, density_grad=True`` raises NameError there; here coef is
always defined.
"""
import ctypes

import numpy as np
import torch

from .sphops import _native
from .sphops import bin_particles, blur, density, density_gradient, gradient_hybrid

_lib = _native.lib

STATE_GRAD, LOG_NORM_GRAD, DENSITY_GRAD, LOG_NORM_DENSITY_GRAD = 1, 2, 4, 8


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(t):
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(t.device.index))


def buffer_value(t):
    """The float value of a one-element model buffer (eps0, alpha), read from
    the device once and remembered on the tensor object for its current
    version: reading a GPU tensor on the host synchronises, which would stall
    every step (and is not allowed while a HIP graph is being captured)."""
    if not torch.is_tensor(t):
        return float(t)
    hit = getattr(t, "_npa_host_value", None)
    if hit is not None and hit[0] == t._version:
        return hit[1]
    v = float(t.reshape(-1)[0])
    t._npa_host_value = (t._version, v)
    return v


def feature_width(C, D, flags):
    return 2 * C + (C * D if flags & STATE_GRAD else 0) + (D if flags & DENSITY_GRAD else 0)


class PerceptionFeatures(torch.autograd.Function):
    """z = [s, blur, LN(coef_s * grad_s), LN(coef_rho * grad_rho / total_mass)]
    (LN optional per flag), in one kernel; backward in one kernel."""

    @staticmethod
    def forward(ctx, s, blur_s, grad_s, grad_rho, dim, coef_s, coef_rho, total_mass, flags):
        B, N, C = s.shape
        for t in (s, blur_s, grad_s, grad_rho):
            if t is not None and (t.dtype != torch.float32 or not t.is_contiguous() or t.device != s.device):
                raise TypeError("perception features take contiguous float32 tensors on one device")
        z = torch.empty(B, N, feature_width(C, dim, flags), dtype=torch.float32, device=s.device)
        _native.check(_lib.sphops_perception_features_forward(
            dim, _ptr(s), _ptr(blur_s), _ptr(grad_s), _ptr(grad_rho), _ptr(z), B * N, C, coef_s, coef_rho,
            total_mass, flags, _stream(s)))
        ctx.save_for_backward(grad_s, grad_rho)
        ctx.args = (dim, coef_s, coef_rho, total_mass, flags, C)
        return z

    @staticmethod
    def backward(ctx, dz):
        grad_s, grad_rho = ctx.saved_tensors
        dim, coef_s, coef_rho, total_mass, flags, C = ctx.args
        dz = dz.contiguous()
        B, N = dz.shape[:2]
        need = ctx.needs_input_grad
        d_s = torch.empty(B, N, C, device=dz.device) if need[0] else None
        d_blur = torch.empty(B, N, C, device=dz.device) if need[1] else None
        d_gs = torch.empty(B, N, C, dim, device=dz.device) if need[2] and grad_s is not None else None
        d_gr = torch.empty(B, N, dim, device=dz.device) if need[3] and grad_rho is not None else None
        _native.check(_lib.sphops_perception_features_backward(
            dim, _ptr(dz), _ptr(grad_s), _ptr(grad_rho), _ptr(d_s), _ptr(d_blur), _ptr(d_gs), _ptr(d_gr), B * N, C,
            coef_s, coef_rho, total_mass, flags, _stream(dz)))
        return d_s, d_blur, d_gs, d_gr, None, None, None, None, None


def perceive(x, s, grid, eps0=0.1, state_grad=True, density_grad=True, log_norm_grad=True,
             log_norm_density_grad=True, stopgrad_pos=True, stopgrad_state=False):
    """NPA.perceive (models/npa.py:87-137) with the NPA constructor's flags
    (models/npa.py:15-29; eps0 may be a float or the model's eps0 buffer).
    Returns (z, x_bin, s_bin, snapshot), z of width 2C (+ C*D) (+ D)."""
    B, N, C = s.shape
    D = grid.dim
    with torch.no_grad():
        snapshot = grid.instantiate(x)
    x_bin, s_bin = bin_particles(x, s, snapshot)
    x_p = x_bin.detach() if stopgrad_pos else x_bin
    s_p = s_bin.detach() if stopgrad_state else s_bin
    rho = density(x_p, snapshot)
    blur_s = blur(x_p, rho, s_p, snapshot)
    # coef = eps / eps0 and coef ** (1 + D) rounded as torch evaluates them on
    # the model's fp32 buffer: a Python float over a tensor is the tensor's
    # reciprocal times the float; the cube is c * c * c, other powers powf
    e0 = buffer_value(eps0)
    coef = np.float32(np.float32(1.0) / np.float32(e0)) * np.float32(grid.eps)
    coef_rho = coef * coef * coef if D == 2 else np.power(coef, np.float32(1 + D))
    flags = 0
    grad_s = grad_rho = None
    if state_grad:
        grad_s = gradient_hybrid(x_p, rho, s_p, snapshot)
        flags |= STATE_GRAD | (LOG_NORM_GRAD if log_norm_grad else 0)
    if density_grad:
        grad_rho = density_gradient(x_p, snapshot)
        flags |= DENSITY_GRAD | (LOG_NORM_DENSITY_GRAD if log_norm_density_grad else 0)
    z = PerceptionFeatures.apply(s_p.contiguous(), blur_s, grad_s, grad_rho, D, float(coef), float(coef_rho),
                                 float(N), flags)
    return z, x_bin, s_bin, snapshot
