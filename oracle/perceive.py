"""NPA.perceive's feature assembly and step_euler's update, restated in torch
(TEST INFRASTRUCTURE ONLY).

Follows ``models/npa.py:83-85`` (``_log_normalize_grad``) and
``models/npa.py:106-135`` (the scaling of the state gradient by eps/eps0, of the
density gradient by (eps/eps0)^(1+D)/N, the optional log-normalisations and the
concatenation [s, blur, grad_s.view(B, N, C*D), grad_rho]).  Works in any
dtype; the tests run it in float64 on the CPU as the checker of the fused HIP
kernels.
"""
import torch


def log_normalize(v):
    """log(1 + |v|) * v / max(|v|, 1e-12) over the last axis (models/npa.py:83-85)."""
    n = v.norm(dim=-1, keepdim=True)
    return torch.log(1.0 + n) * torch.nn.functional.normalize(v, dim=-1)


def features(s, blur, grad_s, grad_rho, eps, eps0, log_norm_grad=True, log_norm_density_grad=True):
    """z of NPA.perceive from the operator outputs; grad_s / grad_rho may be
    None (state_grad / density_grad off).  eps0 as the model's float32 buffer."""
    B, N, C = s.shape
    # eps / eps0 as the reference evaluates it: eps (Python float) over the
    # model's fp32 eps0 buffer, i.e. reciprocal(eps0) * eps in fp32
    coef = torch.reciprocal(torch.tensor([eps0], dtype=torch.float32)) * eps
    coef = coef.to(device=s.device, dtype=s.dtype)
    z = [s, blur]
    if grad_s is not None:
        g = grad_s * coef
        if log_norm_grad:
            g = log_normalize(g)
        z.append(g.reshape(B, N, -1))
    if grad_rho is not None:
        D = grad_rho.shape[-1]
        gr = grad_rho * (coef ** (1 + D))
        gr = gr / N
        if log_norm_density_grad:
            gr = log_normalize(gr)
        z.append(gr)
    return torch.cat(z, dim=-1)


def euler_update(y, x_bin, s_bin, mask, noise, alpha, eps, dt=1.0, noise_std=0.0):
    """The tail of NPA.forward and the update of step_euler
    (models/npa.py:125-133, 189-200): dx = alpha * a * eps / (1 + |a|) from
    y = [a, ds], padded with zeros to x's width; x + dt * dx * mask (+ noise *
    noise_std * sqrt(dt) * mask), s + dt * ds * mask; and |dx| per particle.
    mask (B, N, 1) or None (all ones), noise like x or None."""
    D = y.shape[-1] - s_bin.shape[-1]
    a = y[..., :D]
    dx = alpha * a * eps / (1.0 + a.norm(dim=-1, keepdim=True))
    dx_norm = dx.norm(dim=-1)
    ds = y[..., D:]
    if dx.shape[-1] != x_bin.shape[-1]:
        dx = torch.cat([dx, torch.zeros_like(dx[..., :1])], dim=-1)
    m = 1.0 if mask is None else mask
    x = x_bin + dt * dx * m
    s = s_bin + dt * ds * m
    if noise is not None and noise_std > 0:
        x = x + noise * noise_std * (dt ** 0.5) * m
    return x, s, dx_norm
