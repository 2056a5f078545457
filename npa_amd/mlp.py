"""The NPA MLP (models/npa.py:63-78 of the reference: torch.nn.Linear layers
with a ReLU between) with the weight gradient of each linear layer computed
by ``sphops_linear_weight_grad``.

Over one row per particle the weight gradient dW = dY^T X is a GEMM with a
tiny output and a reduction over 10^5-10^6 rows; the library GEMM takes that
shape with few output tiles and runs at a few TFLOP/s.  ``LinearRows`` keeps
torch's forward and input gradient (both large, well-shaped GEMMs) and
replaces the weight and bias gradients by the row-chunked matrix-core kernel.
``mlp(module, z)`` runs a module the way the module would run itself, with its
``torch.nn.Linear`` layers through ``LinearRows``; the parameters are the
module's own, so optimisers and checkpoints see no difference.
"""
import ctypes

import torch
import torch.nn.functional as F

from .sphops import _native

_lib = _native.lib


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


class LinearRows(torch.autograd.Function):
    """y = x W^T + b over x of shape (..., in); the backward's dW and db come
    from the row-chunked kernel, dx from torch."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return F.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        need_x, need_w, need_b = ctx.needs_input_grad
        dx = dw = db = None
        out_f, in_f = weight.shape
        dy2 = dy.reshape(-1, out_f)
        if need_x:
            dx = (dy2 @ weight).reshape(x.shape)
        if need_w or (need_b and ctx.has_bias):
            x2 = x.reshape(-1, in_f)
            if x2.dtype != torch.float32 or dy2.dtype != torch.float32 or not x2.is_cuda:
                raise TypeError("LinearRows takes float32 GPU tensors")
            x2, dy2 = x2.contiguous(), dy2.contiguous()
            rows = x2.shape[0]
            dw = torch.empty(out_f, in_f, device=x.device)
            db = torch.empty(out_f, device=x.device) if ctx.has_bias else None
            nbytes = _lib.sphops_linear_weight_grad_workspace_bytes(rows, in_f, out_f)
            work = torch.empty(max(nbytes // 4, 1), device=x.device)
            st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(x.device.index))
            _native.check(_lib.sphops_linear_weight_grad(_ptr(x2), _ptr(dy2), _ptr(dw), _ptr(db), rows, in_f, out_f,
                                                         _ptr(work), st))
        return dx, (dw if need_w else None), (db if need_b else None)


def linear(x, layer):
    return LinearRows.apply(x, layer.weight, layer.bias)


def mlp(module, z):
    """``module(z)`` for a ``torch.nn.Linear`` or a ``torch.nn.Sequential`` of
    layers (the shapes NPA's _get_mlp builds), with every Linear through
    ``LinearRows``; any other module runs as it is."""
    if isinstance(module, torch.nn.Linear):
        return linear(z, module)
    if isinstance(module, torch.nn.Sequential):
        for layer in module:
            z = linear(z, layer) if isinstance(layer, torch.nn.Linear) else layer(z)
        return z
    return module(z)
