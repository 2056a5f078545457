"""The NPA MLP (models/npa.py:63-78 of the reference: torch.nn.Linear layers
with a ReLU between) with the weight gradient of each linear layer computed
by ``sphops_linear_weight_grad``.

Over one row per particle the weight gradient dW = dY^T X is a GEMM with a
tiny output and a reduction over 10^5-10^6 rows; the library GEMM takes that
shape with few output tiles and runs at a few TFLOP/s.  ``LinearRows`` keeps
torch's forward and input gradient (both large, well-shaped GEMMs) and
replaces the weight and bias gradients by the row-chunked matrix-core kernel.
A ReLU followed by a Linear with at most 64 outputs (NPA's last layer) runs
as ``ReluLinear``, whose backward computes the input gradient through both in
one kernel.  ``mlp(module, z)`` runs a module the way the module would run
itself, with its ``torch.nn.Linear`` layers through these; the parameters are
the module's own, so optimisers and checkpoints see no difference.
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
            dw, db = _weight_grad(x.reshape(-1, in_f), dy2, ctx.has_bias)
        return dx, (dw if need_w else None), (db if need_b else None)


def _weight_grad(x2, dy2, has_bias, relu_x=False):
    """dW = dy2^T x2 (dy2^T relu(x2) with relu_x) and db = column sums of dy2
    (None without a bias) through ``sphops_linear_weight_grad`` or
    ``sphops_relu_linear_weight_grad``."""
    if x2.dtype != torch.float32 or dy2.dtype != torch.float32 or not x2.is_cuda:
        raise TypeError("the MLP kernels take float32 GPU tensors")
    x2, dy2 = x2.contiguous(), dy2.contiguous()
    rows, in_f = x2.shape
    out_f = dy2.shape[1]
    dw = torch.empty(out_f, in_f, device=x2.device)
    db = torch.empty(out_f, device=x2.device) if has_bias else None
    nbytes = _lib.sphops_linear_weight_grad_workspace_bytes(rows, in_f, out_f)
    work = torch.empty(max(nbytes // 4, 1), device=x2.device)
    st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(x2.device.index))
    fn = _lib.sphops_relu_linear_weight_grad if relu_x else _lib.sphops_linear_weight_grad
    _native.check(fn(_ptr(x2), _ptr(dy2), _ptr(dw), _ptr(db), rows, in_f, out_f, _ptr(work), st))
    return dw, db


class ReluLinear(torch.autograd.Function):
    """y = relu(a) W^T + b (``torch.nn.ReLU`` then ``torch.nn.Linear``).  For
    in_features a multiple of 4 up to 256 the forward is one kernel
    (``sphops_relu_linear_forward``) that never writes relu(a), and the
    backward keeps ``a``; otherwise the forward is torch's and the backward
    keeps h = relu(a).  The backward takes da = (relu(a) > 0) * (dy W) from
    ``sphops_relu_linear_input_grad`` (a <= 0 exactly where relu(a) <= 0, so
    either saved tensor gives the mask) and dW, db from the row-chunked
    kernel."""

    @staticmethod
    def forward(ctx, a, weight, bias):
        out_f, in_f = weight.shape
        fused = (a.is_cuda and a.dtype == torch.float32 and weight.dtype == torch.float32
                 and in_f % 4 == 0 and 4 <= in_f <= RELU_LINEAR_MAX_IN and out_f <= RELU_LINEAR_MAX_OUT)
        ctx.has_bias = bias is not None
        ctx.pre = fused
        if not fused:
            h = torch.relu(a)
            ctx.save_for_backward(h, weight)
            return F.linear(h, weight, bias)
        a2 = a.reshape(-1, in_f).contiguous()
        if a2.data_ptr() % 16:
            a2 = a2.clone()
        w = weight.detach().contiguous()
        b = None if bias is None else bias.detach().contiguous()
        y = torch.empty(a2.shape[0], out_f, device=a.device)
        st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(a.device.index))
        _native.check(_lib.sphops_relu_linear_forward(_ptr(a2), _ptr(w), _ptr(b), _ptr(y), a2.shape[0], in_f,
                                                      out_f, st))
        ctx.save_for_backward(a2, weight)
        return y.reshape(*a.shape[:-1], out_f)

    @staticmethod
    def backward(ctx, dy):
        s, weight = ctx.saved_tensors  # a (ctx.pre) or relu(a)
        need_a, need_w, need_b = ctx.needs_input_grad
        out_f, in_f = weight.shape
        s2 = s.reshape(-1, in_f)
        dy2 = dy.reshape(-1, out_f).contiguous()
        da = dw = db = None
        if need_a:
            if s2.dtype != torch.float32 or dy2.dtype != torch.float32 or not s2.is_cuda:
                raise TypeError("the MLP kernels take float32 GPU tensors")
            s2 = s2.contiguous()
            w = weight.detach().contiguous()
            da2 = torch.empty_like(s2)
            st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(s2.device.index))
            _native.check(_lib.sphops_relu_linear_input_grad(_ptr(dy2), _ptr(w), _ptr(s2), _ptr(da2), s2.shape[0],
                                                             in_f, out_f, st))
            da = da2.reshape(dy.shape[:-1] + (in_f,))
        if need_w or (need_b and ctx.has_bias):
            dw, db = _weight_grad(s2, dy2, ctx.has_bias, relu_x=ctx.pre)
        return da, (dw if need_w else None), (db if need_b else None)


# ReluLinear keeps W's 32-output tiles in registers (the fused forward also
# all of a row's in_features)
RELU_LINEAR_MAX_OUT = 64
RELU_LINEAR_MAX_IN = 256


def linear(x, layer):
    return LinearRows.apply(x, layer.weight, layer.bias)


def relu_linear(a, layer):
    """``layer(torch.relu(a))`` with the fused backward."""
    return ReluLinear.apply(a, layer.weight, layer.bias)


def mlp(module, z):
    """``module(z)`` for a ``torch.nn.Linear`` or a ``torch.nn.Sequential`` of
    layers (the shapes NPA's _get_mlp builds): a ReLU followed by a Linear of at
    most RELU_LINEAR_MAX_OUT outputs through ``ReluLinear``, every other Linear
    through ``LinearRows``; any other module runs as it is."""
    if isinstance(module, torch.nn.Linear):
        return linear(z, module)
    if isinstance(module, torch.nn.Sequential):
        layers = list(module)
        i = 0
        while i < len(layers):
            layer = layers[i]
            nxt = layers[i + 1] if i + 1 < len(layers) else None
            if (type(layer) is torch.nn.ReLU and isinstance(nxt, torch.nn.Linear)
                    and nxt.out_features <= RELU_LINEAR_MAX_OUT):
                z = relu_linear(z, nxt)
                i += 2
                continue
            z = linear(z, layer) if isinstance(layer, torch.nn.Linear) else layer(z)
            i += 1
        return z
    return module(z)
