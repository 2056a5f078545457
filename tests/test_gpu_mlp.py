"""The row-chunked weight and bias gradients of a linear layer
(``sphops_linear_weight_grad`` via npa_amd.mlp) against float64 sums, over
row counts from 0 to 3e5 (inside one 16-row load group, across chunk ends)
and layer shapes that take one to four 32-column tiles per wave, several
32-row bands, exact tile multiples and ragged edges; the feature limit; and
npa_amd.mlp.mlp against the module's own autograd."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(83, 128), (128, 19), (5, 3), (200, 130), (32, 64), (300, 7), (66, 128)]
ROWS = [0, 1, 17, 100, 1000, 33333, 131073, 300000]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("rows", ROWS)
def test_weight_grad_matches_float64(shape, rows):
    import ctypes
    from npa_amd.sphops import _native
    in_f, out_f = shape
    g = torch.Generator(device="cuda").manual_seed(rows + in_f)
    x = torch.randn(rows, in_f, device="cuda", generator=g)
    dy = torch.randn(rows, out_f, device="cuda", generator=g)
    dw = torch.full((out_f, in_f), float("nan"), device="cuda")
    db = torch.full((out_f,), float("nan"), device="cuda")
    nb = _native.lib.sphops_linear_weight_grad_workspace_bytes(rows, in_f, out_f)
    work = torch.empty(max(nb // 4, 1), device="cuda")
    st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(0))
    _native.check(_native.lib.sphops_linear_weight_grad(
        ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(dy.data_ptr()), ctypes.c_void_p(dw.data_ptr()),
        ctypes.c_void_p(db.data_ptr()), rows, in_f, out_f, ctypes.c_void_p(work.data_ptr()), st))
    xd, yd = x.double().cpu(), dy.double().cpu()
    ref_w, ref_b = yd.T @ xd, yd.sum(0)
    bound_w = (yd.abs().T @ xd.abs()) * 1e-5 + 1e-30   # fp32 summation error scale
    bound_b = yd.abs().sum(0) * 1e-5 + 1e-30
    assert torch.all((dw.cpu().double() - ref_w).abs() <= bound_w), f"dW rows={rows} shape={shape}"
    assert torch.all((db.cpu().double() - ref_b).abs() <= bound_b), f"db rows={rows} shape={shape}"


def test_weight_grad_is_deterministic():
    from npa_amd import mlp as M
    lin = torch.nn.Linear(83, 128).cuda()
    x = torch.randn(200000, 83, device="cuda")
    dy = torch.randn(200000, 128, device="cuda")
    grads = []
    for _ in range(2):
        lin.zero_grad()
        M.linear(x, lin).backward(dy)
        grads.append((lin.weight.grad.clone(), lin.bias.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])


@pytest.mark.parametrize("hidden", [None, 32])
def test_mlp_matches_module_autograd(hidden):
    from npa_amd import mlp as M
    torch.manual_seed(0)
    if hidden is None:
        net = torch.nn.Linear(66, 18, bias=False).cuda()
    else:
        net = torch.nn.Sequential(torch.nn.Linear(66, hidden), torch.nn.ReLU(),
                                  torch.nn.Linear(hidden, 18, bias=False)).cuda()
    z = torch.randn(3, 5000, 66, device="cuda", requires_grad=True)
    up = torch.randn(3, 5000, 18, device="cuda")
    out = M.mlp(net, z)
    if hidden is None:
        assert torch.equal(out, net(z))  # the forward is torch's own
    else:
        assert type(out.grad_fn).__name__ == "ReluLinearBackward"  # the fused ReLU + Linear ran
        ref_out = net(z).detach()
        assert torch.allclose(out, ref_out, rtol=1e-5, atol=1e-5 * float(ref_out.abs().max()))
    got = torch.autograd.grad(out, [z] + list(net.parameters()), up)
    ref = torch.autograd.grad(net(z), [z] + list(net.parameters()), up)
    for a, b in zip(got, ref):
        assert torch.allclose(a, b, rtol=1e-4, atol=1e-4 * float(b.abs().max())), "gradient differs"


def test_feature_limit_is_an_error():
    import ctypes
    from npa_amd.sphops import _native
    x = torch.zeros(4, 1, device="cuda")
    p = ctypes.c_void_p(x.data_ptr())
    st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(0))
    for in_f, out_f in ((32769, 1), (1, 32769)):
        with pytest.raises(RuntimeError, match="in_features and out_features"):
            _native.check(_native.lib.sphops_linear_weight_grad(p, p, p, p, 1, in_f, out_f, p, st))


RELU_SHAPES = [(128, 19), (128, 18), (5, 3), (200, 64), (64, 1), (130, 33)]


@pytest.mark.parametrize("shape", RELU_SHAPES)
@pytest.mark.parametrize("rows", [0, 1, 9, 1000, 100003, 131073])
def test_relu_linear_input_grad_matches_float64(shape, rows):
    """da = 0 where h = relu(a) <= 0, else dy W (torch's threshold_backward of
    the Linear's input gradient), against float64."""
    import ctypes
    from npa_amd.sphops import _native
    in_f, out_f = shape
    g = torch.Generator(device="cuda").manual_seed(7 * rows + in_f + out_f)
    h = torch.relu(torch.randn(rows, in_f, device="cuda", generator=g))
    dy = torch.randn(rows, out_f, device="cuda", generator=g)
    w = torch.randn(out_f, in_f, device="cuda", generator=g)
    da = torch.full((rows, in_f), float("nan"), device="cuda")
    st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(0))
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    _native.check(_native.lib.sphops_relu_linear_input_grad(P(dy), P(w), P(h), P(da), rows, in_f, out_f, st))
    hd, yd, wd = h.double().cpu(), dy.double().cpu(), w.double().cpu()
    ref = torch.where(hd <= 0, torch.zeros((), dtype=torch.float64), yd @ wd)
    bound = (yd.abs() @ wd.abs()) * 1e-5 + 1e-30
    got = da.cpu().double()
    assert torch.all(got[hd <= 0] == 0), "masked entries must be exactly zero"
    assert torch.all((got - ref).abs() <= bound), f"da rows={rows} shape={shape}"


def test_relu_linear_output_limit_is_an_error():
    import ctypes
    from npa_amd.sphops import _native
    x = torch.zeros(4, 1, device="cuda")
    p = ctypes.c_void_p(x.data_ptr())
    st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(0))
    with pytest.raises(RuntimeError, match="out_features"):
        _native.check(_native.lib.sphops_relu_linear_input_grad(p, p, p, p, 1, 4, 65, p, st))


@pytest.mark.parametrize("shape", [(128, 19), (128, 18), (4, 3), (256, 64), (64, 1), (132, 33), (20, 40)])
@pytest.mark.parametrize("rows", [0, 1, 9, 1000, 100003, 131073])
def test_relu_linear_forward_matches_float64(shape, rows):
    """y = relu(a) W^T + b (with and without b) against float64, and the
    weight gradient with relu applied to its input against dy^T relu(a)."""
    import ctypes
    from npa_amd.sphops import _native
    in_f, out_f = shape
    g = torch.Generator(device="cuda").manual_seed(11 * rows + in_f + out_f)
    a = torch.randn(rows, in_f, device="cuda", generator=g)
    w = torch.randn(out_f, in_f, device="cuda", generator=g)
    b = torch.randn(out_f, device="cuda", generator=g)
    st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(0))
    P = lambda t: ctypes.c_void_p(0 if t is None else t.data_ptr())
    hd, wd = torch.relu(a).double().cpu(), w.double().cpu()
    for bias in (b, None):
        bd = torch.zeros(out_f, dtype=torch.float64) if bias is None else bias.double().cpu()
        bound = (hd @ wd.abs().T + bd.abs()) * 1e-5 + 1e-30  # fp32 sums, then the rounded + b
        y = torch.full((rows, out_f), float("nan"), device="cuda")
        _native.check(_native.lib.sphops_relu_linear_forward(P(a), P(w), P(bias), P(y), rows, in_f, out_f, st))
        ref = hd @ wd.T + bd
        assert torch.all((y.cpu().double() - ref).abs() <= bound), f"y rows={rows} shape={shape} bias={bias is not None}"
    dy = torch.randn(rows, out_f, device="cuda", generator=g)
    dw = torch.full((out_f, in_f), float("nan"), device="cuda")
    db = torch.full((out_f,), float("nan"), device="cuda")
    nb = _native.lib.sphops_linear_weight_grad_workspace_bytes(rows, in_f, out_f)
    work = torch.empty(max(nb // 4, 1), device="cuda")
    _native.check(_native.lib.sphops_relu_linear_weight_grad(P(a), P(dy), P(dw), P(db), rows, in_f, out_f, P(work),
                                                            st))
    yd = dy.double().cpu()
    assert torch.all((dw.cpu().double() - yd.T @ hd).abs() <= (yd.abs().T @ hd) * 1e-5 + 1e-30)
    assert torch.all((db.cpu().double() - yd.sum(0)).abs() <= yd.abs().sum(0) * 1e-5 + 1e-30)


def test_relu_linear_forward_limits_are_errors():
    import ctypes
    from npa_amd.sphops import _native
    x = torch.zeros(64, device="cuda")
    p = ctypes.c_void_p(x.data_ptr())
    st = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(0))
    for in_f, out_f, msg in ((6, 3, "multiple of 4"), (260, 3, "multiple of 4"), (8, 65, "out_features")):
        with pytest.raises(RuntimeError, match=msg):
            _native.check(_native.lib.sphops_relu_linear_forward(p, p, p, p, 1, in_f, out_f, st))
    with pytest.raises(RuntimeError, match="aligned"):
        _native.check(_native.lib.sphops_relu_linear_forward(ctypes.c_void_p(x.data_ptr() + 4), p, p, p, 1, 8, 3, st))
