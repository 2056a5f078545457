"""Bookkeeping of the pass fusion in npa_amd.sphops.sph (CPU, fake operators).

The fused kernels themselves are checked against the oracle in
test_gpu_parity.py; here the decision logic is: when a grid starts fusing,
when a partner call may take the fused output, and when it must not.
"""
import torch

from npa_amd.sphops import sph


class _Grid:
    pass


class _Snap:
    def __init__(self, grid):
        self.grid = grid


class _Counter:
    def __init__(self):
        self.fused = 0
        self.single = 0


def _fusion(counter):
    def fused(snap, inputs):
        counter.fused += 1
        return inputs[0] + 1.0, inputs[0] * 2.0

    f = sph._PassFusion("pair", fused)
    f.enabled = True
    return f


def _single(counter, which, x):
    def go():
        counter.single += 1
        return x + 1.0 if which == 0 else x * 2.0
    return go


def _call(f, snap, which, x, counter):
    return f.run(snap, which, (x,), _single(counter, which, x))


def test_learns_pair_then_fuses():
    cnt, grid = _Counter(), _Grid()
    f = _fusion(cnt)
    x = torch.arange(4.0)
    s0 = _Snap(grid)
    _call(f, s0, 0, x, cnt)
    _call(f, s0, 1, x, cnt)
    assert (cnt.fused, cnt.single) == (0, 2)
    assert grid._pass_fusion["pair"]["hint"]
    s1 = _Snap(grid)
    a = _call(f, s1, 0, x, cnt)
    b = _call(f, s1, 1, x, cnt)
    assert (cnt.fused, cnt.single) == (1, 2)
    assert torch.equal(a, x + 1.0) and torch.equal(b, x * 2.0)
    # partner first works the same way
    s2 = _Snap(grid)
    b = _call(f, s2, 1, x, cnt)
    a = _call(f, s2, 0, x, cnt)
    assert (cnt.fused, cnt.single) == (2, 2)
    assert torch.equal(a, x + 1.0) and torch.equal(b, x * 2.0)


def _trained(cnt):
    grid = _Grid()
    f = _fusion(cnt)
    x = torch.arange(4.0)
    s0 = _Snap(grid)
    _call(f, s0, 0, x, cnt)
    _call(f, s0, 1, x, cnt)
    return f, grid, x


def test_partner_needs_same_objects_and_versions():
    cnt = _Counter()
    f, grid, x = _trained(cnt)
    s = _Snap(grid)
    _call(f, s, 0, x, cnt)
    other = x.clone()
    b = _call(f, s, 1, other, cnt)          # different tensor object: computed on its own
    assert torch.equal(b, other * 2.0) and cnt.single == 3
    # the fused partner was never collected: the grid stops fusing
    s2 = _Snap(grid)
    _call(f, s2, 0, x, cnt)
    assert not grid._pass_fusion["pair"]["hint"] and cnt.fused == 1 and cnt.single == 4


def test_in_place_change_of_input_blocks_handover():
    cnt = _Counter()
    f, grid, x = _trained(cnt)
    s = _Snap(grid)
    _call(f, s, 0, x, cnt)
    x.add_(1.0)                              # bumps x._version
    b = _call(f, s, 1, x, cnt)
    assert torch.equal(b, x * 2.0) and cnt.single == 3


def test_in_place_change_of_partner_output_blocks_handover():
    cnt = _Counter()
    f, grid, x = _trained(cnt)
    s = _Snap(grid)
    _call(f, s, 0, x, cnt)
    grid._pass_fusion["pair"]["rec"]["outputs"][1].mul_(0.0)
    b = _call(f, s, 1, x, cnt)
    assert torch.equal(b, x * 2.0) and cnt.single == 3


def test_grad_mode_and_snapshot_must_match():
    cnt = _Counter()
    f, grid, x = _trained(cnt)
    s = _Snap(grid)
    with torch.no_grad():
        _call(f, s, 0, x, cnt)
    _call(f, s, 1, x, cnt)
    assert cnt.single == 3
    cnt2 = _Counter()
    f, grid, x = _trained(cnt2)
    _call(f, _Snap(grid), 0, x, cnt2)
    _call(f, _Snap(grid), 1, x, cnt2)       # another snapshot
    assert cnt2.single == 3


def test_output_taken_once():
    cnt = _Counter()
    f, grid, x = _trained(cnt)
    s = _Snap(grid)
    _call(f, s, 0, x, cnt)
    _call(f, s, 1, x, cnt)
    b = _call(f, s, 1, x, cnt)               # a second call computes again
    assert torch.equal(b, x * 2.0)
    assert cnt.fused == 1 and cnt.single == 3


def test_switch_off():
    cnt = _Counter()
    f, grid, x = _trained(cnt)
    f.enabled = False
    s = _Snap(grid)
    _call(f, s, 0, x, cnt)
    _call(f, s, 1, x, cnt)
    assert cnt.fused == 0 and cnt.single == 4


def test_no_strong_reference_to_snapshot_or_inputs():
    import gc
    import weakref
    cnt = _Counter()
    f, grid, x = _trained(cnt)
    s = _Snap(grid)
    y = x.clone()
    _call(f, s, 0, y, cnt)
    _call(f, s, 1, y, cnt)
    ws, wy = weakref.ref(s), weakref.ref(y)
    del s, y
    gc.collect()
    assert ws() is None and wy() is None
