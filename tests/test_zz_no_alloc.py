"""sphops_initialize_noalloc (binning with a static scratch array, no
allocation) against sphops_initialize on a grid object, through the C ABI:
permutation, bin_offsets, block_info and total_blocks must be identical, for
two calls in a row of which the second is smaller (the static array keeps the
first call's contents), and for both modes and boundaries.  Sizes above the
entry point's limits fail with an error before any work is queued."""
import ctypes

import numpy as np
import pytest
import torch

import helpers as H
from npa_amd import workloads

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _noalloc(c):
    """Outputs of sphops_initialize_noalloc for case c (fresh output buffers,
    filled with a sentinel so that unwritten words would show)."""
    from npa_amd.sphops import _native
    import npa_amd.sphops as sp
    dim, B, N = c.dim, c.B, c.N
    G = int(np.prod(c.grid_size))
    grid = sp.HashGrid(dim=dim, boundary=c.boundary, mode=c.mode, grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=N, batch_size=B, max_particles_per_block=c.maxp)
    max_blocks = int(_native.lib.sphops_grid_max_blocks(grid.hashgrid._h))
    x = torch.from_numpy(c.x).cuda()
    perm = torch.full((B, N), -7, dtype=torch.int32, device="cuda")
    bo = torch.full((B * G + 1,), -7, dtype=torch.int32, device="cuda")
    bi = torch.full((max_blocks, 4), -7, dtype=torch.int32, device="cuda")
    tb = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    gs = (ctypes.c_int32 * dim)(*c.grid_size)
    st = _native.lib.sphops_initialize_noalloc(
        dim, 1 if c.periodic else 0,
        1 if c.mode == "particle" else 0, gs, ctypes.c_float(c.eps), N, B,
        c.maxp, _ptr(x), _ptr(perm), _ptr(bo), _ptr(bi), _ptr(tb), _stream())
    assert st == 0, _native.lib.sphops_last_error()
    # the grid object's entry point, on the same positions
    snap = grid.instantiate(x)
    torch.cuda.synchronize()
    return (perm, bo, bi, tb), snap


def _check(c):
    print(f"[no-alloc] {c.name} B={c.B} N={c.N} grid={c.grid_size} {c.boundary} {c.mode}", flush=True)
    (perm, bo, bi, tb), snap = _noalloc(c)
    assert torch.equal(perm, snap.permutation)
    assert torch.equal(bo, snap.bin_offsets)
    if c.mode == "grid":
        assert torch.equal(bi, snap.block_info)
    assert torch.equal(tb, snap.total_blocks.reshape(1))


def test_noalloc_matches_grid_entry_point_twice():
    big = H.workload_case(workloads.make("cfg5", 1.0))   # 2^20 particles, 206 M cells: at the limits
    small = H.random_case("ref2d", 3, 256, 4, 2, 16, 0.1, False, "grid")
    _check(big)
    _check(small)   # second call, smaller: the array holds the first call's contents


@pytest.mark.parametrize("periodic,mode", [(True, "grid"), (False, "particle"), (True, "particle")])
def test_noalloc_modes(periodic, mode):
    c = H.random_case(f"r3d-{mode}", 2, 700, 4, 3, 16, 0.15, periodic, mode, maxp=32)
    _check(c)
    _check(H.random_case("r2d-small", 1, 37, 4, 2, 8, 0.3, periodic, mode, maxp=8))


def test_noalloc_limits_are_errors():
    from npa_amd.sphops import _native
    lib = _native.lib
    gs = (ctypes.c_int32 * 3)(16, 16, 16)
    null = ctypes.c_void_p(0)
    st = lib.sphops_initialize_noalloc(3, 0, 0, gs, ctypes.c_float(0.1), (1 << 20) + 1, 1, 64, null, null, null,
                                       null, null, _stream())
    assert st != 0 and b"above 2^20" in lib.sphops_last_error()
    gs = (ctypes.c_int32 * 3)(1024, 1024, 257)
    st = lib.sphops_initialize_noalloc(3, 0, 0, gs, ctypes.c_float(0.1), 1000, 1, 64, null, null, null, null,
                                       null, _stream())
    assert st != 0 and b"above 2^28" in lib.sphops_last_error()
