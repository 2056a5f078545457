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


_CAPTURE_CHILD = r"""
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
import npa_amd.sphops as sp
from npa_amd.sphops import _native
lib = _native.lib
B, N, gsz, eps = 2, 20000, (24, 20, 28), 0.05
rng = np.random.default_rng(21)
clouds = []
for _ in range(2):
    c = np.zeros((B, N, 4), np.float32)
    c[..., :3] = rng.standard_normal((B, N, 3)) * 0.2
    clouds.append(c)
grid = sp.HashGrid(dim=3, boundary="clamped", mode="grid", grid_size=list(gsz), eps=eps, num_particles=N,
                   batch_size=B, max_particles_per_block=64)
G = int(np.prod(gsz))
max_blocks = int(lib.sphops_grid_max_blocks(grid.hashgrid._h))
i32 = dict(dtype=torch.int32, device="cuda")
x = torch.empty(B, N, 4, device="cuda")
perm, bo = torch.empty(B, N, **i32), torch.empty(B * G + 1, **i32)
bi, tb = torch.empty(max_blocks, 4, **i32), torch.empty(1, **i32)
p = lambda t: ctypes.c_void_p(t.data_ptr())
gs = (ctypes.c_int32 * 3)(*gsz)
graph = torch.cuda.CUDAGraph()
print("capture: the first sphops_initialize_noalloc call of the process", flush=True)
with torch.cuda.graph(graph):
    st = lib.sphops_initialize_noalloc(3, 0, 0, gs, ctypes.c_float(eps), N, B, 64, p(x), p(perm), p(bo), p(bi),
                                       p(tb), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
assert st == 0, lib.sphops_last_error()
for r, c in enumerate((clouds[0], clouds[1], clouds[0])):
    for t in (perm, bo, bi, tb):
        t.fill_(-7)   # every word must be written by the replay
    x.copy_(torch.from_numpy(c))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    snap = grid.instantiate(torch.from_numpy(c).cuda())
    torch.cuda.synchronize()
    assert torch.equal(perm, snap.permutation), r
    assert torch.equal(bo, snap.bin_offsets), r
    assert torch.equal(bi, snap.block_info), r
    assert torch.equal(tb, snap.total_blocks.reshape(1)), r
    print("replay", r, "matches sphops_initialize", flush=True)
"""


def test_noalloc_under_graph_capture():
    """The entry point is for callers that cannot allocate, such as code under
    HIP graph capture: in a fresh process whose first call of it is made
    under capture (so the per-device scratch lookup happens inside the
    capture), the captured graph, replayed on two position sets (and the
    first again) with eager work in between, gives sphops_initialize's
    outputs bit for bit on every replay."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[no-alloc] graph capture in a child process", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True, text=True, timeout=240)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("matches sphops_initialize") == 3
