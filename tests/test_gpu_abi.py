"""C-ABI contract checks that need a grid on the GPU: the neighbour-list fill
must follow the candidates call for the same positions and bin_offsets, and
its index buffer is limited to 2^30 entries; a backward can reuse the
(x, weight) records its forward packed."""
import ctypes

import numpy as np
import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu


def _setup():
    import npa_amd.sphops as sp
    c = H.random_case("abi3d", 1, 300, 4, 3, 8, 0.25, False, "grid", uniform=False, sigma=0.2)
    grid = sp.HashGrid(dim=3, boundary="clamped", mode="grid", grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=c.N, batch_size=c.B, max_particles_per_block=c.maxp)
    x = torch.from_numpy(c.x).cuda()
    snap = grid.instantiate(x)
    xb, _ = sp.bin_particles(x, torch.zeros(c.B, c.N, 4, device="cuda"), snap)
    return grid, snap, xb.contiguous()


def test_fill_follows_candidates():
    from npa_amd.sphops import _native
    lib = _native.lib
    grid, snap, xb = _setup()
    hg = grid.hashgrid
    n = xb.shape[0] * xb.shape[1]
    start = torch.empty(n, dtype=torch.int32, device="cuda")
    count = torch.empty(n, dtype=torch.int32, device="cuda")
    total = torch.zeros(2, dtype=torch.int64, device="cuda")  # pairs found, pairs not stored
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    xp, bp = ctypes.c_void_p(xb.data_ptr()), ctypes.c_void_p(snap.bin_offsets.data_ptr())
    _native.check(lib.sphops_neighbor_candidates(hg._h, xp, bp, 0, st))
    cap = 300 * 300
    index = torch.empty(cap, dtype=torch.int32, device="cuda")

    def fill(x_ptr, bo_ptr, cap):
        return lib.sphops_neighbor_fill(hg._h, x_ptr, bo_ptr, ctypes.c_void_p(start.data_ptr()),
                                        ctypes.c_void_p(index.data_ptr()), cap, ctypes.c_void_p(count.data_ptr()),
                                        ctypes.c_void_p(total.data_ptr()), st)

    def rows():
        s, c, idx = start.cpu().numpy(), count.cpu().numpy(), index.cpu().numpy()
        return [idx[s[k]:s[k] + c[k]].tolist() if c[k] >= 0 else c[k] for k in range(n)]

    # another bin_offsets tensor (same contents, other storage) is refused
    other = snap.bin_offsets.clone()
    assert fill(xp, ctypes.c_void_p(other.data_ptr()), cap) != 0
    assert b"must follow" in lib.sphops_last_error()
    # an index buffer above 2^30 entries is refused
    assert fill(xp, bp, (1 << 30) + 1) != 0
    assert b"above 2^30" in lib.sphops_last_error()
    # the matching call works, twice, and gives the same rows (where a row
    # lands may differ); the total is the sum of the counts
    assert fill(xp, bp, cap) == 0
    torch.cuda.synchronize()
    first = rows()
    assert total.tolist() == [int(count.sum().item()), 0]
    assert fill(xp, bp, cap) == 0
    torch.cuda.synchronize()
    assert rows() == first
    # the grid's own first build (sized before any total is known) stores the
    # same counts where it stored a row
    ref = hg.neighbor_list(xb, snap.bin_offsets)
    torch.cuda.synchronize()
    stored = ref[1] >= 0
    assert torch.equal(ref[1][stored], count[stored])
    # a buffer one entry short of the total: some row is not stored, and its
    # count encodes its stencil candidates; the total still counts it, and the
    # second word counts the pairs of the rows not stored
    need = int(total[0].item())
    assert fill(xp, bp, need - 1) == 0
    torch.cuda.synchronize()
    c = count.cpu().numpy()
    assert (c < 0).any() and int(total[0].item()) == need
    assert np.all(c[c < 0] <= -2)
    assert int(total[1].item()) == sum(len(first[k]) for k in np.flatnonzero(c < 0))


def test_fill_after_tiles_is_refused():
    """sphops_neighbor_tiles reuses the grid scratch that holds the fill's
    work split, so a fill after it must be refused until the candidates call
    runs again (then it works)."""
    from npa_amd.sphops import _native
    lib = _native.lib
    grid, snap, xb = _setup()
    hg = grid.hashgrid
    n = xb.shape[0] * xb.shape[1]
    i32 = dict(dtype=torch.int32, device="cuda")
    start, count, order = torch.empty(n, **i32), torch.empty(n, **i32), torch.empty(n, **i32)
    total = torch.zeros(2, dtype=torch.int64, device="cuda")
    cap = 300 * 300
    index = torch.empty(cap, **i32)
    tcap = int(lib.sphops_neighbor_tile_capacity(hg._h))
    wcap = 2 * int(lib.sphops_neighbor_wave_capacity(hg._h))
    units, waves = torch.empty(2 * tcap, **i32), torch.empty(wcap, **i32)
    counts = torch.zeros(2, **i32)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    xp, bp = ctypes.c_void_p(xb.data_ptr()), ctypes.c_void_p(snap.bin_offsets.data_ptr())
    p = lambda t, off=0: ctypes.c_void_p(t.data_ptr() + off)

    def fill():
        return lib.sphops_neighbor_fill(hg._h, xp, bp, p(start), p(index), cap, p(count), p(total), st)

    _native.check(lib.sphops_neighbor_candidates(hg._h, xp, bp, 1, st))
    assert fill() == 0
    _native.check(lib.sphops_neighbor_tiles(hg._h, xp, bp, p(count), p(units), p(counts), p(order), p(waves),
                                            p(counts, 4), st))
    assert fill() != 0
    assert b"must follow" in lib.sphops_last_error()
    # the tile build replaced the split instantiate derived: vouching for
    # bin_offsets no longer skips the work, and the fill is complete
    _native.check(lib.sphops_neighbor_candidates(hg._h, xp, bp, 1, st))
    assert fill() == 0
    torch.cuda.synchronize()
    assert total.tolist() == [int(count.sum().item()), 0]
    ref = hg.neighbor_list(xb, snap.bin_offsets)
    torch.cuda.synchronize()
    stored = ref[1] >= 0
    assert torch.equal(ref[1][stored], count[stored])


def _rows(start, count, index):
    """Rows of a list; None for a row that was not stored."""
    s, c, idx = start.cpu().numpy(), count.cpu().numpy(), index.cpu().numpy()
    return [idx[s[k]:s[k] + c[k]].tolist() if c[k] >= 0 else None for k in range(len(c))]


def _same_stored(rows, ref):
    assert len(rows) == len(ref)
    assert all(r is None or r == q for r, q in zip(rows, ref))


@pytest.mark.parametrize("mode", ["grid", "particle"])
def test_split_from_initialize(mode):
    """sphops_initialize derives the fill's work split from the sorted keys;
    a candidates call that vouches for the bin_offsets that call wrote
    reuses it, and the rows equal those of a split computed from the
    positions.  After another snapshot on the same grid the older
    bin_offsets no longer matches, and the split is computed again (the
    Python layer vouches only for the tensor the last initialize wrote)."""
    import npa_amd.sphops as sp
    from npa_amd.sphops import _native
    lib = _native.lib
    c = H.random_case("split3d", 2, 400, 4, 3, 8, 0.25, False, mode, uniform=False, sigma=0.2)
    grid = sp.HashGrid(dim=3, boundary="clamped", mode=mode, grid_size=list(c.grid_size), eps=c.eps,
                       num_particles=c.N, batch_size=c.B, max_particles_per_block=c.maxp)
    hg = grid.hashgrid
    n = c.B * c.N
    i32 = dict(dtype=torch.int32, device="cuda")
    cap = n * n
    bufs = [(torch.empty(n, **i32), torch.empty(n, **i32), torch.empty(cap, **i32)) for _ in range(2)]
    total = torch.zeros(2, dtype=torch.int64, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())

    def build(xb, bo, vouch, out):
        start, count, index = out
        _native.check(lib.sphops_neighbor_candidates(hg._h, p(xb), p(bo), vouch, st))
        _native.check(lib.sphops_neighbor_fill(hg._h, p(xb), p(bo), p(start), p(index), cap, p(count), p(total),
                                               st))
        torch.cuda.synchronize()
        assert int(total[1].item()) == 0
        return _rows(start, count, index)

    x1 = torch.from_numpy(c.x).cuda()
    snap1 = grid.instantiate(x1)
    xb1 = sp.bin_particles(x1, torch.zeros(c.B, c.N, 4, device="cuda"), snap1)[0].contiguous()
    reused = build(xb1, snap1.bin_offsets, 1, bufs[0])
    computed = build(xb1, snap1.bin_offsets, 0, bufs[1])
    assert reused == computed
    # a second snapshot (other positions) on the same grid
    x2 = x1.flip(1).contiguous() * 0.9
    snap2 = grid.instantiate(x2)
    xb2 = sp.bin_particles(x2, torch.zeros(c.B, c.N, 4, device="cuda"), snap2)[0].contiguous()
    assert build(xb1, snap1.bin_offsets, 1, bufs[0]) == computed
    second = build(xb2, snap2.bin_offsets, 0, bufs[1])
    plan1 = hg.neighbor_list(xb1, snap1.bin_offsets)
    plan2 = hg.neighbor_list(xb2, snap2.bin_offsets)
    torch.cuda.synchronize()
    _same_stored(_rows(plan1[0], plan1[1], plan1[2]), computed)
    _same_stored(_rows(plan2[0], plan2[1], plan2[2]), second)


def test_packed_records_reused_by_backward():
    """sphops_args.packed: a forward writes its (x, weight) records there and
    a backward given them (packed_valid) skips its own packing; its results
    equal, bit for bit, those of a backward that packs again.  A backward
    claiming valid records without a buffer, or a misaligned buffer, fails."""
    import npa_amd.sphops as sp
    from npa_amd.sphops import _native as O
    grid, snap, xb = _setup()
    hg = grid.hashgrid
    B, N = xb.shape[:2]
    C = 16
    g = torch.Generator(device="cuda").manual_seed(3)
    sb = torch.randn(B, N, C, device="cuda", generator=g)
    m = torch.rand(B, N, device="cuda", generator=g) + 0.5
    bo = snap.bin_offsets
    from npa_amd.sphops.sph import _plan
    nbr = _plan(snap, xb)
    rho = torch.empty(B, N, device="cuda")
    hg.op_forward(O.OP_DENSITY, xb, rho, bo, mass=m, nbr=nbr)
    up1 = torch.randn(B, N, C, device="cuda", generator=g)
    up2 = torch.randn(B, N, C, 3, device="cuda", generator=g)
    packed = torch.empty(B * N, 4, device="cuda")
    blur, hyb = torch.empty_like(sb), torch.empty(B, N, C, 3, device="cuda")
    hg.op_forward(O.OP_BLUR_GRADIENT_HYBRID, xb, blur, bo, mass=m, rho=rho, state=sb, nbr=nbr, out2=hyb,
                  packed=packed)

    def bwd(pk):
        gx, gs, gr = torch.empty_like(xb), torch.empty_like(sb), torch.empty_like(rho)
        # the grid's scratch holds other records in between (mass-weighted)
        hg.op_forward(O.OP_DENSITY, xb, torch.empty_like(rho), bo, mass=m, nbr=nbr)
        hg.op_backward(O.OP_BLUR_GRADIENT_HYBRID, xb, up1, bo, m, rho=rho, state=sb, grad_x=gx, grad_state=gs,
                       grad_rho=gr, nbr=nbr, upstream2=up2, packed=pk)
        torch.cuda.synchronize()
        return gx, gs, gr

    for a, b in zip(bwd(packed), bwd(None)):
        assert torch.equal(a, b)
    with pytest.raises(RuntimeError, match="packed_valid needs packed"):
        hg._args(O.OP_BLUR, xb, bo, m, rho, sb, packed=None, packed_valid=True)
    bad = torch.empty(B * N * 4 + 1, device="cuda")[1:].view(B * N, 4)
    with pytest.raises(TypeError, match="16-byte aligned"):
        hg._args(O.OP_BLUR, xb, bo, m, rho, sb, packed=bad, packed_valid=True)


def test_copy_words_to_host():
    """sphops_copy_words_to_host writes device words into pinned host memory
    (the list totals' read-back), visible once the stream is synchronised;
    more than 256 words are refused."""
    from npa_amd.sphops import _native
    lib = _native.lib
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    src = torch.randint(-2**31, 2**31 - 1, (256,), dtype=torch.int32, device="cuda")
    dst = torch.zeros(256, dtype=torch.int32, pin_memory=True)
    for words in (8, 1, 256):
        dst.zero_()
        _native.check(lib.sphops_copy_words_to_host(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()),
                                                    words, st))
        torch.cuda.synchronize()
        assert torch.equal(dst[:words], src[:words].cpu())
        assert not bool(dst[words:].any())
    assert lib.sphops_copy_words_to_host(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), 257,
                                         st) != 0
    assert b"at most 256" in lib.sphops_last_error()
