"""Pins the binning oracle (oracle/binning.py) against closed forms and brute force."""
import itertools

import numpy as np
import pytest

from oracle import binning


def test_floor_cell_matches_float_floor():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * 3).astype(np.float32)
    inv = binning.inv_eps_f32(0.1)
    got = binning.floor_cell_ftz(x, inv)
    ref = np.floor((x * inv).astype(np.float32).astype(np.float64)).astype(np.int64)
    np.testing.assert_array_equal(got, ref)


def test_flush_to_zero_special_cases():
    inv = binning.inv_eps_f32(0.5)
    tiny = np.float32(-1e-40)           # negative subnormal: flushed, cell offset 0
    assert binning.floor_cell_ftz(np.array([tiny]), inv)[0] == 0
    assert binning.floor_cell_ftz(np.array([np.float32(-1e-30)]), inv)[0] == -1  # normal stays
    # a normal input whose product is subnormal is flushed too
    inv_small = np.float32(1e-10)
    assert binning.floor_cell_ftz(np.array([np.float32(-1e-30)]), inv_small)[0] == 0
    assert binning.floor_cell_ftz(np.array([np.float32(np.nan)]), inv)[0] == 0
    assert binning.floor_cell_ftz(np.array([np.float32(np.inf)]), inv)[0] == 2 ** 31 - 1
    assert binning.floor_cell_ftz(np.array([np.float32(-np.inf)]), inv)[0] == -(2 ** 31)


def test_inv_eps_is_fp32_reciprocal_of_fp32_eps():
    for eps in (0.1, 0.2, 0.0026222667656838894, 1 / 47):
        e = np.float32(eps)
        assert binning.inv_eps_f32(eps) == np.float32(1.0) / e


@pytest.mark.parametrize("periodic", [False, True])
def test_pos2cell_boundary(periodic):
    gs = (8, 6)
    eps = 0.25
    x = np.array([[-10.0, 10.0], [0.0, 0.0], [-0.01, -0.01], [0.9999, 0.7499], [1.0, 0.75]], np.float32)
    c = binning.pos2cell(x, gs, eps, periodic)
    raw = np.floor(x.astype(np.float64) / eps).astype(np.int64) + np.array([4, 3])
    if periodic:
        ref = np.mod(raw, gs)
    else:
        ref = np.clip(raw, 0, np.array(gs) - 1)
    np.testing.assert_array_equal(c, ref)


@pytest.mark.parametrize("dim", [2, 3])
def test_row_major_hash_is_bijective(dim):
    gs = (5, 4, 3)[:dim]
    cells = np.array(list(itertools.product(*[range(g) for g in gs])))
    h = binning.cell_hash(cells, gs, "grid")
    assert sorted(h.tolist()) == list(range(int(np.prod(gs))))
    # x is the fastest axis
    one = np.zeros((1, dim), np.int64)
    one[0, 0] = 1
    assert binning.cell_hash(one, gs, "grid")[0] == 1
    np.testing.assert_array_equal(binning.hash2cell(h, gs, "grid"), cells)


@pytest.mark.parametrize("dim", [2, 3])
def test_morton_hash_interleaves_bits(dim):
    gs = (16,) * dim
    cells = np.array(list(itertools.product(*[range(g) for g in gs])))
    h = binning.cell_hash(cells, gs, "particle")
    assert sorted(h.tolist()) == list(range(16 ** dim))
    # bit b of axis d lands at bit b*dim + d
    for d in range(dim):
        for b in range(4):
            c = np.zeros((1, dim), np.int64)
            c[0, d] = 1 << b
            assert binning.cell_hash(c, gs, "particle")[0] == 1 << (b * dim + d)
    np.testing.assert_array_equal(binning.hash2cell(h, gs, "particle"), cells)


def test_dilate_ten_bits():
    v = np.arange(1024)
    for dim in (2, 3):
        d = binning.dilate(v, dim)
        back = np.zeros_like(v)
        for b in range(10):
            back |= ((d >> (b * dim)) & 1) << b
        np.testing.assert_array_equal(back, v)
    assert binning.dilate(np.array([1024 + 5]), 2)[0] == binning.dilate(np.array([5]), 2)[0]


def _instantiate_brute(x, gs, eps, periodic, mode, maxp):
    """Per-particle loops: slot = #(smaller key) + #(same key, smaller index)."""
    B, N = x.shape[:2]
    G = int(np.prod(gs))
    keys = binning.cell_keys(x, gs, eps, periodic, mode).reshape(-1)
    perm = np.zeros(B * N, np.int64)
    for k in range(B * N):
        slot = np.sum(keys < keys[k]) + np.sum(keys[:k] == keys[k])
        perm[k] = slot - (k // N) * N
    bo = np.array([np.sum(keys < c) for c in range(B * G + 1)])
    rows = []
    for c in range(B * G):
        n = int(np.sum(keys == c))
        for s0 in range(0, n, maxp):
            rows.append((c, s0, min(maxp, n - s0), c // G))
    return perm.reshape(B, N), bo, rows


@pytest.mark.parametrize("dim,periodic,mode", [(2, False, "grid"), (2, True, "grid"), (3, False, "grid"),
                                               (2, False, "particle"), (3, True, "particle")])
def test_instantiate_matches_brute_force(dim, periodic, mode):
    rng = np.random.default_rng(3)
    B, N = 2, 60
    gs = (4,) * dim
    x = ((rng.random((B, N, 2 if dim == 2 else 4)) - 0.5) * 1.2).astype(np.float32)
    x[0, :10, :dim] = 0.05  # a crowded cell
    res = binning.instantiate(x, gs, 0.25, periodic, mode, maxp=4)
    perm, bo, rows = _instantiate_brute(x, gs, 0.25, periodic, mode, 4)
    np.testing.assert_array_equal(res["permutation"], perm)
    np.testing.assert_array_equal(res["bin_offsets"], bo)
    if mode == "grid":
        assert res["total_blocks"] == len(rows)
        np.testing.assert_array_equal(res["block_info"][:len(rows)], np.array(rows))
        assert np.all(res["block_info"][len(rows):] == 0)
        assert res["block_info"].shape[0] == binning.max_blocks(gs, N, B, 4, mode)
    # the permutation is a bijection per cloud and stable within each cell
    for b in range(B):
        assert sorted(res["permutation"][b].tolist()) == list(range(N))


def test_bin_unbin_round_trip():
    rng = np.random.default_rng(5)
    x = rng.random((3, 50, 2)).astype(np.float32)
    s = rng.random((3, 50, 7)).astype(np.float32)
    m = rng.random((3, 50)).astype(np.float32)
    res = binning.instantiate(x, (5, 5), 0.3, False, "grid", 8)
    xb, sb, mb = binning.bin_particles(x, s, m, res["permutation"])
    xu, su, mu = binning.unbin_particles(xb, sb, mb, res["permutation"])
    np.testing.assert_array_equal(xu, x)
    np.testing.assert_array_equal(su, s)
    np.testing.assert_array_equal(mu, m)
    # binned keys are sorted
    keys = binning.cell_keys(xb, (5, 5), 0.3, False, "grid").reshape(-1)
    assert np.all(np.diff(keys) >= 0)


def test_max_blocks_formula():
    assert binning.max_blocks((16, 16), 256, 3, 64, "grid") == 3 * min(256, 256 + 4)
    assert binning.max_blocks((4, 4), 4096, 2, 32, "grid") == 2 * (16 + 128)
    assert binning.max_blocks((4, 4), 10, 1, 32, "particle") == 1
