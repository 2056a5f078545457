"""numpy restatement of the reference's spatial-hash binning (test oracle only).

Everything here is integer or exactly-emulated fp32 arithmetic, so results are
compared bit-exactly with the HIP path.

Reference semantics followed:
* cell coordinate: ``floor(x * inv_eps) + G/2`` with ``inv_eps = 1.0f/eps``
  computed in fp32 on the host (``sphops/sph_cuda.cu:1838-1839``,
  ``sphops/utils.cuh:426-440``).  The reference is built with
  ``--use_fast_math`` (``sphops/CMakeLists.txt:26``), i.e. flush-to-zero: a
  subnormal ``x`` or a subnormal product counts as 0.
* boundary: clamp to ``[0, G-1]`` or ``positive_mod`` (``utils.cuh:370-424``).
* hash: row-major ``(z*Gy + y)*Gx + x`` in grid mode, Morton interleave of the
  10 low bits in particle mode (``utils.cuh:442-523``).
* global key ``b*G + hash``; ``bin_offsets`` = exclusive scan of per-cell
  counts over ``B*G + 1`` entries with global values (``sph_cuda.cu:1960-1967``).
* permutation: destination slot of each particle inside its cloud
  (``sph_cuda.cu:60-84``).  The reference's intra-cell order comes from an
  atomic race; the canonical order used here (ascending original index) is one
  of its possible outputs.
* block table rows ``{global_cell, offset_in_cell, count, batch}`` for every
  ``MAXP``-sized slice of every non-empty cell, in cell order, zero rows after
  ``total_blocks`` (``sph_cuda.cu:168-206, 1969-1991``; ``max_blocks`` from
  ``sph_cuda.cu:1849-1854``).
"""
import math

import numpy as np

FLT_MIN = np.float32(np.finfo(np.float32).tiny)
INT32_MIN = -(2 ** 31)
INT32_MAX = 2 ** 31 - 1


def f32(v):
    return np.float32(v)


def inv_eps_f32(eps):
    """``m_config.inv_eps = 1.0f / eps`` with eps already rounded to fp32
    (the nanobind ctor takes ``float eps``; ``sph_cuda.cu:1839``)."""
    return np.float32(1.0) / np.float32(eps)


def floor_cell_ftz(x, inv_eps):
    """``__float2int_rd(x * inv_eps)`` under flush-to-zero, as int64 values that
    are already saturated to the int32 range (``utils.cuh:430-437``).

    NaN converts to 0; out-of-range values saturate (PTX ``cvt.rmi.s32.f32``)."""
    x = np.asarray(x, dtype=np.float32)
    xz = np.where(np.abs(x) < FLT_MIN, np.float32(0.0), x)
    with np.errstate(over="ignore", invalid="ignore"):
        p = (xz * np.float32(inv_eps)).astype(np.float32)
    p = np.where(np.abs(p) < FLT_MIN, np.float32(0.0), p)
    fl = np.floor(p.astype(np.float64))
    out = np.zeros(fl.shape, dtype=np.int64)
    ok = ~np.isnan(fl)
    out[ok] = np.clip(fl[ok], INT32_MIN, INT32_MAX).astype(np.int64)
    return out


def _wrap_i32(v):
    """int32 two's-complement wrap of an int64 array (device ``int`` add)."""
    return ((np.asarray(v, dtype=np.int64) + 2 ** 31) % 2 ** 32) - 2 ** 31


def pos2cell(x, grid_size, eps, periodic):
    """Per-axis integer cell coordinates, shape ``x.shape[:-1] + (D,)``.

    ``x`` holds positions with at least D components (3D positions are float4;
    only x,y,z are used, ``utils.cuh:433-437``)."""
    D = len(grid_size)
    inv = inv_eps_f32(eps)
    cells = []
    for d in range(D):
        G = int(grid_size[d])
        c = _wrap_i32(floor_cell_ftz(x[..., d], inv) + G // 2)
        if periodic:
            c = np.mod(c, G)  # equals i & (G-1) for power-of-two G
        else:
            c = np.clip(c, 0, G - 1)
        cells.append(c)
    return np.stack(cells, axis=-1)


def dilate(v, dim):
    """Spread the 10 low bits of ``v`` with 1 (2D) or 2 (3D) zero bits between
    them (Morton interleave helper, ``utils.cuh:481-501``); written as a plain
    bit loop so it is independent of the reference's mask constants."""
    v = np.asarray(v, dtype=np.int64) & 0x3FF
    out = np.zeros_like(v)
    step = dim
    for bit in range(10):
        out |= ((v >> bit) & 1) << (bit * step)
    return out


def cell_hash(cells, grid_size, mode):
    """Hash of integer cell coordinates (``utils.cuh:442-453``)."""
    D = len(grid_size)
    if mode == "grid":
        if D == 2:
            return cells[..., 1] * grid_size[0] + cells[..., 0]
        return (cells[..., 2] * grid_size[1] + cells[..., 1]) * grid_size[0] + cells[..., 0]
    h = dilate(cells[..., 0], D) | (dilate(cells[..., 1], D) << 1)
    if D == 3:
        h |= dilate(cells[..., 2], D) << 2
    return h


def hash2cell(h, grid_size, mode):
    """Inverse of :func:`cell_hash` for in-range hashes."""
    D = len(grid_size)
    h = np.asarray(h, dtype=np.int64)
    if mode == "grid":
        x = h % grid_size[0]
        if D == 2:
            return np.stack([x, h // grid_size[0]], axis=-1)
        y = (h // grid_size[0]) % grid_size[1]
        z = h // (grid_size[0] * grid_size[1])
        return np.stack([x, y, z], axis=-1)
    comps = []
    for d in range(D):
        c = np.zeros_like(h)
        for bit in range(10):
            c |= ((h >> (bit * D + d)) & 1) << bit
        comps.append(c)
    return np.stack(comps, axis=-1)


def max_blocks(grid_size, num_particles, batch_size, maxp, mode):
    """``HashGrid::_init`` block-table capacity (``sph_cuda.cu:1849-1860``)."""
    if mode != "grid":
        return 1
    G = int(np.prod(grid_size))
    per_batch = min(num_particles, G + (num_particles + maxp - 1) // maxp)
    return per_batch * batch_size


def cell_keys(x, grid_size, eps, periodic, mode):
    """Global sort key ``b*G + hash`` for every particle, shape (B, N), int64."""
    B, N = x.shape[:2]
    G = int(np.prod(grid_size))
    cells = pos2cell(x, grid_size, eps, periodic)
    h = cell_hash(cells, grid_size, mode)
    return h + (np.arange(B, dtype=np.int64) * G)[:, None]


def instantiate(x, grid_size, eps, periodic, mode, maxp):
    """Oracle for ``HashGrid.instantiate`` (``sphops/sph.py:80-105``).

    Returns a dict with ``permutation`` (B,N) int32, ``bin_offsets`` (B*G+1,)
    int32, ``block_info`` (max_blocks,4) int32 (grid mode; ``None`` in particle
    mode, where the reference leaves the tensor untouched), ``total_blocks``,
    ``keys`` (B,N) and ``order`` (B*N,) = source index of each sorted slot."""
    x = np.asarray(x, dtype=np.float32)
    B, N = x.shape[:2]
    G = int(np.prod(grid_size))
    keys = cell_keys(x, grid_size, eps, periodic, mode)
    flat = keys.reshape(-1)
    order = np.argsort(flat, kind="stable")
    slot = np.empty(B * N, dtype=np.int64)
    slot[order] = np.arange(B * N, dtype=np.int64)
    perm = (slot.reshape(B, N) - (np.arange(B, dtype=np.int64) * N)[:, None]).astype(np.int32)
    counts = np.bincount(flat, minlength=B * G).astype(np.int64)
    offsets = np.zeros(B * G + 1, dtype=np.int64)
    np.cumsum(counts, out=offsets[1:])
    res = dict(permutation=perm, bin_offsets=offsets.astype(np.int32), keys=keys,
               order=order, counts=counts)
    if mode == "grid":
        mb = max_blocks(grid_size, N, B, maxp, mode)
        nz = np.nonzero(counts)[0]
        nblk = (counts[nz] + maxp - 1) // maxp
        total = int(nblk.sum())
        info = np.zeros((mb, 4), dtype=np.int64)
        cell_rep = np.repeat(nz, nblk)
        first = np.repeat(np.cumsum(nblk) - nblk, nblk)
        sub = np.arange(total, dtype=np.int64) - first
        info[:total, 0] = cell_rep
        info[:total, 1] = sub * maxp
        info[:total, 2] = np.minimum(maxp, counts[cell_rep] - sub * maxp)
        info[:total, 3] = cell_rep // G
        res["block_info"] = info.astype(np.int32)
        res["total_blocks"] = total
    else:
        res["block_info"] = None
        res["total_blocks"] = 0
    return res


def bin_particles(x, s, m, perm):
    """Scatter ``out[b, perm[b,i]] = in[b, i]`` (``sph_cuda.cu:86-123``)."""
    B, N = perm.shape
    bi = np.arange(B)[:, None]
    xo = np.empty_like(x)
    so = np.empty_like(s)
    mo = np.empty_like(m)
    xo[bi, perm] = x
    so[bi, perm] = s
    mo[bi, perm] = m
    return xo, so, mo


def unbin_particles(xb, sb, mb, perm):
    """Gather ``out[b, i] = in[b, perm[b,i]]`` (``sph_cuda.cu:125-167``)."""
    B, N = perm.shape
    bi = np.arange(B)[:, None]
    return xb[bi, perm], sb[bi, perm], mb[bi, perm]


def wrap_positions(x, grid_size, eps, periodic):
    """``HashGrid.wrap_positions`` (``sphops/sph.py:107-123``): remainder into
    ``[-L/2, L/2)`` per axis with ``L = G*eps``; identity when clamped.  Only
    the first D components are returned (the reference stacks D axes)."""
    if not periodic:
        return x
    D = len(grid_size)
    out = []
    for d in range(D):
        L = np.float32(grid_size[d] * eps)  # python float product, then fp32 tensor
        half = np.float32(0.5) * L
        v = np.asarray(x[..., d], dtype=np.float32) + half
        out.append((np.mod(v, L) - half).astype(np.float32))
    return np.stack(out, axis=-1)


def required_bits(num_keys):
    """Number of radix bits that cover keys in ``[0, num_keys)``."""
    return max(1, int(math.ceil(math.log2(max(2, num_keys)))))
