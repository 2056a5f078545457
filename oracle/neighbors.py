"""Neighbour candidates exactly as the reference traverses them (oracle only).

For a binned particle i in cell c, the reference visits the 3^D cells around c
(clamped: only in-bounds cells; periodic: wrapped indices), reads each cell's
contiguous slice ``[bin_offsets[k], bin_offsets[k+1])`` and keeps the pairs
with ``|r|^2 < eps^2`` evaluated in fp32 (``sphops/sph_cuda.cu:1561-1640`` grid
mode, ``:324-346`` particle mode; ``sphops/utils.cuh:321-362`` for the periodic
minimum-image displacement).  The displacement and the squared distance are
emulated here operation by operation in fp32 (no fused multiply-add), which is
the arithmetic the HIP kernels use, so the pair set is bit-identical.
"""
import itertools
from dataclasses import dataclass

import numpy as np

from . import binning


@dataclass(frozen=True)
class GridSpec:
    """Static grid parameters (``HashGrid.__init__``, ``sphops/sph.py:48-78``)."""
    grid_size: tuple
    eps: float
    periodic: bool
    mode: str = "grid"
    maxp: int = 64

    @property
    def dim(self):
        return len(self.grid_size)

    @property
    def num_cells(self):
        return int(np.prod(self.grid_size))

    @property
    def pos_width(self):
        return 2 if self.dim == 2 else 4

    def eps32(self):
        return np.float32(self.eps)

    def eps2_f32(self):
        e = np.float32(self.eps)
        return np.float32(e * e)

    def box_f32(self):
        """``L[d] = float(G_d) * eps`` and ``0.5f * L`` in fp32 (``sph_cuda.cu:1842-1846``)."""
        e = np.float32(self.eps)
        L = np.array([np.float32(np.float32(g) * e) for g in self.grid_size], dtype=np.float32)
        return L, (np.float32(0.5) * L).astype(np.float32)

    def coefficients(self):
        """(poly6, spiky) coefficients as ``HashGrid::_init`` derives them:
        ``ie = 1.0f/eps`` and its powers by fp32 multiplies, times a double
        constant, rounded to fp32 (``sph_cuda.cu:1862-1878``)."""
        import math
        ie = binning.inv_eps_f32(self.eps)
        ie2 = np.float32(ie * ie)
        ie4 = np.float32(ie2 * ie2)
        if self.dim == 2:
            ie5 = np.float32(ie4 * ie)
            ie8 = np.float32(ie4 * ie4)
            c6 = np.float32(4.0 / math.pi * float(ie8))
            cs = np.float32(10.0 / math.pi * float(ie5))
        else:
            ie6 = np.float32(ie4 * ie2)
            ie9 = np.float32(np.float32(ie4 * ie4) * ie)
            c6 = np.float32(315.0 / (64.0 * math.pi) * float(ie9))
            cs = np.float32(15.0 / math.pi * float(ie6))
        return float(c6), float(cs)

    def check(self):
        if self.periodic and min(self.grid_size) < 3:
            raise ValueError("periodic grids need at least 3 cells per axis")


def displacement_f32(x_from, x_to, spec):
    """``GridConfig::displacement(from, to)`` in fp32: ``to - from``, wrapped to
    ``[-L/2, L/2)`` with ``fmodf`` when periodic.  Inputs (..., >=D) fp32."""
    D = spec.dim
    L, half = spec.box_f32()
    out = []
    for d in range(D):
        v = (np.asarray(x_to[..., d], np.float32) - np.asarray(x_from[..., d], np.float32)).astype(np.float32)
        if spec.periodic:
            t = np.fmod((v + half[d]).astype(np.float32), L[d]).astype(np.float32)
            t = np.where(t < 0, (t + L[d]).astype(np.float32), t)
            v = (t - half[d]).astype(np.float32)
        out.append(v)
    return np.stack(out, axis=-1)


def sqnorm_f32(r):
    """``dot(r, r)`` evaluated left to right in fp32 without contraction."""
    acc = (r[..., 0] * r[..., 0]).astype(np.float32)
    for d in range(1, r.shape[-1]):
        acc = (acc + (r[..., d] * r[..., d]).astype(np.float32)).astype(np.float32)
    return acc


def stencil_offsets(dim):
    return np.array(list(itertools.product((-1, 0, 1), repeat=dim)), dtype=np.int64)[:, ::-1]


@dataclass
class Pairs:
    """In-radius pairs grouped by query.  ``q`` indexes the query list,
    ``i``/``j`` are flat binned indices (``b*N + slot``), ``r`` is the fp32
    displacement ``x_j - x_i`` and ``rb`` the fp32 displacement ``x_i - x_j``
    (both wrapped), ``starts`` the first pair of each query, ``ncand`` the
    number of stencil candidates (particles in the query's 3^D cells) of
    each query."""
    q: np.ndarray
    i: np.ndarray
    j: np.ndarray
    r: np.ndarray
    rb: np.ndarray
    starts: np.ndarray
    queries: np.ndarray
    ncand: np.ndarray = None


def candidate_pairs(xb, bin_offsets, spec, queries=None):
    """Enumerate the in-radius pairs of ``queries`` (flat binned indices;
    default: all) against the stencil of their cell."""
    spec.check()
    xb = np.asarray(xb, dtype=np.float32)
    B, N = xb.shape[:2]
    flat = xb.reshape(B * N, -1)
    if queries is None:
        queries = np.arange(B * N, dtype=np.int64)
    queries = np.asarray(queries, dtype=np.int64)
    Q = queries.shape[0]
    G = spec.num_cells
    gs = np.array(spec.grid_size, dtype=np.int64)
    ci = binning.pos2cell(flat[queries], spec.grid_size, spec.eps, spec.periodic)
    offs = stencil_offsets(spec.dim)
    nc = ci[:, None, :] + offs[None, :, :]
    if spec.periodic:
        valid = np.ones(nc.shape[:2], dtype=bool)
        nc = np.mod(nc, gs)
    else:
        valid = np.all((nc >= 0) & (nc < gs), axis=-1)
        nc = np.clip(nc, 0, gs - 1)
    h = binning.cell_hash(nc, spec.grid_size, spec.mode)
    gk = (queries // N)[:, None] * G + h
    bo = np.asarray(bin_offsets, dtype=np.int64)
    start = bo[gk]
    cnt = np.where(valid, bo[gk + 1] - start, 0)
    cnt_flat = cnt.ravel()
    rep = np.repeat(np.arange(cnt_flat.size, dtype=np.int64), cnt_flat)
    first = np.repeat(np.cumsum(cnt_flat) - cnt_flat, cnt_flat)
    within = np.arange(rep.size, dtype=np.int64) - first
    j = start.ravel()[rep] + within
    qidx = rep // offs.shape[0]
    i = queries[qidx]
    r = displacement_f32(flat[i], flat[j], spec)
    keep = sqnorm_f32(r) < spec.eps2_f32()
    qidx, i, j, r = qidx[keep], i[keep], j[keep], r[keep]
    rb = displacement_f32(flat[j], flat[i], spec)
    counts = np.bincount(qidx, minlength=Q)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int64)
    return Pairs(q=qidx, i=i, j=j, r=r, rb=rb, starts=starts, queries=queries, ncand=cnt.sum(axis=1))
