"""Shared test utilities: case construction, oracle evaluation, tolerances.

Tolerance used for every fp32 output (written once, here):
    |gpu - ref| <= RTOL * |ref| + ATOL * (mag + rms)
with RTOL = 1e-5, ATOL = 1e-6, ``mag`` the oracle's sum of absolute pair
terms for that element (the scale of fp32 summation error; equal to |ref|
when no term cancels) and ``rms`` the root-mean-square of the whole
reference tensor (the absolute 1e-6 expressed in the tensor's own units; it
covers elements whose only terms are pairs at |r| ~ h, where fp32 and the
exact value differ by ~1e-14 of a typical term but mag is ~0).  Integer and
index outputs are compared exactly.
"""
from dataclasses import dataclass, field

import numpy as np

from oracle import binning, neighbors, sph

RTOL = 1e-5
ATOL = 1e-6


@dataclass
class Case:
    name: str
    x: np.ndarray
    s: np.ndarray
    m: np.ndarray
    grid_size: tuple
    eps: float
    periodic: bool
    mode: str
    maxp: int
    queries: np.ndarray = None   # flat binned indices checked by the oracle (None: all)
    extra: dict = field(default_factory=dict)

    @property
    def dim(self):
        return len(self.grid_size)

    @property
    def B(self):
        return self.x.shape[0]

    @property
    def N(self):
        return self.x.shape[1]

    @property
    def C(self):
        return self.s.shape[2]

    @property
    def spec(self):
        return neighbors.GridSpec(tuple(self.grid_size), self.eps, self.periodic, self.mode, self.maxp)

    @property
    def boundary(self):
        return "periodic" if self.periodic else "clamped"


def pack_pos(x2or3):
    B, N, D = x2or3.shape
    if D == 2:
        return np.ascontiguousarray(x2or3, dtype=np.float32)
    out = np.zeros((B, N, 4), dtype=np.float32)
    out[..., :3] = x2or3
    return out


def random_case(name, B, N, C, dim, grid, eps, periodic, mode="grid", maxp=64, sigma=1.0, seed=42,
                uniform=True, mass="rand"):
    """The reference's test.py inputs (``sphops/test.py:107-154``): positions
    (rand-0.5)*2*sigma (or randn*sigma), states randn, masses rand+1e-3."""
    rng = np.random.default_rng(seed)
    if uniform:
        x = (rng.random((B, N, dim)) - 0.5) * 2.0 * sigma
    else:
        x = rng.standard_normal((B, N, dim)) * sigma
    s = rng.standard_normal((B, N, C)).astype(np.float32)
    m = (rng.random((B, N)) + 1e-3).astype(np.float32) if mass == "rand" else np.ones((B, N), np.float32)
    return Case(name, pack_pos(x), s, m, (grid,) * dim if np.isscalar(grid) else tuple(grid), eps, periodic,
                mode, maxp)


def workload_case(wl, queries=None, seed=7):
    rng = np.random.default_rng(seed)
    m = np.ones((wl.B, wl.N), np.float32)
    return Case(wl.name, wl.x, wl.s, m, wl.grid_size, wl.h, wl.periodic, wl.mode, wl.maxp, queries)


def oracle_binning(c):
    return binning.instantiate(c.x, c.grid_size, c.eps, c.periodic, c.mode, c.maxp)


def oracle_context(c, xb, bin_offsets):
    pairs = neighbors.candidate_pairs(xb, bin_offsets, c.spec, c.queries)
    return sph.Context(pairs, c.spec)


def assert_close(name, got, ref, mag, rtol=RTOL, atol=ATOL, skip=None):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    mag = np.asarray(mag, dtype=np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    err = np.abs(got - ref)
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    bound = rtol * np.abs(ref) + atol * (mag + rms)
    bad = err > bound
    if skip is not None:
        sk = np.broadcast_to(skip.reshape(skip.shape + (1,) * (bad.ndim - skip.ndim)), bad.shape)
        bad &= ~sk
    if bad.any():
        ratio = np.where(bad, err / np.maximum(bound, 1e-300), 0.0)
        idx = np.unravel_index(np.argmax(ratio), ratio.shape)
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{bad.size} elements out of tolerance; worst at {idx}: "
            f"got {got[idx]!r} ref {ref[idx]!r} err {err[idx]:.3e} bound {bound[idx]:.3e} "
            f"mag {mag[idx]:.3e} rms {rms:.3e}")
    return float(np.max(err / np.maximum(bound, 1e-300))) if err.size else 0.0


def hybrid_bound(raw, raw_mag, M_mag, L):
    """First-order error scale of raw @ inv(M): |d raw| |L| + |raw| |L| |dM| |L|."""
    aL = np.abs(L)
    t1 = np.einsum("qfd,qde->qfe", raw_mag, aL)
    LML = np.einsum("qab,qbc,qcd->qad", aL, M_mag, aL)
    t2 = np.einsum("qfd,qde->qfe", np.abs(raw), LML)
    return t1 + t2


def indefinite_matrices(dim, tol=1e-3, seed=8):
    """Symmetric indefinite matrices Q diag(e) Q^T with one negative
    eigenvalue: ``big`` has det < -tol (inverted), ``small`` has
    -tol < det < 0 (the |det| < tol branch gives the identity)."""
    rng = np.random.default_rng(seed)
    out = {}
    for kind, lo, hi in (("big", 0.05, 2.0), ("small", 1e-4, 2.5e-4)):
        Q, _ = np.linalg.qr(rng.standard_normal((64, dim, dim)))
        e = rng.uniform(lo, hi, (64, dim)) ** (1.0 / dim) * rng.choice([1.0, 1.5], (64, dim))
        e[:, 0] *= -1.0
        out[kind] = np.einsum("qab,qb,qcb->qac", Q, e, Q)
    return out
