"""Native class surface of the gfx950 sphops library.

Mirrors the reference's nanobind module ``sph_cuda``
(``sphops/sph_cuda.cu:3228-3441``): the classes ``HashGrid2DPeriodic``,
``HashGrid2DBox``, ``HashGrid3DPeriodic``, ``HashGrid3DBox`` and their
particle-mode ``VHashGrid*`` twins, with the same constructor arguments,
read-only properties and method argument order, plus the module function
``safe_inv_sym_mat``.

Argument checks follow the reference: a tensor of the wrong dtype, device,
layout or rank raises ``TypeError`` (nanobind's ndarray type check,
``sph_cuda.cu:12-18``); a wrong size raises ``RuntimeError`` with the
reference's message (``validate_array_shape``, ``utils.cuh:526-566``); a
failure inside the library raises ``RuntimeError``.

Every call enqueues work on the current HIP stream of the tensor's device and
returns without synchronising.
"""
import ctypes
import os
import weakref

import torch

from . import _native

_lib = _native.lib
_check = _native.check

CLAMPED, PERIODIC = 0, 1
MODE_GRID, MODE_PARTICLE = 0, 1


def _stream(t):
    """torch's current stream on t's device, as the raw handle (the C ABI's
    `stream` argument); the raw query skips building a Stream object."""
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(t.device.index))


def _arr(t, name, dtype, ndim):
    """nanobind-style type check: dtype, device, C-contiguity and rank."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if t.device.type != "cuda":
        raise TypeError(f"{name}: expected a GPU tensor, got device {t.device}")
    if not t.is_contiguous():
        raise TypeError(f"{name}: expected a C-contiguous tensor")
    if t.dim() != ndim:
        raise TypeError(f"{name}: expected {ndim} dimensions, got {t.dim()}")
    return ctypes.c_void_p(t.data_ptr())


def _validate_shape(t, expected, name):
    """``validate_array_shape`` (``sphops/utils.cuh:526-566``)."""
    if t.dim() != len(expected):
        raise RuntimeError(f"{name} must have {len(expected)} dimensions, got {t.dim()}")
    if tuple(t.shape) != tuple(expected):
        exp = "(" + ", ".join(str(v) for v in expected) + ")"
        act = "(" + ", ".join(str(v) for v in t.shape) + ")"
        raise RuntimeError(f"{name} must have shape {exp}, got {act}")


_F32, _I32 = torch.float32, torch.int32


def next_index_capacity(total, unstored, used_capacity, slack_shift):
    """Index capacity for the next snapshot's neighbour list from the last
    list's pair total, the pairs of its rows that were not stored and the
    capacity it had: the total plus a margin of total >> slack_shift plus
    1024.  A list that did not fit although its buffer held the total had
    uneven slices (the fill allocates rows per slice of the buffer), so the
    margin grows (the shift drops, down to 1).  Returns (capacity, shift)."""
    if unstored and used_capacity >= total and slack_shift > 1:
        slack_shift -= 1
    return total + (total >> slack_shift) + 1024, slack_shift


class NeighborPlan(tuple):
    """A snapshot's neighbour list and its schedules (``neighbor_list``):
    the tuple ``(start, count, index, order, waves, wave_count, waves_split,
    wave_count_split[, device counts])``, plus ``tiles``: the cell tiles of
    the pass-B backward ``(units, unit count (device), order of the other
    particles, their split waves, their wave count (host bound), its device
    copy)``, or None; and ``cells``: the cell tiles of
    ``sphops_neighbor_fill_tiled`` ``(own-cell entries per particle, cell
    table, its count (device))``, or None."""

    def __new__(cls, *items):
        return super().__new__(cls, items)

    tiles = None
    cells = None
    capacity = 0


class _HashGridNative:
    """Common implementation of the eight grid classes."""

    _dim = 2
    _boundary = CLAMPED
    _mode = MODE_GRID

    def __init__(self, *args, **kwargs):
        names = ["grid_size_x", "grid_size_y"] + (["grid_size_z"] if self._dim == 3 else []) + [
            "eps", "particle_count", "batch_size", "max_particles_per_block"]
        vals = dict(zip(names, args))
        for k, v in kwargs.items():
            if k not in names:
                raise TypeError(f"unexpected keyword argument {k!r}")
            if k in vals:
                raise TypeError(f"duplicate argument {k!r}")
            vals[k] = v
        vals.setdefault("max_particles_per_block", 64)
        missing = [n for n in names if n not in vals]
        if missing:
            raise TypeError(f"missing arguments: {missing}")
        self._sizes = [int(vals[n]) for n in names[: self._dim]]
        self._eps = float(torch.tensor(float(vals["eps"]), dtype=torch.float32))
        self._n = int(vals["particle_count"])
        self._b = int(vals["batch_size"])
        self._maxp = int(vals["max_particles_per_block"])
        for name, v in (("particle_count", self._n), ("batch_size", self._b),
                        ("max_particles_per_block", self._maxp)):
            if v < 0 or v >= 2 ** 32:
                raise TypeError(f"{name} must fit an unsigned 32-bit integer")
        gs = (ctypes.c_int32 * self._dim)(*self._sizes)
        handle = ctypes.c_void_p()
        self._h = None
        _check(_lib.sphops_grid_create(self._dim, self._boundary, self._mode, gs, ctypes.c_float(self._eps),
                                       self._n, self._b, self._maxp, ctypes.byref(handle)))
        self._h = handle
        # kept on the instance: at interpreter exit module globals may already be gone
        self._destroy = _lib.sphops_grid_destroy
        self._device = torch.device("cuda", torch.cuda.current_device())
        self._pw = 2 if self._dim == 2 else 4
        self._cells = 1
        for s in self._sizes:
            self._cells *= s
        c6, cs = ctypes.c_float(), ctypes.c_float()
        _check(_lib.sphops_grid_coefficients(self._h, ctypes.byref(c6), ctypes.byref(cs)))
        self.smoothing_coef, self.spiky_coef = c6.value, cs.value

    def __del__(self):
        h = getattr(self, "_h", None)
        destroy = getattr(self, "_destroy", None)
        if h and destroy is not None:
            destroy(h)
            self._h = None

    # ---- properties (sph_cuda.cu:3229-3237)
    @property
    def grid_size_x(self):
        return self._sizes[0]

    @property
    def grid_size_y(self):
        return self._sizes[1]

    @property
    def eps(self):
        return self._eps

    @property
    def particle_count(self):
        return self._n

    @property
    def batch_size(self):
        return self._b

    @property
    def max_blocks(self):
        return int(_lib.sphops_grid_max_blocks(self._h))

    @property
    def max_particles_per_block(self):
        return self._maxp

    @property
    def cell_count(self):
        return self._cells

    # ---- shape helpers
    def _pos(self, t, name):
        p = _arr(t, name, _F32, 3)
        _validate_shape(t, (self._b, self._n, self._pw), name)
        return p

    def _bn(self, t, name):
        p = _arr(t, name, _F32, 2)
        _validate_shape(t, (self._b, self._n), name)
        return p

    def _state(self, t, name, C):
        p = _arr(t, name, _F32, 3)
        _validate_shape(t, (self._b, self._n, C), name)
        return p

    def _offsets(self, t):
        p = _arr(t, "bin_offsets", _I32, 1)
        _validate_shape(t, (self._b * self._cells + 1,), "bin_offsets")
        return p

    def _blocks(self, t):
        if t is None:
            return ctypes.c_void_p()
        if not isinstance(t, torch.Tensor) or t.dtype != _I32 or t.dim() != 2 or t.shape[-1] != 4:
            raise TypeError("block_info: expected an int32 tensor of shape (max_blocks, 4)")
        if self._mode == MODE_GRID:
            _validate_shape(t, (self.max_blocks, 4), "block_info")
        return ctypes.c_void_p(t.data_ptr())

    # ---- binning (sph_cuda.cu:1926-2056)
    def initialize(self, positions, permutation, bin_offsets, block_info, total_blocks=None, inverse=None):
        """``inverse`` (B, N) int32, optional: receives the inverse permutation
        (``sphops_initialize_inverse``), with which ``bin_particles`` performs
        the unbin as a scatter."""
        x = self._pos(positions, "positions")
        bo = self._offsets(bin_offsets)
        pm = _arr(permutation, "permutation", _I32, 2)
        _validate_shape(permutation, (self._b, self._n), "permutation")
        if self._mode == MODE_GRID:
            bi = _arr(block_info, "block_info", _I32, 2)
            _validate_shape(block_info, (self.max_blocks, 4), "block_info")
        else:
            bi = ctypes.c_void_p(block_info.data_ptr()) if block_info is not None else ctypes.c_void_p()
        tb = ctypes.c_void_p()
        if total_blocks is not None:
            tb = _arr(total_blocks, "total_blocks", _I32, 1)
        if inverse is None:
            _check(_lib.sphops_initialize(self._h, x, pm, bo, bi, tb, _stream(positions)))
        else:
            iv = _arr(inverse, "inverse", _I32, 2)
            _validate_shape(inverse, (self._b, self._n), "inverse")
            _check(_lib.sphops_initialize_inverse(self._h, x, pm, iv, bo, bi, tb, _stream(positions)))
        # the library derived the list fill's work split from the same sorted
        # keys; a list built on this very tensor, unmodified, reuses it
        self._split_source = (weakref.ref(bin_offsets), bin_offsets._version)

    def bin_particles(self, input_positions, input_state, input_mass, permutation, output_positions,
                      output_state, output_mass):
        C = input_state.shape[2] if input_state.dim() == 3 else -1
        args = self._move_args(input_positions, input_state, input_mass, permutation, output_positions,
                               output_state, output_mass, C,
                               ("input_positions", "input_state", "input_mass", "permutation",
                                "output_positions", "output_state", "output_mass"))
        _check(_lib.sphops_bin_particles(self._h, *args, C, _stream(input_positions)))

    def backward_bin_particles(self, grad_output_positions, grad_output_state, grad_output_mass, permutation,
                               grad_input_positions, grad_input_state, grad_input_mass):
        C = grad_output_state.shape[2] if grad_output_state.dim() == 3 else -1
        args = self._move_args(grad_output_positions, grad_output_state, grad_output_mass, permutation,
                               grad_input_positions, grad_input_state, grad_input_mass, C,
                               ("grad_output_positions", "grad_output_state", "grad_output_mass", "permutation",
                                "grad_input_positions", "grad_input_state", "grad_input_mass"))
        _check(_lib.sphops_backward_bin_particles(self._h, *args, C, _stream(grad_output_positions)))

    def _move_args(self, ip, is_, im, perm, op, os_, om, C, names):
        # the masses may be None together: their rows are not moved
        if (im is None) != (om is None):
            raise ValueError(f"{names[2]} and {names[6]} must both be tensors or both be None")
        bn = lambda t, name: ctypes.c_void_p() if t is None else self._bn(t, name)
        out = [self._pos(ip, names[0]), self._state(is_, names[1], C), bn(im, names[2])]
        out.append(_arr(perm, names[3], _I32, 2))
        _validate_shape(perm, (self._b, self._n), names[3])
        out += [self._pos(op, names[4]), self._state(os_, names[5], C), bn(om, names[6])]
        return out

    # ---- forward operators (sph_cuda.cu:2058-2499)
    def density_forward(self, binned_positions, mass, rho, bin_offsets, block_info):
        _check(_lib.sphops_density_forward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(mass, "mass"),
            self._bn(rho, "rho"), self._offsets(bin_offsets), self._blocks(block_info),
            _stream(binned_positions)))

    def count_forward(self, binned_positions, count, bin_offsets, block_info):
        _check(_lib.sphops_count_forward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(count, "count"),
            self._offsets(bin_offsets), self._blocks(block_info), _stream(binned_positions)))

    def blur_forward(self, binned_positions, rho, mass, state_in, state_out, bin_offsets, block_info):
        C = state_in.shape[2] if state_in.dim() == 3 else -1
        _check(_lib.sphops_blur_forward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(rho, "rho"),
            self._bn(mass, "mass"), self._state(state_in, "state_in", C),
            self._state(state_out, "state_out", C), C, self._offsets(bin_offsets), self._blocks(block_info),
            _stream(binned_positions)))

    def gradient_forward(self, binned_positions, rho, mass, state_in, state_gradient_out, bin_offsets, block_info):
        C = state_in.shape[2] if state_in.dim() == 3 else -1
        go = _arr(state_gradient_out, "state_gradient_out", _F32, 4)
        _validate_shape(state_gradient_out, (self._b, self._n, C, self._dim), "state_gradient_out")
        _check(_lib.sphops_gradient_forward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(rho, "rho"),
            self._bn(mass, "mass"), self._state(state_in, "state_in", C), go, C, self._offsets(bin_offsets),
            self._blocks(block_info), _stream(binned_positions)))

    def gradient_hybrid_forward(self, binned_positions, rho, mass, state_in, out, bin_offsets, block_info,
                                tol=1e-3):
        """Fused ``raw @ safe_inv(M, tol)`` (no native counterpart in the
        reference; replaces the composite of ``sphops/sph.py:474-484``)."""
        C = state_in.shape[2] if state_in.dim() == 3 else -1
        go = _arr(out, "out", _F32, 4)
        _validate_shape(out, (self._b, self._n, C, self._dim), "out")
        _check(_lib.sphops_gradient_hybrid_forward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(rho, "rho"),
            self._bn(mass, "mass"), self._state(state_in, "state_in", C), go, C, ctypes.c_float(tol),
            self._offsets(bin_offsets), self._blocks(block_info), _stream(binned_positions)))

    def density_gradient_forward(self, binned_positions, mass, density_gradient_out, bin_offsets, block_info):
        go = _arr(density_gradient_out, "density_gradient_out", _F32, 3)
        _validate_shape(density_gradient_out, (self._b, self._n, self._dim), "density_gradient_out")
        _check(_lib.sphops_density_gradient_forward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(mass, "mass"), go,
            self._offsets(bin_offsets), self._blocks(block_info), _stream(binned_positions)))

    def moment_matrix_forward(self, binned_positions, rho, mass, moment_matrix_out, bin_offsets, block_info):
        mo = _arr(moment_matrix_out, "moment_matrix_out", _F32, 4)
        _validate_shape(moment_matrix_out, (self._b, self._n, self._dim, self._dim), "moment_matrix_out")
        _check(_lib.sphops_moment_matrix_forward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(rho, "rho"),
            self._bn(mass, "mass"), mo, self._offsets(bin_offsets), self._blocks(block_info),
            _stream(binned_positions)))

    # ---- backward operators (sph_cuda.cu:2501-3046)
    def density_backward(self, binned_positions, mass, dL_rho_out, grad_x, bin_offsets, block_info, dLdx=True):
        if not dLdx:
            return
        _check(_lib.sphops_density_backward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(mass, "mass"),
            self._bn(dL_rho_out, "grad_output_rho"), self._pos(grad_x, "grad_x"), self._offsets(bin_offsets),
            self._blocks(block_info), 1, _stream(binned_positions)))

    def blur_backward(self, binned_positions, rho, mass, state_in, dL_blur_state_out, grad_x, grad_s, grad_rho,
                      bin_offsets, block_info, dLdx=True, dLds=True, dLdrho=True):
        if not (dLdx or dLds or dLdrho):
            return
        C = state_in.shape[2] if state_in.dim() == 3 else -1
        ds_only = dLds and not dLdx and not dLdrho
        gx = ctypes.c_void_p() if ds_only else self._pos(grad_x, "grad_x")
        gr = ctypes.c_void_p() if ds_only else self._bn(grad_rho, "grad_rho")
        _check(_lib.sphops_blur_backward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(rho, "rho"),
            self._bn(mass, "mass"), self._state(state_in, "state_in", C),
            self._state(dL_blur_state_out, "dL_blur_state_out", C), gx, self._state(grad_s, "grad_s", C), gr, C,
            self._offsets(bin_offsets), self._blocks(block_info), int(bool(dLdx)), int(bool(dLds)),
            int(bool(dLdrho)), _stream(binned_positions)))

    def density_gradient_backward(self, binned_positions, mass, dL_density_gradient_out, grad_x, bin_offsets,
                                  block_info, dLdx=True):
        if not dLdx:
            return
        dl = _arr(dL_density_gradient_out, "dL_density_gradient_out", _F32, 3)
        _validate_shape(dL_density_gradient_out, (self._b, self._n, self._dim), "dL_density_gradient_out")
        _check(_lib.sphops_density_gradient_backward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(mass, "mass"), dl,
            self._pos(grad_x, "grad_x"), self._offsets(bin_offsets), self._blocks(block_info), 1,
            _stream(binned_positions)))

    def gradient_backward(self, binned_positions, rho, mass, state_in, dL_grad_state_out, grad_x, grad_s, grad_rho,
                          bin_offsets, block_info, dLdx=True, dLds=True, dLdrho=True):
        if not (dLdx or dLds or dLdrho):
            return
        C = state_in.shape[2] if state_in.dim() == 3 else -1
        dl = _arr(dL_grad_state_out, "dL_grad_state_out", _F32, 4)
        _validate_shape(dL_grad_state_out, (self._b, self._n, C, self._dim), "dL_grad_state_out")
        ds_only = dLds and not dLdx and not dLdrho
        gx = ctypes.c_void_p() if ds_only else self._pos(grad_x, "grad_x")
        gr = ctypes.c_void_p() if ds_only else self._bn(grad_rho, "grad_rho")
        _check(_lib.sphops_gradient_backward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(rho, "rho"),
            self._bn(mass, "mass"), self._state(state_in, "state_in", C), dl, gx,
            self._state(grad_s, "grad_s", C), gr, C, self._offsets(bin_offsets), self._blocks(block_info),
            int(bool(dLdx)), int(bool(dLds)), int(bool(dLdrho)), _stream(binned_positions)))

    def moment_matrix_backward(self, binned_positions, rho, mass, dL_moment_matrix_out, grad_x, grad_rho,
                               bin_offsets, block_info, dLdx=True, dLdrho=True):
        if not (dLdx or dLdrho):
            return
        dl = _arr(dL_moment_matrix_out, "dL_moment_matrix_out", _F32, 4)
        _validate_shape(dL_moment_matrix_out, (self._b, self._n, self._dim, self._dim), "dL_moment_matrix_out")
        _check(_lib.sphops_moment_matrix_backward(
            self._h, self._pos(binned_positions, "binned_positions"), self._bn(rho, "rho"),
            self._bn(mass, "mass"), dl, self._pos(grad_x, "grad_x"), self._bn(grad_rho, "grad_rho"),
            self._offsets(bin_offsets), self._blocks(block_info), 1, 1, _stream(binned_positions)))


    # ---- generic operator interface with an optional neighbour list
    def neighbor_list(self, x_bin, bin_offsets):
        """In-radius neighbour list of the binned particles plus its
        traversal schedules, as a :class:`NeighborPlan`: ``(start (B*N,),
        count (B*N,), index, order (B*N,), waves (2 words per wave), wave
        launch estimate, waves_split, its estimate, device counts)``.  Row i
        is ``index[start[i] : start[i] + count[i]]``; a particle whose row did
        not fit in ``index`` has ``count = -1 - (its stencil candidates)``
        and the operators walk its stencil instead, so results never depend
        on the buffer sizes.  Nothing is read back synchronously: the index
        capacity and the launch sizes are estimates from the previous
        snapshot's totals, copied to the host asynchronously; the kernels
        read the true wave counts on the device."""
        x = self._pos(x_bin, "binned_positions")
        bo = self._offsets(bin_offsets)
        dev = x_bin.device
        n = self._b * self._n
        st = _stream(x_bin)
        capturing = torch.cuda.is_current_stream_capturing()
        if not capturing:
            self._consume_readback()
        start = torch.empty(max(n, 1), dtype=_I32, device=dev)
        count = torch.empty(max(n, 1), dtype=_I32, device=dev)
        order = torch.empty(max(n, 1), dtype=_I32, device=dev)
        wcap = 2 * max(int(_lib.sphops_neighbor_wave_capacity(self._h)), 1)
        waves = torch.empty(wcap, dtype=_I32, device=dev)
        waves2 = torch.empty(wcap, dtype=_I32, device=dev)
        # device counts: [0:2] in-radius pairs (int64), [2:4] pairs of rows not
        # stored (int64), [4] waves, [5] split waves, [6] tile units, [7] waves
        # of the particles outside the tiles, [8] cell tiles
        small = torch.empty(9, dtype=_I32, device=dev)  # every word read is written by a kernel
        cap = self._capacity(n)
        index = torch.empty(max(cap, 1), dtype=_I32, device=dev)
        tiles = self._tile_buffers(dev, n, wcap) if self.tiles_enabled else None
        src = getattr(self, "_split_source", None)
        reuse = src is not None and src[0]() is bin_offsets and bin_offsets._version == src[1]
        _check(_lib.sphops_neighbor_candidates(self._h, x, bo, 1 if reuse else 0, st))
        cells = None
        if tiles is None and self._cells_wanted():
            ccap = max(int(_lib.sphops_neighbor_cell_capacity(self._h)), 1)
            cells = (torch.empty(max(n, 1), dtype=_I32, device=dev), torch.empty(2 * ccap, dtype=_I32, device=dev),
                     small[8:9])
            _check(_lib.sphops_neighbor_fill_tiled(
                self._h, x, bo, ctypes.c_void_p(start.data_ptr()), ctypes.c_void_p(index.data_ptr()), cap,
                ctypes.c_void_p(count.data_ptr()), ctypes.c_void_p(small.data_ptr()),
                ctypes.c_void_p(cells[0].data_ptr()), ctypes.c_void_p(cells[1].data_ptr()),
                ctypes.c_void_p(small.data_ptr() + 32), st))
        else:
            _check(_lib.sphops_neighbor_fill(self._h, x, bo, ctypes.c_void_p(start.data_ptr()),
                                             ctypes.c_void_p(index.data_ptr()), cap,
                                             ctypes.c_void_p(count.data_ptr()), ctypes.c_void_p(small.data_ptr()),
                                             st))
        _check(_lib.sphops_neighbor_schedule(self._h, ctypes.c_void_p(count.data_ptr()),
                                             ctypes.c_void_p(order.data_ptr()), ctypes.c_void_p(waves.data_ptr()),
                                             ctypes.c_void_p(small.data_ptr() + 16), ctypes.c_void_p(waves2.data_ptr()),
                                             ctypes.c_void_p(small.data_ptr() + 20), st))
        if tiles is not None:
            # after the fill: the tile build reuses the grid scratch that holds
            # the fill's work split
            _check(_lib.sphops_neighbor_tiles(
                self._h, x, bo, ctypes.c_void_p(count.data_ptr()), ctypes.c_void_p(tiles[0].data_ptr()),
                ctypes.c_void_p(small.data_ptr() + 24), ctypes.c_void_p(tiles[1].data_ptr()),
                ctypes.c_void_p(tiles[2].data_ptr()), ctypes.c_void_p(small.data_ptr() + 28), st))
        if not capturing:
            self._start_readback(small, cap, tiles is not None)
        e1, e2, e3 = self._wave_estimates(n)
        plan = NeighborPlan(start, count, index, order, waves, e1, waves2, e2, small)
        plan.capacity = cap
        if tiles is not None:
            plan.tiles = (tiles[0], small[6:7], tiles[1], tiles[2], e3, small[7:8])
        plan.cells = cells
        self._last_plan = plan
        return plan

    # Largest index buffer (entries) a snapshot allocates; rows that do not
    # fit are walked on the stencil instead.  At most 2^30 (the library's
    # limit).
    max_list_entries = 1 << 30
    # Index entries per particle for a grid's first snapshot, before any
    # total has been read back.
    first_capacity_per_particle = 40

    def _capacity(self, n):
        fixed = getattr(self, "_capture_capacity", 0)
        if fixed:
            return fixed
        est = getattr(self, "_index_capacity", 0)
        if not est:
            est = self.first_capacity_per_particle * max(n, 1)
        return int(min(est, self.max_list_entries))

    def _wave_estimates(self, n):
        bounds = getattr(self, "_wave_bounds", None)
        if getattr(self, "_capture_capacity", 0) and bounds:
            return bounds
        hint = getattr(self, "_wave_counts", None)
        if hint:
            return tuple(int(c) + c // 16 + 8 for c in hint)
        first = max(n // 8, 1)
        return (first, first, first)

    # Index-buffer margin over the last total, as a right shift of the total
    # (3: 1/8); lowered (a larger margin) when a list did not fit although
    # its buffer held the total, i.e. the fill's slices were uneven.
    _slack_shift = 3

    def _start_readback(self, small, cap, tiles):
        """Copy the device counts to pinned host memory without waiting
        (the tile counts are valid only for a plan with tiles)."""
        rb = getattr(self, "_rb", None)
        if rb is None:
            self._rb = rb = torch.empty(8, dtype=_I32, pin_memory=True)
        # a small kernel writes them into the pinned buffer (no copy-engine
        # transfer on the stream)
        _check(_lib.sphops_copy_words_to_host(ctypes.c_void_p(small.data_ptr()), ctypes.c_void_p(rb.data_ptr()), 8,
                                              _stream(small)))
        self._rb_cap = cap
        self._rb_tiles = tiles
        self._rb_event = torch.cuda.Event()
        self._rb_event.record()

    def _consume_readback(self, wait=False):
        """Take the counts of an earlier snapshot once they have arrived
        (waits only with ``wait``): they size the next index buffer and
        launches."""
        ev = getattr(self, "_rb_event", None)
        if ev is None:
            return
        if wait:
            ev.synchronize()
        elif not ev.query():
            return
        v = self._rb.tolist()
        total = (v[0] & 0xFFFFFFFF) | (v[1] << 32)
        unstored = (v[2] & 0xFFFFFFFF) | (v[3] << 32)
        self._index_capacity, self._slack_shift = next_index_capacity(total, unstored, self._rb_cap,
                                                                      self._slack_shift)
        first = max(self._b * self._n // 8, 1)
        self._wave_counts = (v[4], v[5], v[7] if self._rb_tiles else first)
        self._rb_event = None

    # Cell tiles for the pass-B backward (sphops_neighbor_tiles): opt-in
    # (NPA_SPHOPS_TILES=1, or this attribute), because at cfg5 the tiled
    # kernel is slower than the lane-split list kernel it replaces for
    # well-filled cells.
    tiles_enabled = os.environ.get("NPA_SPHOPS_TILES", "0") == "1"

    # Cell pairs of sphops_neighbor_fill_tiled: the pass-B backward evaluates
    # each pair inside a cell of 16 to 64 particles once for both ends (3D
    # clamped grids).  Opt-in (NPA_SPHOPS_CELLS=1, or this attribute): at cfg5
    # the list kernel spends little on those pairs, whose rows it finds in
    # L1, and the pass-B backward takes 0.96 ms with them against 0.85 ms
    # without.
    cells_enabled = os.environ.get("NPA_SPHOPS_CELLS", "0") == "1"

    def _cells_wanted(self):
        return self.cells_enabled and self._dim == 3 and self._boundary == CLAMPED

    def _tile_buffers(self, dev, n, wcap):
        cap = max(int(_lib.sphops_neighbor_tile_capacity(self._h)), 1)
        return (torch.empty(2 * cap, dtype=_I32, device=dev), torch.empty(max(n, 1), dtype=_I32, device=dev),
                torch.empty(wcap, dtype=_I32, device=dev))

    def set_capture_capacity(self, index_capacity, wave_margin=1.25):
        """Fix the sizes a list build uses, so that a whole step can be
        captured in a HIP graph (``torch.cuda.graph``) and replayed: every
        list gets an index buffer of ``index_capacity`` entries, and the pair
        kernels launch for ``wave_margin`` times the wave counts of the last
        eager build (the kernels read the true counts on the device and
        serve every wave whatever the launch).  Rows that do not fit are
        walked on the stencil (slower, same results); ``list_overflow`` tells
        whether that happened.  ``index_capacity = 0`` returns to the
        default sizing from the read-back totals."""
        self._consume_readback(wait=True)
        self._capture_capacity = max(int(index_capacity), 0)
        if self._capture_capacity > self.max_list_entries:
            raise RuntimeError(f"index_capacity above max_list_entries ({self.max_list_entries})")
        if self._capture_capacity:
            cap = max(int(_lib.sphops_neighbor_wave_capacity(self._h)), 0)
            hint = getattr(self, "_wave_counts", None)
            n = self._b * self._n
            self._wave_bounds = (tuple(min(cap, int(c * wave_margin) + 64) for c in hint) if hint
                                 else (max(n // 8, 1),) * 3)

    def list_overflow(self):
        """True if the last list built did not store every row (its index
        buffer was too small; those rows were walked on the stencil).  Reads
        the count back (synchronises)."""
        plan = getattr(self, "_last_plan", None)
        if plan is None:
            return False
        return int(plan[8][2:4].cpu().view(torch.int64).item()) > 0

    def reset_list_overflow(self):
        self._last_plan = None

    # Per operator: trailing dims of (first output, second output) after (B, N);
    # "C" stands for the channel count, "D" for the spatial dimension.
    _OUT_DIMS = {
        _native.OP_COUNT: ((), None), _native.OP_DENSITY: ((), None), _native.OP_DENSITY_GRADIENT: (("D",), None),
        _native.OP_MOMENT_MATRIX: (("D", "D"), None), _native.OP_BLUR: (("C",), None),
        _native.OP_GRADIENT: (("C", "D"), None), _native.OP_GRADIENT_HYBRID: (("C", "D"), None),
        _native.OP_DENSITY_PAIR: ((), ("D",)), _native.OP_BLUR_GRADIENT_HYBRID: (("C",), ("C", "D")),
    }

    def _numel(self, dims, C):
        n = self.batch_size * self.particle_count
        for d in dims:
            n *= C if d == "C" else self._dim
        return n

    def _args(self, op, x, bin_offsets, mass=None, rho=None, state=None, tol=1e-3, nbr=None, packed=None,
              packed_valid=False, **buffers):
        """Build ``sphops_args``; every buffer is checked for dtype, device,
        contiguity and element count against ``op``'s output shapes.
        ``packed`` ((B*N, 4) float32) receives the operator's (x, weight)
        records, or with ``packed_valid`` already holds them."""
        if op not in self._OUT_DIMS:
            raise RuntimeError(f"unknown operator {op}")
        a = _native.Args()
        a.x = self._pos(x, "binned_positions")
        a.bin_offsets = self._offsets(bin_offsets)
        if mass is not None:
            a.mass = self._bn(mass, "mass")
        if rho is not None:
            a.rho = self._bn(rho, "rho")
        C = 0
        if state is not None:
            C = state.shape[2] if state.dim() == 3 else -1
            a.state = self._state(state, "state_in", C)
        a.feature_dim = max(C, 0)
        a.tol = tol
        first, second = self._OUT_DIMS[op]
        BN = self.batch_size * self.particle_count
        sizes = {"upstream": self._numel(first, C), "out": self._numel(first, C),
                 "upstream2": self._numel(second, C) if second else None,
                 "out2": self._numel(second, C) if second else None,
                 "grad_x": BN * self._pw, "grad_state": BN * C, "grad_rho": BN}
        for name, t in buffers.items():
            if t is None:
                continue
            if t.dtype != _F32 or not t.is_contiguous() or t.device.type != "cuda":
                raise TypeError(f"{name}: expected a contiguous float32 GPU tensor")
            if sizes[name] is None or t.numel() != sizes[name]:
                raise RuntimeError(f"{name}: expected {sizes[name]} elements, got {t.numel()}")
            setattr(a, "out" if name == "grad_x" else name, t.data_ptr())
        if packed is not None:
            if (packed.dtype != _F32 or not packed.is_contiguous() or packed.device.type != "cuda"
                    or packed.data_ptr() % 16):
                raise TypeError("packed: expected a contiguous, 16-byte aligned float32 GPU tensor")
            if packed.numel() != 4 * BN:
                raise RuntimeError(f"packed: expected {4 * BN} elements, got {packed.numel()}")
            a.packed, a.packed_valid = packed.data_ptr(), int(bool(packed_valid))
        elif packed_valid:
            raise RuntimeError("packed_valid needs packed")
        if nbr is not None:
            a.nbr_start, a.nbr_count, a.nbr_index = nbr[0].data_ptr(), nbr[1].data_ptr(), nbr[2].data_ptr()
            if len(nbr) > 3:
                a.nbr_order, a.nbr_waves, a.nbr_wave_count = nbr[3].data_ptr(), nbr[4].data_ptr(), nbr[5]
            if len(nbr) > 6:
                a.nbr_waves_split, a.nbr_wave_count_split = nbr[6].data_ptr(), nbr[7]
            if len(nbr) > 8 and nbr[8] is not None:  # the wave counts on the device
                a.nbr_wave_count_device = nbr[8].data_ptr() + 16
                a.nbr_wave_count_split_device = nbr[8].data_ptr() + 20
            cells = getattr(nbr, "cells", None)
            if cells is not None:
                a.nbr_own, a.cells, a.cell_count = cells[0].data_ptr(), cells[1].data_ptr(), cells[2].data_ptr()
            tiles = getattr(nbr, "tiles", None)
            if tiles is not None:
                a.tile_units, a.tile_unit_count = tiles[0].data_ptr(), tiles[1].data_ptr()
                a.nbr_order_sparse, a.nbr_waves_sparse = tiles[2].data_ptr(), tiles[3].data_ptr()
                a.nbr_wave_count_sparse, a.nbr_wave_count_sparse_device = tiles[4], tiles[5].data_ptr()
        return a

    def op_forward(self, op, x, out, bin_offsets, mass=None, rho=None, state=None, tol=1e-3, nbr=None, out2=None,
                   packed=None):
        """Forward of operator ``op`` (``_native.OP_*``) into ``out`` (and
        ``out2`` for the fused codes), optionally over a neighbour list;
        ``packed``, if given, receives the (x, weight) records for the
        backward to reuse."""
        a = self._args(op, x, bin_offsets, mass, rho, state, tol=tol, nbr=nbr, packed=packed, out=out, out2=out2)
        _check(_lib.sphops_forward(self._h, op, ctypes.byref(a), _stream(x)))

    def op_backward(self, op, x, upstream, bin_offsets, mass, rho=None, state=None, grad_x=None, grad_state=None,
                    grad_rho=None, dLdx=True, dLds=True, dLdrho=True, nbr=None, upstream2=None, packed=None):
        """Backward of operator ``op``: gradients w.r.t. x, state and rho
        written into the given buffers according to the flags; ``packed``,
        if given, holds the records the forward wrote for the same x, mass
        and rho."""
        a = self._args(op, x, bin_offsets, mass, rho, state, nbr=nbr, packed=packed, packed_valid=packed is not None,
                       upstream=upstream, upstream2=upstream2, grad_x=grad_x, grad_state=grad_state,
                       grad_rho=grad_rho)
        _check(_lib.sphops_backward(self._h, op, int(bool(dLdx)), int(bool(dLds)), int(bool(dLdrho)),
                                    ctypes.byref(a), _stream(x)))


class _Grid3DProps:
    @property
    def grid_size_z(self):
        return self._sizes[2]


def _make(name, dim, boundary, mode):
    bases = (_Grid3DProps, _HashGridNative) if dim == 3 else (_HashGridNative,)
    return type(name, bases, {"_dim": dim, "_boundary": boundary, "_mode": mode, "__module__": __name__})


HashGrid2DPeriodic = _make("HashGrid2DPeriodic", 2, PERIODIC, MODE_GRID)
HashGrid2DBox = _make("HashGrid2DBox", 2, CLAMPED, MODE_GRID)
VHashGrid2DPeriodic = _make("VHashGrid2DPeriodic", 2, PERIODIC, MODE_PARTICLE)
VHashGrid2DBox = _make("VHashGrid2DBox", 2, CLAMPED, MODE_PARTICLE)
HashGrid3DPeriodic = _make("HashGrid3DPeriodic", 3, PERIODIC, MODE_GRID)
HashGrid3DBox = _make("HashGrid3DBox", 3, CLAMPED, MODE_GRID)
VHashGrid3DPeriodic = _make("VHashGrid3DPeriodic", 3, PERIODIC, MODE_PARTICLE)
VHashGrid3DBox = _make("VHashGrid3DBox", 3, CLAMPED, MODE_PARTICLE)


def safe_inv_sym_mat(in_matrix, out_matrix, tol=1e-3):
    """Module function ``safe_inv_sym_mat(in, out, tol)`` (``sph_cuda.cu:3181-3226``)."""
    if not isinstance(in_matrix, torch.Tensor) or in_matrix.dim() != 4:
        raise TypeError("in_matrix: expected a 4-d float32 tensor")
    B, N, D = in_matrix.shape[0], in_matrix.shape[1], in_matrix.shape[2]
    if D not in (2, 3):
        raise RuntimeError("safe_inverse only supports 2x2 or 3x3 matrices.")
    pi = _arr(in_matrix, "in_matrix", _F32, 4)
    po = _arr(out_matrix, "out_matrix", _F32, 4)
    _validate_shape(in_matrix, (B, N, D, D), "in_matrix")
    _validate_shape(out_matrix, (B, N, D, D), "out_matrix")
    _check(_lib.sphops_safe_inv_sym_mat(pi, po, B * N, D, ctypes.c_float(tol), _stream(in_matrix)))
