"""gfx950 sphops: spatial-hash binning and SPH neighbour perception.

Drop-in for the reference package ``sphops`` (``sphops/__init__.py:2-3``):
the same names are exported, backed by ``libsphops_hip.so``.
"""
from .sph import (HashGrid, HashGridSnapshot, bin_particles, unbin_particles, count, density, blur, gradient,
                  density_gradient, moment_matrix, gradient_hybrid, safe_inv_sym_mat)

__all__ = ["HashGrid", "HashGridSnapshot", "bin_particles", "unbin_particles", "count", "density", "blur",
           "gradient", "density_gradient", "moment_matrix", "gradient_hybrid", "safe_inv_sym_mat"]
