"""ctypes binding of libsphops_hip.so (the C ABI in include/sphops_hip.h).

The library is built in-tree (``npa_amd/_lib``) by ``__graft_entry__.build()``
or ``make -C npa_amd/csrc``.  There is no fallback: if the library is missing
or cannot be loaded, importing this module raises ImportError.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get(
    "SPHOPS_HIP_LIB", os.path.join(os.path.dirname(_HERE), "_lib", "libsphops_hip.so"))
ABI_VERSION = 21

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"libsphops_hip.so not found at {LIB_PATH}; build it with "
        "`python -c 'import __graft_entry__ as g; g.build()'` or `make -C npa_amd/csrc`")

lib = ctypes.CDLL(LIB_PATH)

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_u32 = ctypes.c_uint32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double

_SIGNATURES = {
    "sphops_abi_version": ([], _i32),
    "sphops_last_error": ([], ctypes.c_char_p),
    "sphops_grid_create": ([_i32, _i32, _i32, ctypes.POINTER(ctypes.c_int32), _f32, _u32, _u32, _u32,
                            ctypes.POINTER(_p)], _i32),
    "sphops_grid_destroy": ([_p], None),
    "sphops_grid_max_blocks": ([_p], _i64),
    "sphops_grid_coefficients": ([_p, ctypes.POINTER(_f32), ctypes.POINTER(_f32)], _i32),
    "sphops_initialize": ([_p, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_initialize_inverse": ([_p, _p, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_initialize_noalloc": ([_i32, _i32, _i32, ctypes.POINTER(ctypes.c_int32), _f32, _u32, _u32, _u32,
                                   _p, _p, _p, _p, _p, _p], _i32),
    "sphops_bin_particles": ([_p, _p, _p, _p, _p, _p, _p, _p, _u32, _p], _i32),
    "sphops_backward_bin_particles": ([_p, _p, _p, _p, _p, _p, _p, _p, _u32, _p], _i32),
    "sphops_count_forward": ([_p, _p, _p, _p, _p, _p], _i32),
    "sphops_density_forward": ([_p, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_blur_forward": ([_p, _p, _p, _p, _p, _p, _u32, _p, _p, _p], _i32),
    "sphops_gradient_forward": ([_p, _p, _p, _p, _p, _p, _u32, _p, _p, _p], _i32),
    "sphops_density_gradient_forward": ([_p, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_moment_matrix_forward": ([_p, _p, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_gradient_hybrid_forward": ([_p, _p, _p, _p, _p, _p, _u32, _f32, _p, _p, _p], _i32),
    "sphops_density_backward": ([_p, _p, _p, _p, _p, _p, _p, _i32, _p], _i32),
    "sphops_blur_backward": ([_p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _p, _p, _i32, _i32, _i32, _p], _i32),
    "sphops_density_gradient_backward": ([_p, _p, _p, _p, _p, _p, _p, _i32, _p], _i32),
    "sphops_gradient_backward": ([_p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _p, _p, _i32, _i32, _i32, _p],
                                 _i32),
    "sphops_moment_matrix_backward": ([_p, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _p], _i32),
    "sphops_safe_inv_sym_mat": ([_p, _p, _i64, _i32, _f32, _p], _i32),
    "sphops_perception_features_forward": ([_i32, _p, _p, _p, _p, _p, _i64, _u32, _f32, _f32, _f32, _i32, _p],
                                           _i32),
    "sphops_perception_features_backward": ([_i32, _p, _p, _p, _p, _p, _p, _p, _i64, _u32, _f32, _f32, _f32, _i32,
                                             _p], _i32),
    "sphops_euler_update_forward": ([_i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _u32, _f32, _f32, _f32,
                                     _f32, _f32, _p], _i32),
    "sphops_euler_update_backward": ([_i32, _i32, _p, _p, _p, _p, _p, _p, _i64, _u32, _f32, _f32, _f32, _p], _i32),
    "sphops_splat_forward": ([_p, _p, _p, _i64, _i64, _i32, _i32, _f64, _f64, _f64, _i32, _i32, _f64, _p, _p, _p],
                             _i32),
    "sphops_splat_workspace_bytes": ([_i64], _i64),
    "sphops_splat_backward": ([_p, _p, _p, _i64, _i64, _i32, _i32, _f64, _f64, _f64, _i32, _i32, _f64, _p, _p, _p,
                               _p], _i32),
    "sphops_linear_weight_grad": ([_p, _p, _p, _p, _i64, _i32, _i32, _p, _p], _i32),
    "sphops_linear_weight_grad_workspace_bytes": ([_i64, _i32, _i32], _i64),
    "sphops_relu_linear_input_grad": ([_p, _p, _p, _p, _i64, _i32, _i32, _p], _i32),
    "sphops_relu_linear_forward": ([_p, _p, _p, _p, _i64, _i32, _i32, _p], _i32),
    "sphops_relu_linear_weight_grad": ([_p, _p, _p, _p, _i64, _i32, _i32, _p, _p], _i32),
    "sphops_forward": ([_p, _i32, _p, _p], _i32),
    "sphops_backward": ([_p, _i32, _i32, _i32, _i32, _p, _p], _i32),
    "sphops_neighbor_candidates": ([_p, _p, _p, _i32, _p], _i32),
    "sphops_copy_words_to_host": ([_p, _p, _u32, _p], _i32),
    "sphops_neighbor_fill": ([_p, _p, _p, _p, _p, _i64, _p, _p, _p], _i32),
    "sphops_neighbor_fill_tiled": ([_p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_neighbor_cell_capacity": ([_p], _i64),
    "sphops_neighbor_schedule": ([_p, _p, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_neighbor_tiles": ([_p, _p, _p, _p, _p, _p, _p, _p, _p, _p], _i32),
    "sphops_neighbor_tile_capacity": ([_p], _i64),
    "sphops_neighbor_wave_capacity": ([_p], _i64),
}


class Args(ctypes.Structure):
    """``sphops_args`` (include/sphops_hip.h)."""
    _fields_ = [("x", _p), ("mass", _p), ("rho", _p), ("state", _p), ("upstream", _p), ("out", _p),
                ("grad_state", _p), ("grad_rho", _p), ("feature_dim", _u32), ("tol", _f32),
                ("bin_offsets", _p), ("nbr_start", _p), ("nbr_count", _p), ("nbr_index", _p), ("nbr_order", _p),
                ("nbr_waves", _p), ("nbr_wave_count", ctypes.c_int32), ("nbr_waves_split", _p),
                ("nbr_wave_count_split", ctypes.c_int32), ("upstream2", _p), ("out2", _p),
                ("nbr_wave_count_device", _p), ("nbr_wave_count_split_device", _p),
                ("tile_units", _p), ("tile_unit_count", _p), ("nbr_order_sparse", _p), ("nbr_waves_sparse", _p),
                ("nbr_wave_count_sparse", ctypes.c_int32), ("nbr_wave_count_sparse_device", _p),
                ("packed", _p), ("packed_valid", ctypes.c_int32), ("nbr_own", _p), ("cells", _p),
                ("cell_count", _p)]


(OP_COUNT, OP_DENSITY, OP_DENSITY_GRADIENT, OP_MOMENT_MATRIX, OP_BLUR, OP_GRADIENT, OP_GRADIENT_HYBRID,
 OP_DENSITY_PAIR, OP_BLUR_GRADIENT_HYBRID) = range(9)

for _name, (_args, _res) in _SIGNATURES.items():
    _fn = getattr(lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res

if lib.sphops_abi_version() != ABI_VERSION:
    raise ImportError(f"{LIB_PATH}: ABI version {lib.sphops_abi_version()} != expected {ABI_VERSION}")

EXPORTED = tuple(_SIGNATURES)


def check(status):
    """Raise RuntimeError with the library's message on a nonzero status."""
    if status != 0:
        raise RuntimeError(lib.sphops_last_error().decode("utf-8", "replace"))
