"""The C-ABI library loads and exports every symbol include/sphops_hip.h declares
(no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "sphops_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sphops_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_reference_surface():
    names = declared()
    for meth in ("initialize", "bin_particles", "backward_bin_particles", "count_forward", "density_forward",
                 "blur_forward", "gradient_forward", "density_gradient_forward", "moment_matrix_forward",
                 "density_backward", "blur_backward", "density_gradient_backward", "gradient_backward",
                 "moment_matrix_backward", "safe_inv_sym_mat"):
        assert f"sphops_{meth}" in names


def test_library_exports_every_declared_symbol():
    from npa_amd.sphops import _native
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared()) == set(_native.EXPORTED)


def test_abi_version_and_error_channel():
    from npa_amd.sphops import _native
    hdr = open(HEADER).read()
    version = int(re.search(r"#define SPHOPS_ABI_VERSION (\d+)", hdr).group(1))
    assert _native.lib.sphops_abi_version() == version == _native.ABI_VERSION
    # a failing call without touching the GPU: invalid dimension
    h = ctypes.c_void_p()
    gs = (ctypes.c_int32 * 2)(4, 4)
    st = _native.lib.sphops_grid_create(5, 0, 0, gs, ctypes.c_float(0.1), 10, 1, 64, ctypes.byref(h))
    assert st != 0
    assert b"dim must be 2 or 3" in _native.lib.sphops_last_error()
    st = _native.lib.sphops_grid_create(2, 1, 0, gs, ctypes.c_float(0.1), 10, 1, 64, ctypes.byref(h))
    gs2 = (ctypes.c_int32 * 2)(2, 4)
    st = _native.lib.sphops_grid_create(2, 1, 0, gs2, ctypes.c_float(0.1), 10, 1, 64, ctypes.byref(h))
    assert st != 0 and b"at least 3 cells" in _native.lib.sphops_last_error()
    gs3 = (ctypes.c_int32 * 2)(8, 16)
    st = _native.lib.sphops_grid_create(2, 0, 1, gs3, ctypes.c_float(0.1), 10, 1, 64, ctypes.byref(h))
    assert st != 0 and b"Morton" in _native.lib.sphops_last_error()
    st = _native.lib.sphops_safe_inv_sym_mat(None, None, 4, 4, ctypes.c_float(1e-3), None)
    assert st != 0 and b"2x2 or 3x3" in _native.lib.sphops_last_error()


def test_args_struct_matches_header():
    """The ctypes mirror of sphops_args lists the header's fields in order."""
    from npa_amd.sphops import _native
    hdr = open(HEADER).read()
    body = re.search(r"typedef struct sphops_args \{(.*?)\} sphops_args;", hdr, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = [re.sub(r"\[.*\]", "", decl.split()[-1].lstrip("*")) for decl in body.split(";") if decl.strip()]
    assert names == [f[0] for f in _native.Args._fields_]


def test_header_is_plain_c(tmp_path):
    """The ABI header compiles as strict C99 (no C++ in the boundary), so a
    cgo / FFI binding can include it as it is."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        import pytest
        pytest.skip("gcc not available")
    src = tmp_path / "abi.c"
    src.write_text('#include "sphops_hip.h"\nint main(void) { return sizeof(sphops_args) ? 0 : 1; }\n')
    r = subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.dirname(HEADER),
                        "-c", str(src), "-o", str(tmp_path / "abi.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
