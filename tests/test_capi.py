"""CPU checks of the C-ABI library (no kernel launches): libkan_hip.so loads,
exports every entry point include/kan_hip.h declares, and its host-side
validation returns the documented status codes and messages before any
launch (csrc/kan_ops.h:27-78 of the reference for the limits and texts)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kan_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kan_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from torchsplinekan_amd import _lib
    return _lib


def test_library_exports_every_declared_symbol(lib):
    names = _declared()
    assert len(names) >= 15
    raw = ctypes.CDLL(lib.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), n
    # and the Python binding types every one of them
    assert set(names) <= set(lib.SIGNATURES)


def test_library_matches_its_sources(lib, tmp_path, monkeypatch):
    """The library carries the digest of the sources it was built from; the
    loader refuses one whose digest differs from the sources beside it."""
    from torchsplinekan_amd import build_lib
    built = lib.LIB.kan_hip_source_hash().decode()
    assert built == build_lib.source_hash()
    # a changed source changes the digest
    csrc = tmp_path / "csrc"
    csrc.mkdir()
    for f in os.listdir(build_lib.CSRC):
        if f.endswith((".hip", ".h")):
            (csrc / f).write_bytes(open(os.path.join(build_lib.CSRC, f), "rb").read())
    monkeypatch.setattr(build_lib, "CSRC", str(csrc))
    assert build_lib.source_hash() == built
    with open(csrc / "kan_capi.hip", "a") as f:
        f.write("\n// edited\n")
    assert build_lib.source_hash() != built
    with pytest.raises(ImportError, match="stale"):
        lib._load()


def test_limits(lib):
    assert lib.limits() == (71, 65535)


def test_routes_are_set_explicitly(lib, routes):
    """Routing switches: defaults from the environment at load, changed only
    through kan_hip_set_route; out-of-range values and unknown routes are
    rejected with KAN_ERR_INVALID and leave the switch unchanged."""
    env_default = {"fused_dx": 0, "compact_e": -1, "edge_fused": 1, "gemm_tile": -1}
    for name, want in env_default.items():
        var = "KAN_HIP_" + name.upper()
        if var not in os.environ:
            assert lib.get_route(name) == want, name
    for name, good, bad in [("fused_dx", 1, 2), ("compact_e", -1, -2), ("edge_fused", 0, 3),
                            ("gemm_tile", 3, 4)]:
        lib.set_route(name, good)
        assert lib.get_route(name) == good
        assert lib.LIB.kan_hip_set_route(lib.ROUTES[name], bad) == lib.KAN_ERR_INVALID
        assert "route" in lib.last_error()
        assert lib.get_route(name) == good
    assert lib.LIB.kan_hip_set_route(7, 0) == lib.KAN_ERR_INVALID
    assert lib.LIB.kan_hip_get_route(7) == -2
    # a changed environment is not read again
    os.environ["KAN_HIP_GEMM_TILE"] = "128"
    try:
        lib.set_route("gemm_tile", -1)
        assert lib.get_route("gemm_tile") == -1
    finally:
        del os.environ["KAN_HIP_GEMM_TILE"]
    from torchsplinekan_amd import _C
    assert _C.CUDA_MAX_DEG0_BASIS == 71 and _C.CUDA_MAX_IN_FEATURES == 65535
    assert _C.HAS_FUSED_KERNELS is True


def test_basis_impl_switch(lib):
    L = lib.LIB
    assert L.kan_hip_get_basis_impl() == 1
    assert L.kan_hip_set_basis_impl(7) == lib.KAN_ERR_INVALID
    assert "basis impl must be 0" in lib.last_error()
    assert L.kan_hip_set_basis_impl(0) == lib.KAN_OK
    assert L.kan_hip_get_basis_impl() == 0
    assert L.kan_hip_set_basis_impl(1) == lib.KAN_OK


def test_validation_before_launch(lib):
    L = lib.LIB
    # unsupported dtype code
    assert L.kan_hip_basis(7, None, None, None, 4, 4, 5, 3, None) == lib.KAN_ERR_INVALID
    assert "FP32 and FP64" in lib.last_error()
    # grid beyond the kernel limit: G + 2k = 72
    assert L.kan_hip_basis(0, None, None, None, 4, 4, 66, 3, None) == lib.KAN_ERR_LIMIT
    assert "G + 2k <= 71" in lib.last_error()
    # in_features beyond the limit
    assert L.kan_hip_forward(0, None, None, None, None, None, None, None, None, 0,
                             4, 65536, 4, 5, 3, None) == lib.KAN_ERR_LIMIT
    assert "in_features <= 65535" in lib.last_error()
    # spline order
    assert L.kan_hip_basis(0, None, None, None, 4, 4, 5, 4, None) == lib.KAN_ERR_INVALID
    # null pointers of non-empty buffers
    assert L.kan_hip_basis(0, None, None, None, 4, 4, 5, 3, None) == lib.KAN_ERR_INVALID
    assert "must not be NULL" in lib.last_error()
    # edge statistic: R beyond 72, and s without base_weight
    assert L.kan_hip_edge_abs_mean(0, None, 1, None, 1, 1, None, 0, 4, 4, 4, 73,
                                   None) == lib.KAN_ERR_LIMIT
    assert L.kan_hip_edge_abs_mean(0, 1, 1, None, 1, 1, None, 0, 4, 4, 4, 8,
                                   None) == lib.KAN_ERR_INVALID
    # a gradient that needs an absent operand
    assert L.kan_hip_backward(0, None, None, None, None, None, None, None, None, 1, None, None,
                              None, 0, 4, 4, 4, 5, 3, None) == lib.KAN_ERR_INVALID
    assert "without base_weight" in lib.last_error()
    # timing class
    assert L.kan_hip_timing_read(9, None, None, None) == lib.KAN_ERR_INVALID


def test_aug_width(lib):
    L = lib.LIB
    # [H | silu(x)] row padded to a multiple of 4 elements
    assert L.kan_hip_aug_width(1024, 10, 3, 1) == 1024 * 13 + 1024
    assert L.kan_hip_aug_width(16, 5, 3, 1) == 16 * 8 + 16
    assert L.kan_hip_aug_width(3, 4, 1, 0) == 16      # 15 -> 16
    assert L.kan_hip_aug_width(3, 0, 1, 0) == -1


def test_edge_linear_supported(lib):
    """The folded layer backward's range (host-side query, no device call):
    float32, 0 < out_features <= 512, num_basis + 1 <= 16, at least one
    sample."""
    L, f32, f64 = lib.LIB, lib.KAN_DTYPE_F32, lib.KAN_DTYPE_F64
    assert L.kan_hip_edge_linear_supported(f32, 16384, 512, 512, 11) == 1
    assert L.kan_hip_edge_linear_supported(f32, 1, 1, 4, 15) == 1
    assert L.kan_hip_edge_linear_supported(f32, 100, 8, 516, 11) == 0
    assert L.kan_hip_edge_linear_supported(f32, 100, 8, 70, 11) == 1
    assert L.kan_hip_edge_linear_supported(f32, 100, 8, 64, 16) == 0
    assert L.kan_hip_edge_linear_supported(f32, 0, 8, 64, 11) == 0
    assert L.kan_hip_edge_linear_supported(f64, 100, 8, 64, 11) == 0


def test_edge_linear_forward_queries_and_refusals(lib):
    """The one-pass forward's range, workspace size (partial sums of the
    statistic per 128 samples: 4 * ceil(n / 128) * I * O bytes) and the
    refusals that come before any launch (no device call)."""
    L, f32, f64 = lib.LIB, lib.KAN_DTYPE_F32, lib.KAN_DTYPE_F64
    assert L.kan_hip_edge_linear_forward_supported(f32, 16384, 512, 512, 11) == 1
    assert L.kan_hip_edge_linear_forward_supported(f32, 1, 1, 1300, 15) == 1
    assert L.kan_hip_edge_linear_forward_supported(f32, 100, 8, 64, 16) == 0
    assert L.kan_hip_edge_linear_forward_supported(f32, 0, 8, 64, 11) == 0
    assert L.kan_hip_edge_linear_forward_supported(f32, 100, 8, 0, 11) == 0
    assert L.kan_hip_edge_linear_forward_supported(f64, 100, 8, 64, 11) == 0
    nb = ctypes.c_size_t(0)
    assert L.kan_hip_edge_linear_forward_workspace(f32, 16384, 512, 512, 11,
                                                   ctypes.byref(nb)) == lib.KAN_OK
    assert nb.value == 4 * 128 * 512 * 512
    assert L.kan_hip_edge_linear_forward_workspace(f32, 129, 3, 200, 7,
                                                   ctypes.byref(nb)) == lib.KAN_OK
    assert nb.value == 4 * 2 * 3 * 200
    assert L.kan_hip_edge_linear_forward_workspace(f64, 129, 3, 200, 7,
                                                   ctypes.byref(nb)) == lib.KAN_ERR_LIMIT
    assert L.kan_hip_edge_linear_forward_workspace(f32, 129, 3, 200, 7, None) == \
        lib.KAN_ERR_INVALID
    # refusals before any launch (the pointers are never dereferenced)
    need = 4 * 2 * 3 * 200
    p = 4096
    fwd = L.kan_hip_edge_linear_forward
    assert fwd(f32, p, p, p, p, None, p, p, need, 129, 3, 200, 7, None) == lib.KAN_ERR_INVALID
    assert "must not be NULL" in lib.last_error()
    assert fwd(f32, p, p, None, p, p, p, p, need, 129, 3, 200, 7, None) == lib.KAN_ERR_INVALID
    assert "both be given" in lib.last_error()
    assert fwd(f32, p, p, p, p, p, p, p, need - 4, 129, 3, 200, 7, None) == lib.KAN_ERR_WORKSPACE
    assert fwd(f32, p, p, p, p, p, p, None, need, 129, 3, 200, 7, None) == lib.KAN_ERR_WORKSPACE
    assert fwd(f64, p, p, p, p, p, p, p, need, 129, 3, 200, 7, None) == lib.KAN_ERR_LIMIT
    assert fwd(f32, p, p, p, p, p, p, p, need, 129, 3, 200, 16, None) == lib.KAN_ERR_LIMIT
    assert "num_basis + 1 <= 16" in lib.last_error()


def test_c_header_compiles_as_c(tmp_path):
    """The header is plain C (no C++ or torch types in the signatures)."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / "t.c"
    src.write_text('#include "kan_hip.h"\nint main(void){return KAN_OK;}\n')
    r = subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER),
                        "-c", str(src), "-o", str(tmp_path / "t.o")], capture_output=True,
                       text=True)
    assert r.returncode == 0, r.stderr
