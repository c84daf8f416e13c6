"""ctypes binding of libkan_hip.so (declarations in include/kan_hip.h).

torch is imported before the library is opened so that the HIP runtime torch
already loaded (same soname, libamdhip64.so.7) is the one the kernels use:
streams and device pointers handed over from torch are then valid in the
library.  Loading fails loudly (ImportError) when the library is missing, lacks
an entry point, or was built from other sources than those in csrc/ (the
library carries a digest of its sources and flags, see build_lib).
"""

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL open, see module docstring)

from . import build_lib as _build_lib

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libkan_hip.so")

KAN_DTYPE_F32 = 0
KAN_DTYPE_F64 = 1
KAN_OK = 0
KAN_ERR_INVALID = 1
KAN_ERR_LIMIT = 2
KAN_ERR_HIP = 3
KAN_ERR_WORKSPACE = 4
KAN_NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024  # fixed scratch of kan_hip_infer_noalloc

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "kan_hip_last_error": (ctypes.c_char_p, []),
    "kan_hip_source_hash": (ctypes.c_char_p, []),
    "kan_hip_limits": (_int, [ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "kan_hip_set_basis_impl": (_int, [_i64]),
    "kan_hip_get_basis_impl": (_i64, []),
    "kan_hip_set_route": (_int, [_int, _int]),
    "kan_hip_get_route": (_int, [_int]),
    "kan_hip_basis": (_int, [_int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_basis_grad": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_basis_silu": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_basis_silu_grad": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                       _vp]),
    "kan_hip_edge_abs_mean_double_backward_workspace": (_int, [_int, _i64, _i64, _i64, _i64,
                                                                ctypes.POINTER(_sz)]),
    "kan_hip_edge_abs_mean_double_backward": (_int, [_int] + [_vp] * 15 + [_sz, _i64, _i64, _i64,
                                                                           _i64, _vp]),
    "kan_hip_pack_weight": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_infer_workspace": (_int, [_int, _i64, _i64, _i64, _i64, _i64, _int,
                                       ctypes.POINTER(_sz)]),
    "kan_hip_infer": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i64, _i64, _i64, _i64,
                             _int, _vp]),
    "kan_hip_infer_noalloc": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                     _int, _vp]),
    "kan_hip_matmul_workspace": (_int, [_int, _int, _int, _i64, _i64, _i64, ctypes.POINTER(_sz)]),
    "kan_hip_matmul": (_int, [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64,
                              _vp, _sz, _vp]),
    "kan_hip_basis_deriv": (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                   _vp]),
    "kan_hip_basis_deriv_contract": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                            _i64, _i64, _i64, _vp]),
    "kan_hip_silu_deriv": (_int, [_int, _vp, _vp, _vp, _i64, _i64, _vp]),
    "kan_hip_aug_width": (_i64, [_i64, _i64, _i64, _int]),
    "kan_hip_forward_workspace": (_int, [_int, _i64, _i64, _i64, _i64, _i64, _int,
                                         ctypes.POINTER(_sz)]),
    "kan_hip_forward": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                               _i64, _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_pack_basis": (_int, [_int, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp]),
    "kan_hip_backward_workspace": (_int, [_int, _i64, _i64, _i64, _i64, _i64, _int, _int, _int,
                                          ctypes.POINTER(_sz)]),
    "kan_hip_backward": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _vp, _sz, _i64, _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_edge_workspace": (_int, [_int, _i64, _i64, _i64, _i64, _int, ctypes.POINTER(_sz)]),
    "kan_hip_edge_abs_mean": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                     _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_edge_abs_mean_backward": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                              _vp, _sz, _i64, _i64, _i64, _i64, _vp]),
    "kan_hip_edge_linear_supported": (_int, [_int, _i64, _i64, _i64, _i64]),
    "kan_hip_edge_linear_backward": (_int, [_int] + [_vp] * 11 + [_sz, _i64, _i64, _i64, _i64,
                                                                _vp]),
    "kan_hip_edge_linear_forward_supported": (_int, [_int, _i64, _i64, _i64, _i64]),
    "kan_hip_edge_linear_forward_workspace": (_int, [_int, _i64, _i64, _i64, _i64,
                                                     ctypes.POINTER(_sz)]),
    "kan_hip_edge_linear_forward": (_int, [_int] + [_vp] * 7 + [_sz, _i64, _i64, _i64, _i64,
                                                               _vp]),
    "kan_hip_refit_gram": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                  _vp]),
    "kan_hip_stream_probe": (_int, [_int, _vp, _vp, _i64, _vp]),
    "kan_hip_edge_reg_workspace": (_int, [_int, _i64, ctypes.POINTER(_sz)]),
    "kan_hip_edge_reg": (_int, [_int, _vp, _i64, ctypes.c_double, ctypes.c_double, _vp, _vp, _sz,
                                _vp]),
    "kan_hip_edge_reg_backward": (_int, [_int, _vp, _vp, _i64, ctypes.c_double, ctypes.c_double,
                                         _vp, _sz, _vp, _vp]),
    "kan_hip_timing_enable": (_int, [_int]),
    "kan_hip_timing_read": (_int, [_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64),
                                   ctypes.POINTER(ctypes.c_double)]),
}


class KanHipError(RuntimeError):
    """A non-zero status from libkan_hip.so (message from kan_hip_last_error)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m torchsplinekan_amd.build_lib` "
            "(or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError as exc:
            raise ImportError(f"{LIB_PATH} does not export {name}: rebuild it") from exc
        fn.restype = res
        fn.argtypes = args
    if os.path.isdir(_build_lib.CSRC):
        built = lib.kan_hip_source_hash().decode()
        if built != _build_lib.source_hash():
            raise ImportError(
                f"{LIB_PATH} is stale: it was built from other sources than those in "
                f"{_build_lib.CSRC}; rebuild it with `python -m torchsplinekan_amd.build_lib`")
    return lib


LIB = _load()


def last_error() -> str:
    msg = LIB.kan_hip_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(status: int) -> None:
    if status != KAN_OK:
        raise KanHipError(status, last_error())


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return KAN_DTYPE_F32
    if dtype == torch.float64:
        return KAN_DTYPE_F64
    raise RuntimeError(f"only FP32 and FP64 inputs are supported, got {dtype}")


def ptr(t):
    """Device pointer of a tensor, or None for an absent optional."""
    if t is None:
        return None
    return t.data_ptr() if t.numel() > 0 else None


def stream_of(device: torch.device) -> int:
    """hipStream_t handle of the current torch stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


# routing switches of kan_hip_set_route (KAN_ROUTE_* in include/kan_hip.h) and
# the values each takes
ROUTES = {"fused_dx": 0, "compact_e": 1, "edge_fused": 2, "gemm_tile": 3}
GEMM_TILES = {"auto": -1, "256": 0, "128": 1, "256x64": 2, "256w4": 3}


def set_route(name: str, value: int) -> None:
    """Sets one routing switch for the whole process (a choice between
    kernel routes with the same results; see include/kan_hip.h)."""
    check(LIB.kan_hip_set_route(ROUTES[name], int(value)))


def get_route(name: str) -> int:
    return int(LIB.kan_hip_get_route(ROUTES[name]))


class route:
    """Context manager: `with route("gemm_tile", 1): ...` sets a switch and
    restores its previous value on exit."""

    def __init__(self, name: str, value: int):
        self.name, self.value = name, int(value)

    def __enter__(self):
        self.saved = get_route(self.name)
        set_route(self.name, self.value)
        return self

    def __exit__(self, *exc):
        set_route(self.name, self.saved)
        return False


def limits():
    a, b = _i64(), _i64()
    check(LIB.kan_hip_limits(ctypes.byref(a), ctypes.byref(b)))
    return int(a.value), int(b.value)


# kernel classes of kan_hip_timing_read
TIMING_CLASSES = {"contraction": 0, "basis": 1, "basis_grad": 2, "edge": 3, "edge_grad": 4,
                  "other": 5, "stream": 6}


def timing_enable(on: bool) -> None:
    """Starts (clearing earlier records) or stops HIP-event timing of launches."""
    check(LIB.kan_hip_timing_enable(int(bool(on))))


def timing_read(kernel_class: str):
    """(total_ms, launches, total_work) recorded for one kernel class."""
    ms, n, w = ctypes.c_double(), _i64(), ctypes.c_double()
    check(LIB.kan_hip_timing_read(TIMING_CLASSES[kernel_class], ctypes.byref(ms), ctypes.byref(n),
                                  ctypes.byref(w)))
    return float(ms.value), int(n.value), float(w.value)
