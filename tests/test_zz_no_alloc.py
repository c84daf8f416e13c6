"""kan_hip_infer_noalloc (the inference entry point that allocates nothing)
against kan_hip_infer, both through the C-ABI, on two calls in a row (the
second on a smaller batch, so the scratch holds the first call's larger
contents), fp32 and fp64: identical outputs where both plan the same split
count, within rounding (1e-6 fp32, 1e-14 fp64) where the fixed scratch
bounds the split slices; a call whose basis and output exceed the fixed
scratch is refused before any launch."""

import ctypes

import pytest
import torch

from tests._util import make_grid, normwise, np64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from torchsplinekan_amd import _C, _lib  # noqa: F401
    return _lib


def _packed_layer(I, O, G, k, dtype, seed):
    from torchsplinekan_amd import _C
    g = torch.Generator().manual_seed(seed)
    sw = (torch.randn(O, I, G + k, generator=g, dtype=torch.float64) * 0.1).to(dtype).cuda()
    bw = (torch.randn(O, I, generator=g, dtype=torch.float64) * 0.3).to(dtype).cuda()
    sc = (torch.rand(O, I, generator=g, dtype=torch.float64) + 0.5).to(dtype).cuda()
    grid = make_grid(I, G, k, "nonuniform", seed=seed, dtype=dtype).cuda()
    return grid, _C.pack_weight(bw, sw, sc, k, True)


def _infer(lib, x, grid, waug, O, G, k):
    """Output of the existing entry point, with a workspace from torch."""
    L = lib.LIB
    code = lib.dtype_code(x.dtype)
    n, I = x.shape
    nbytes = ctypes.c_size_t(0)
    lib.check(L.kan_hip_infer_workspace(code, n, I, O, G, k, 1, ctypes.byref(nbytes)))
    ws = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device="cuda")
    y = torch.empty(n, O, dtype=x.dtype, device="cuda")
    lib.check(L.kan_hip_infer(code, x.data_ptr(), grid.data_ptr(), waug.data_ptr(), y.data_ptr(),
                              ws.data_ptr(), nbytes.value, n, I, O, G, k, 1,
                              lib.stream_of(x.device)))
    return y, nbytes.value


def _infer_noalloc(lib, x, grid, waug, O, G, k):
    n, I = x.shape
    y = torch.full((n, O), float("nan"), dtype=x.dtype, device="cuda")
    lib.check(lib.LIB.kan_hip_infer_noalloc(lib.dtype_code(x.dtype), x.data_ptr(), grid.data_ptr(),
                                            waug.data_ptr(), y.data_ptr(), n, I, O, G, k, 1,
                                            lib.stream_of(x.device)))
    return y


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_noalloc_matches_infer_on_two_calls(lib, dtype):
    I, O, G, k = 1024, 1024, 10, 3
    grid, waug = _packed_layer(I, O, G, k, dtype, seed=3)
    g = torch.Generator().manual_seed(4)
    for n in (512 if dtype == torch.float32 else 256, 7):   # most of the scratch, then less
        print(f"noalloc vs infer {dtype} n={n}", flush=True)
        x = ((torch.rand(n, I, generator=g, dtype=torch.float64) * 2.2 - 1.1)
             .to(dtype).cuda())
        ref, need = _infer(lib, x, grid, waug, O, G, k)
        got = _infer_noalloc(lib, x, grid, waug, O, G, k)
        torch.cuda.synchronize()
        if need <= lib.KAN_NOALLOC_SCRATCH_BYTES:
            # the same plan (split count, tiles) as the workspace call
            assert torch.equal(got, ref)
        else:
            # the scratch bounds the split slices: another split count, the
            # same product summed in another order
            tol = 1e-6 if dtype == torch.float32 else 1e-14
            assert normwise(np64(got), np64(ref)) < tol


def test_noalloc_refuses_beyond_the_scratch(lib):
    I, O, G, k = 1024, 1024, 10, 3
    grid, waug = _packed_layer(I, O, G, k, torch.float32, seed=5)
    n = 2048   # 2048 x 14336 floats of basis alone: 117 MB > 64 MiB
    x = torch.zeros(n, I, device="cuda")
    y = torch.zeros(n, O, device="cuda")
    rc = lib.LIB.kan_hip_infer_noalloc(0, x.data_ptr(), grid.data_ptr(), waug.data_ptr(),
                                       y.data_ptr(), n, I, O, G, k, 1, lib.stream_of(x.device))
    assert rc == lib.KAN_ERR_WORKSPACE
    assert "fixed" in lib.last_error() and "kan_hip_infer" in lib.last_error()
    torch.cuda.synchronize()
    assert bool((y == 0).all())   # nothing was launched


def test_noalloc_python_wrapper(lib):
    from torchsplinekan_amd import _C
    I, O, G, k = 64, 48, 5, 3
    grid, waug = _packed_layer(I, O, G, k, torch.float32, seed=6)
    x = (torch.rand(33, I) * 2 - 1).cuda()
    assert torch.equal(_C.kan_infer_noalloc(x, grid, waug, k, True), _C.kan_infer(x, grid, waug, k, True))
