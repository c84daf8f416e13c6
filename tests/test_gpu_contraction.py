"""GPU parity of the fp32 contraction engine in its tile configurations
(256x256 over 8 waves of 128x64, 256x256 over 4 waves of 128x128, and
128x128 with 64x64 per wave), each forced through KAN_HIP_GEMM_TILE, on
layer shapes chosen so that the
forward (NT), input-gradient (NT against the transposed weight; both the
two-pass route and, with KAN_HIP_FUSED_DX=1, dx contracted in the GEMM
epilogue, where the spline columns of one feature straddle two wave blocks
when R does not divide the block width) and parameter-gradient (TN, split
over samples) products see whole tiles, ragged row and column edges, K tails that
are not a multiple of the 32-deep slab, unaligned leading dimensions
(out_features not a multiple of 4) and several split-K counts.

Checked against the fp64 oracle (oracle/kan_oracle.py, kan_forward and
kan_backward, which follow csrc/kan_cpu.cpp:11-290) at the fp32 bar:
normwise relative error max|u - v| / max|v| <= 1e-5 per tensor.
"""

import os

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests._util import make_grid, normwise, np64

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5

# N, I, O, G, k, kind: what each shape exercises in the three products
SHAPES = [
    (512, 32, 256, 5, 3, "uniform"),       # whole 256-tiles in the forward; K = 288 = 9 slabs
    (600, 37, 300, 7, 3, "uniform"),       # ragged rows/cols everywhere; K tails 407 and 300
    (300, 33, 19, 7, 2, "nonuniform"),     # out_features 19: unaligned D rows, guarded TN/NN
    (4096, 20, 64, 5, 1, "uniform"),       # long sample axis: parameter product split up to 16
    (520, 64, 520, 3, 2, "repeated"),      # both tile dims just past a multiple of 256
]


@pytest.fixture(scope="module")
def C():
    from torchsplinekan_amd import _C
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return _C


@pytest.fixture
def tile_env():
    names = ("KAN_HIP_GEMM_TILE", "KAN_HIP_FUSED_DX")
    old = {n: os.environ.get(n) for n in names}
    yield
    for n, v in old.items():
        if v is None:
            os.environ.pop(n, None)
        else:
            os.environ[n] = v


@pytest.mark.parametrize("fused_dx", ["0", "1"])
@pytest.mark.parametrize("tile", ["256", "256w4", "128"])
@pytest.mark.parametrize("shape", SHAPES)
def test_contraction_configs_match_oracle(C, tile_env, tile, shape, fused_dx):
    N, I, O, G, k, kind = shape
    print(f"contraction tile={tile} fused_dx={fused_dx} shape={shape}", flush=True)
    os.environ["KAN_HIP_GEMM_TILE"] = tile
    os.environ["KAN_HIP_FUSED_DX"] = fused_dx
    g = torch.Generator().manual_seed(N + I)
    grid = make_grid(I, G, k, kind, seed=N)
    x = torch.rand(N, I, generator=g, dtype=torch.float64) * 2.2 - 1.1
    sw = torch.randn(O, I, G + k, generator=g, dtype=torch.float64) * 0.1
    bw = (torch.rand(O, I, generator=g, dtype=torch.float64) * 2 - 1) / np.sqrt(I)
    sc = torch.rand(O, I, generator=g, dtype=torch.float64) + 0.5
    D = torch.randn(N, O, generator=g, dtype=torch.float64)
    f = lambda t: t.float().cuda()
    y, H = C.kan_forward(f(x), f(grid), f(bw), f(sw), f(sc), k, True)
    gx, gbw, gsw, gsc = C.kan_backward(f(D), f(x), f(grid), f(bw), f(sw), f(sc), H, k, True)
    torch.cuda.synchronize()
    # the oracle sees exactly the fp32 operands the device saw
    a = lambda t: np64(t.float())
    ry, rH = ko.kan_forward(a(x), a(grid), a(bw), a(sw), a(sc), k)
    rgx, rgbw, rgsw, rgsc = ko.kan_backward(a(D), a(x), a(grid), a(bw), a(sw), a(sc), k,
                                            basis=rH)
    for name, got, ref in [("y", y, ry), ("dx", gx, rgx), ("dbase_w", gbw, rgbw),
                           ("dcoef", gsw, rgsw), ("dscaler", gsc, rgsc)]:
        err = normwise(np64(got), ref)
        assert err < FP32_TOL, (name, err)


@pytest.mark.parametrize("shape", [(300, 37, 96, 7, 3, "uniform"), (257, 33, 19, 4, 1, "repeated")])
def test_fused_dx_without_base_branch(C, tile_env, shape):
    """The fused input gradient with two partial slots per feature (no base
    columns), spline features straddling wave blocks (R = 10 and R = 5)."""
    N, I, O, G, k, kind = shape
    print(f"fused dx, no base branch, shape={shape}", flush=True)
    os.environ["KAN_HIP_FUSED_DX"] = "1"
    g = torch.Generator().manual_seed(N)
    grid = make_grid(I, G, k, kind, seed=N)
    x = torch.rand(N, I, generator=g, dtype=torch.float64) * 2.2 - 1.1
    sw = torch.randn(O, I, G + k, generator=g, dtype=torch.float64) * 0.1
    D = torch.randn(N, O, generator=g, dtype=torch.float64)
    f = lambda t: t.float().cuda()
    empty = torch.empty(0, device="cuda")
    y, H = C.kan_forward(f(x), f(grid), empty, f(sw), empty, k, False)
    gx, gbw, gsw, gsc = C.kan_backward(f(D), f(x), f(grid), empty, f(sw), empty, H, k, False)
    torch.cuda.synchronize()
    a = lambda t: np64(t.float())
    ry, rH = ko.kan_forward(a(x), a(grid), None, a(sw), None, k)
    rgx, _, rgsw, _ = ko.kan_backward(a(D), a(x), a(grid), None, a(sw), None, k, basis=rH)
    assert gbw is None and gsc is None
    for name, got, ref in [("y", y, ry), ("dx", gx, rgx), ("dcoef", gsw, rgsw)]:
        err = normwise(np64(got), ref)
        assert err < FP32_TOL, (name, err)
