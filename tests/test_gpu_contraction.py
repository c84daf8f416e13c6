"""GPU parity of the fp32 contraction engine in its tile configurations
(256x256 over 8 waves of 128x64, 256x256 over 4 waves of 128x128, and
128x128 with 64x64 per wave), each forced through the gemm_tile route, on
layer shapes chosen so that the
forward (NT), input-gradient (NT against the transposed weight; the
two-pass routes through the full E (compact_e route 0) and through its
compact form (the k+1 span-window values per item; compact_e route 1
forces it, by default it serves rows of R >= 25), and, with
fused_dx route 1, dx contracted in the GEMM epilogue, where the spline
columns of one feature straddle two wave blocks when R does not divide the
block width) and parameter-gradient (TN, split
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


@pytest.mark.parametrize("dx_route", ["full", "compact", "fused"])
@pytest.mark.parametrize("tile", ["256", "256w4", "128"])
@pytest.mark.parametrize("shape", SHAPES)
def test_contraction_configs_match_oracle(C, routes, tile, shape, dx_route):
    N, I, O, G, k, kind = shape
    print(f"contraction tile={tile} dx_route={dx_route} shape={shape}", flush=True)
    routes.set_route("gemm_tile", routes.GEMM_TILES[tile])
    routes.set_route("fused_dx", 1 if dx_route == "fused" else 0)
    routes.set_route("compact_e", 1 if dx_route == "compact" else 0)
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
def test_fused_dx_without_base_branch(C, routes, shape):
    """The fused input gradient with two partial slots per feature (no base
    columns), spline features straddling wave blocks (R = 10 and R = 5)."""
    N, I, O, G, k, kind = shape
    print(f"fused dx, no base branch, shape={shape}", flush=True)
    routes.set_route("fused_dx", 1)
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


@pytest.mark.parametrize("tile", ["256", "128"])
@pytest.mark.parametrize("shape", [
    (600, 37, 300, 7, 3, "uniform", True),
    (300, 33, 19, 7, 2, "nonuniform", True),
    (257, 33, 19, 4, 1, "repeated", False),
    (520, 9, 70, 65, 3, "uniform", True),     # R = 68: rows across 3 wave blocks
    (1000, 130, 64, 10, 3, "nonuniform", False),
])
def test_compact_input_product_matches_full_route(C, routes, tile, shape):
    """dx through the compact input-side product (the k+1 span-window values
    of E per item and the base columns, then the input gradient from them)
    equals dx through the full E [n, ld] element for element (the same
    products in the same order), and both hold the fp32 bar against the
    oracle; x up to 1.1 outside [-1, 1] takes the zero-basis path, and a
    window that crosses wave blocks is completed by each of them."""
    N, I, O, G, k, kind, base = shape
    print(f"compact E tile={tile} shape={shape}", flush=True)
    routes.set_route("gemm_tile", routes.GEMM_TILES[tile])
    routes.set_route("fused_dx", 0)
    g = torch.Generator().manual_seed(3 * N + I)
    grid = make_grid(I, G, k, kind, seed=I)
    x = torch.rand(N, I, generator=g, dtype=torch.float64) * 2.2 - 1.1
    sw = torch.randn(O, I, G + k, generator=g, dtype=torch.float64) * 0.1
    bw = (torch.rand(O, I, generator=g, dtype=torch.float64) * 2 - 1) / np.sqrt(I)
    sc = torch.rand(O, I, generator=g, dtype=torch.float64) + 0.5
    D = torch.randn(N, O, generator=g, dtype=torch.float64)
    f = lambda t: t.float().cuda()
    bwd = f(bw) if base else torch.empty(0, device="cuda")
    y, H = C.kan_forward(f(x), f(grid), bwd, f(sw), f(sc), k, True)
    out = {}
    for route in ("0", "1"):
        routes.set_route("compact_e", int(route))
        out[route] = C.kan_backward(f(D), f(x), f(grid), bwd, f(sw), f(sc), H, k, True)
    torch.cuda.synchronize()
    gx_full, gx_comp = out["0"][0], out["1"][0]
    assert torch.equal(gx_comp, gx_full)
    for a_, b_ in zip(out["0"][1:], out["1"][1:]):
        assert (a_ is None and b_ is None) or torch.equal(a_, b_)
    a = lambda t: np64(t.float())
    _, rH = ko.kan_forward(a(x), a(grid), a(bw) if base else None, a(sw), a(sc), k)
    rgx = ko.kan_backward(a(D), a(x), a(grid), a(bw) if base else None, a(sw), a(sc), k,
                          basis=rH)[0]
    assert normwise(np64(gx_comp), rgx) < FP32_TOL
