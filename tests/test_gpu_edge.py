"""GPU parity of the fused edge statistic a[o,i] = mean_n |phi[n,o,i]| and its
backward against the CPU oracle, and of forward_with_regularization with
reg_impl="fused" against the dense path (mirrors
tests/test_fused_regularization.py:58-107 of the reference).
"""

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests._util import normwise, np64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from torchsplinekan_amd import _C
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return _C


def _edge_inputs(N, I, O, R, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(N, I, generator=g, dtype=torch.float64)
    H = torch.rand(N, I, R, generator=g, dtype=torch.float64)
    bw = torch.randn(O, I, generator=g, dtype=torch.float64) * 0.3
    W = torch.randn(O, I, R, generator=g, dtype=torch.float64) * 0.2
    ga = torch.randn(O, I, generator=g, dtype=torch.float64)
    return [t.to(dtype) for t in (s, H, bw, W, ga)]


# (N, I, O, R): every k-step class of the fp32 MFMA kernels (R+1 = 2, 5, 9, 12, 14, 21,
# 30, 45, 69), outputs beyond one 512-wide block and beyond one staged 1024-row
# chunk, ragged sample counts and a sample count that is split across blocks.
# Output widths cover every (tiles per wave, sample-sharing waves) tiling of the
# forward and parameter kernels (O = 3..33 -> 2x4, 64/70 -> 4x4, 200 -> 4x2,
# 300 -> 4x1, >= 512 -> 8x1); (8192, 260, 20, 7) runs the input kernel with
# several sample blocks per workgroup on weights staged once.  The fused
# backward's tilings (one chunk covering O): O <= 32 -> 2x4, 33..64 -> 4x4,
# 65..128 -> 4x2 (100; output partials of 2 waves added per group of 2 tiles),
# 129..256 -> 4x1 (200), 257..512 -> 8x1 (300, 512).
SHAPES = [(37, 5, 3, 4), (300, 16, 40, 8), (1000, 9, 70, 13), (64, 3, 300, 68),
          (5000, 4, 6, 11), (77, 3, 5, 1), (513, 2, 33, 20), (129, 3, 17, 29), (70, 2, 9, 44),
          (200, 2, 1300, 11), (3000, 3, 600, 7), (2000, 3, 200, 11), (4097, 5, 64, 11),
          (8192, 260, 20, 7), (2100, 3, 512, 11), (700, 2, 300, 8), (1200, 3, 100, 3)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("base", [True, False])
@pytest.mark.parametrize("route", ["auto", "separate"])
def test_edge_abs_mean_and_backward_match_oracle(C, monkeypatch, shape, dtype, base, route):
    """route "auto": fp32 layers with O <= 512 and R + 1 <= 16 take the fused
    backward kernel (both gradient sides from one phi); "separate" forces the
    parameter and input kernels (KAN_HIP_EDGE_FUSED=0)."""
    N, I, O, R = shape
    if route == "separate" and dtype == torch.float64:
        pytest.skip("the route applies to the fp32 MFMA kernels only")
    monkeypatch.setenv("KAN_HIP_EDGE_FUSED", "0" if route == "separate" else "1")
    print(f"edge {shape} {dtype} base={base} route={route}", flush=True)
    s, H, bw, W, ga = _edge_inputs(N, I, O, R, dtype, seed=N + O)
    empty = torch.empty(0, dtype=dtype, device="cuda")
    sd = s.cuda() if base else empty
    bwd = bw.cuda() if base else empty
    a = C.edge_abs_mean(sd, H.cuda(), bwd, W.cuda())
    ra = ko.edge_abs_mean(np64(s) if base else None, np64(H), np64(bw) if base else None,
                          np64(W))
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    assert normwise(np64(a), ra) < tol
    ds, dH, dbw, dW = C.edge_abs_mean_backward(ga.cuda(), sd, H.cuda(), bwd, W.cuda(),
                                               True, True, True, True)
    rds, rdH, rdbw, rdW = ko.edge_abs_mean_backward(np64(ga), np64(s) if base else None,
                                                    np64(H), np64(bw) if base else None,
                                                    np64(W))
    # fp32: sign(phi) may flip where |phi| is at rounding level; the normwise
    # bound allows for a handful of such terms.
    gtol = 1e-12 if dtype == torch.float64 else 1e-4
    assert normwise(np64(dH), rdH) < gtol
    assert normwise(np64(dW), rdW) < gtol
    if base:
        assert normwise(np64(ds), rds) < gtol
        assert normwise(np64(dbw), rdbw) < gtol
    else:
        assert ds is None and dbw is None


def test_edge_at_the_in_features_limit(C):
    """in_features = 65535 and R = 72 (the widest augmented rows, k-steps 19 and
    5 column tiles): the fp32 kernels' per-tile buffer offsets reach 15 rows x
    I x R x 4 bytes = 283 MB, and the last feature's rows end at the end of H.
    Forward and backward against the oracle."""
    N, I, O, R = 23, 65535, 2, 72
    print(f"edge at the limit {(N, I, O, R)}", flush=True)
    s, H, bw, W, ga = _edge_inputs(N, I, O, R, torch.float32, seed=11)
    a = C.edge_abs_mean(s.cuda(), H.cuda(), bw.cuda(), W.cuda())
    ra = ko.edge_abs_mean(np64(s), np64(H), np64(bw), np64(W))
    assert normwise(np64(a), ra) < 1e-5
    ds, dH, dbw, dW = C.edge_abs_mean_backward(ga.cuda(), s.cuda(), H.cuda(), bw.cuda(),
                                               W.cuda(), True, True, True, True)
    rds, rdH, rdbw, rdW = ko.edge_abs_mean_backward(np64(ga), np64(s), np64(H), np64(bw),
                                                    np64(W))
    for got, ref in ((ds, rds), (dH, rdH), (dbw, rdbw), (dW, rdW)):
        assert normwise(np64(got), ref) < 1e-4


def test_edge_backward_partial_requests(C):
    s, H, bw, W, ga = _edge_inputs(100, 6, 10, 8, torch.float64, seed=3)
    d = [t.cuda() for t in (s, H, bw, W, ga)]
    ds, dH, dbw, dW = C.edge_abs_mean_backward(d[4], d[0], d[1], d[2], d[3],
                                               False, True, False, False)
    assert ds is None and dbw is None and dW is None and dH is not None
    ds, dH, dbw, dW = C.edge_abs_mean_backward(d[4], d[0], d[1], d[2], d[3],
                                               False, False, True, True)
    assert dH is None and dbw is not None and dW is not None


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_forward_with_regularization_fused_matches_dense(C, dtype):
    from torchsplinekan_amd import KAN
    torch.manual_seed(0)
    net = KAN([6, 8, 5], grid_size=5, backend="cuda").to("cuda", dtype)
    x = (torch.rand(200, 6, device="cuda", dtype=dtype) * 2.4 - 1.2)
    res = {}
    for impl in ("fused", "dense", "checkpoint"):
        for p in net.parameters():
            p.grad = None
        xx = x.clone().requires_grad_()
        y, r = net.forward_with_regularization(xx, 1e-2, 1e-2, reg_impl=impl, chunk_size=64)
        (y.square().mean() + r).backward()
        res[impl] = [y.detach(), r.detach(), xx.grad] + [p.grad for p in net.parameters()]
    tol = 1e-10 if dtype == torch.float64 else 5e-5
    for impl in ("dense", "checkpoint"):
        for a, b in zip(res["fused"], res[impl]):
            assert normwise(np64(a), np64(b)) < tol
