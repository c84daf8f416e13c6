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


# (N, I, O, R): every tiling of the folded backward (O = 4, 7 -> 2x4, 33, 64 ->
# 4x4, 100 -> 4x2, 200 -> 4x1, 300 and 512 -> 8x1; odd widths leave partial
# output tiles), ragged sample counts, sample splits across blocks (4097, 6000)
# and R + 1 at 5, 12 and 16.
LINEAR_SHAPES = [(37, 5, 4, 4), (90, 3, 7, 6), (300, 7, 64, 11), (250, 4, 33, 11),
                 (1000, 9, 100, 15), (513, 3, 200, 11), (700, 2, 300, 8), (4097, 5, 512, 11),
                 (6000, 3, 64, 11)]


@pytest.mark.parametrize("shape", LINEAR_SHAPES)
def test_edge_linear_backward_matches_oracle(C, shape):
    """kan_hip_edge_linear_backward: the gradients of a layer's output
    y = s bw^T + H W^T and of its edge statistic together (grad_y folded into
    the edge kernel's g) against the oracle's edge backward plus the linear
    layer's products in float64."""
    N, I, O, R = shape
    print(f"edge linear {shape}", flush=True)
    s, H, bw, W, ga = _edge_inputs(N, I, O, R, torch.float32, seed=N + 7 * O)
    gy = torch.randn(N, O, generator=torch.Generator().manual_seed(O), dtype=torch.float64).float()
    assert C.edge_linear_supported(H.cuda(), W.cuda())
    ds, dH, dbw, dW = C.edge_linear_backward(ga.cuda(), gy.cuda(), s.cuda(), H.cuda(), bw.cuda(),
                                             W.cuda(), True, True, True, True)
    rds, rdH, rdbw, rdW = ko.edge_abs_mean_backward(np64(ga), np64(s), np64(H), np64(bw), np64(W))
    D = np64(gy)
    rds = rds + D @ np64(bw)
    rdH = rdH + (D @ np64(W).reshape(O, I * R)).reshape(N, I, R)
    rdbw = rdbw + D.T @ np64(s)
    rdW = rdW + (D.T @ np64(H).reshape(N, I * R)).reshape(O, I, R)
    for name, got, ref in (("ds", ds, rds), ("dH", dH, rdH), ("dbw", dbw, rdbw), ("dW", dW, rdW)):
        assert normwise(np64(got), ref) < 1e-4, name
    # a partial request leaves the other outputs unwritten and the rest equal
    ds2, dH2, dbw2, dW2 = C.edge_linear_backward(ga.cuda(), gy.cuda(), s.cuda(), H.cuda(),
                                                 bw.cuda(), W.cuda(), False, True, False, True)
    assert ds2 is None and dbw2 is None
    assert torch.equal(dH2, dH) and torch.equal(dW2, dW)
    # weight gradients only: the parameter kernel with grad_y added
    ds3, dH3, dbw3, dW3 = C.edge_linear_backward(ga.cuda(), gy.cuda(), s.cuda(), H.cuda(),
                                                 bw.cuda(), W.cuda(), False, False, True, True)
    assert ds3 is None and dH3 is None
    assert normwise(np64(dbw3), rdbw) < 1e-4 and normwise(np64(dW3), rdW) < 1e-4


def test_edge_linear_supported_range(C):
    mk = lambda N, I, O, R, dt=torch.float32: (torch.empty(N, I, R, dtype=dt, device="cuda"),
                                               torch.empty(O, I, R, dtype=dt, device="cuda"))
    assert C.edge_linear_supported(*mk(10, 3, 512, 15))
    assert not C.edge_linear_supported(*mk(10, 3, 516, 11))   # O > 512
    assert C.edge_linear_supported(*mk(10, 3, 70, 11))
    assert not C.edge_linear_supported(*mk(10, 3, 64, 16))    # R + 1 > 16
    assert not C.edge_linear_supported(*mk(10, 3, 64, 11, torch.float64))


def _reg_grads(net, x, impl, create_graph=False):
    for p in net.parameters():
        p.grad = None
    y, r = net.forward_with_regularization(x, 1e-2, 1e-2, reg_impl=impl, chunk_size=256)
    loss = y.square().mean() + r
    if not create_graph:
        loss.backward()
        return [y.detach(), r.detach()] + [p.grad for p in net.parameters()] + \
               ([x.grad] if x.requires_grad else [])
    params = list(net.parameters())
    gs = torch.autograd.grad(loss, params, create_graph=True)
    second = torch.autograd.grad(sum((g * g).sum() for g in gs), params)
    return list(gs) + list(second)


@pytest.mark.parametrize("x_grad", [True, False])
def test_regularized_layers_folded_backward_match_dense(C, monkeypatch, x_grad):
    """KAN([16, 64, 100, 12]) fp32: every layer's output and edge statistic go
    through EdgeLinear; with x requiring
    grad the first layer takes the folded kernel as well, without it the
    weight-only branch.
    * Gradients against the unfolded native path (separate output products
      and edge backward, summed by autograd): the same kernels form phi, so
      the sign patterns agree and only summation order differs: 1e-5.
    * Output and regulariser against the dense path: 1e-5.  (Gradients of
      the native and the dense path differ by sign flips of phi at rounding
      level, up to 4e-4 normwise on dbw at these sizes, with or without the
      fold; their agreement at the reference's shapes and tolerance is
      test_forward_with_regularization_fused_matches_dense.)"""
    from torchsplinekan_amd import KAN
    from torchsplinekan_amd import fused as fz
    torch.manual_seed(1)
    net = KAN([16, 64, 100, 12], grid_size=7, backend="cuda").to("cuda")
    x = torch.rand(3000, 16, device="cuda") * 2.2 - 1.1
    res = {}
    for impl in ("fused", "dense"):
        xx = x.clone().requires_grad_(x_grad)
        res[impl] = _reg_grads(net, xx, impl)
    monkeypatch.setattr(fz, "edge_linear_applies", lambda *a: False)
    res["unfolded"] = _reg_grads(net, x.clone().requires_grad_(x_grad), "fused")
    for a, b in zip(res["fused"], res["unfolded"]):
        assert normwise(np64(a), np64(b)) < 1e-5
    for a, b in zip(res["fused"][:2], res["dense"][:2]):
        assert normwise(np64(a), np64(b)) < 1e-5


def test_regularized_layers_folded_backward_recorded(C):
    """create_graph through EdgeLinear (its recorded branch: the separate
    differentiable pieces): first and second derivatives with respect to the
    parameters against the dense path."""
    from torchsplinekan_amd import KAN
    torch.manual_seed(2)
    net = KAN([6, 8, 4], grid_size=5, backend="cuda").to("cuda")
    x = torch.rand(400, 6, device="cuda") * 2.2 - 1.1
    f = _reg_grads(net, x.clone().requires_grad_(), "fused", create_graph=True)
    d = _reg_grads(net, x.clone().requires_grad_(), "dense", create_graph=True)
    for a, b in zip(f, d):
        assert normwise(np64(a), np64(b)) < 1e-4
