"""GPU parity of the fused edge statistic a[o,i] = mean_n |phi[n,o,i]| and its
backward against the CPU oracle, and of forward_with_regularization with
reg_impl="fused" against the dense path (mirrors
tests/test_fused_regularization.py:58-107 of the reference).
"""

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests import _netcheck, _slack
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
# 129..256 -> 4x1 (200), 257..512 -> 8x1 (300, 512).  The forward of layers with
# O <= 64 and R + 1 <= 16 stages groups of 4 features through LDS, with 16-byte
# loads where I % 4 == 0 (I = 4, 8, 12, 16, 260; every k-step class) and scalar loads
# with partial groups otherwise (I = 1, 3, 5, 7); O = 3..64.
SHAPES = [(37, 5, 3, 4), (300, 16, 40, 8), (1000, 9, 70, 13), (64, 3, 300, 68),
          (5000, 4, 6, 11), (77, 3, 5, 1), (513, 2, 33, 20), (129, 3, 17, 29), (70, 2, 9, 44),
          (200, 2, 1300, 11), (3000, 3, 600, 7), (2000, 3, 200, 11), (4097, 5, 64, 11),
          (8192, 260, 20, 7), (2100, 3, 512, 11), (700, 2, 300, 8), (1200, 3, 100, 3),
          (333, 7, 48, 14), (1500, 1, 64, 10), (999, 8, 50, 15), (130, 12, 10, 2)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("base", [True, False])
@pytest.mark.parametrize("route", ["auto", "separate"])
def test_edge_abs_mean_and_backward_match_oracle(C, routes, shape, dtype, base, route):
    """route "auto": fp32 layers with O <= 512 and R + 1 <= 16 take the fused
    backward kernel (both gradient sides from one phi); "separate" forces the
    parameter and input kernels (edge_fused route 0)."""
    N, I, O, R = shape
    if route == "separate" and dtype == torch.float64:
        pytest.skip("the route applies to the fp32 MFMA kernels only")
    routes.set_route("edge_fused", 0 if route == "separate" else 1)
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
    if not base:
        assert ds is None and dbw is None
    _check_edge_grads((ds, dH, dbw, dW), ga, s if base else None, H, bw if base else None, W,
                      dtype)


def _check_edge_grads(got, ga, s, H, bw, W, dtype, D=None, which=(True, True, True, True)):
    """Device edge gradients against the oracle: fp64 at 1e-12 and fp32 at
    1e-5 normwise, with the terms whose sign the device's precision cannot
    decide (|phi| within its rounding bound) counted and bounded term by
    term (tests/_slack.py; operands shared exactly, so no extra allowance)."""
    a = lambda t: None if t is None else np64(t)
    fp64 = dtype == torch.float64
    refs, slacks, n_amb = _slack.edge_backward_full(a(ga), a(s), a(H), a(bw), a(W), D=a(D),
                                                    extra=0, unit=2.0 ** -53 if fp64 else 2.0 ** -24)
    N, O, I = H.shape[0], W.shape[0], W.shape[1]
    tol = 1e-12 if fp64 else 1e-5
    names = ("ds", "dH", "dbw", "dW")
    for name, want, g, ref, slack in zip(names, which, got, refs, slacks):
        if not want or ref is None:
            continue
        e = _slack.within(np64(g), ref, slack, tol)
        assert e < tol, (name, e, n_amb)
    print(f"  {n_amb} of {N * O * I} terms within {'fp64' if fp64 else 'fp32'} rounding of "
          "phi = 0", flush=True)
    assert n_amb <= max(3, 1e-4 * N * O * I)


@pytest.mark.parametrize("shape", [(23, 65535, 2, 72), (23, 65535, 5, 11), (70, 65532, 40, 14)])
def test_edge_at_the_in_features_limit(C, shape):
    """in_features at the limit.  R = 72 (the widest augmented rows, k-steps 19
    and 5 column tiles): the fp32 kernels' per-tile buffer offsets reach 15
    rows x I x R x 4 bytes = 283 MB, and the last feature's rows end at the
    end of H.  O <= 64 with R + 1 <= 16 takes the kernels staged through LDS:
    I = 65535 (scalar loads, a last group of 3 features; chunk offsets up to
    22 rows x I x R x 4 bytes) and I = 65532 (16-byte loads, two chunks per
    split with a ragged second one).  Forward and backward against the
    oracle."""
    N, I, O, R = shape
    print(f"edge at the limit {(N, I, O, R)}", flush=True)
    s, H, bw, W, ga = _edge_inputs(N, I, O, R, torch.float32, seed=11)
    a = C.edge_abs_mean(s.cuda(), H.cuda(), bw.cuda(), W.cuda())
    ra = ko.edge_abs_mean(np64(s), np64(H), np64(bw), np64(W))
    assert normwise(np64(a), ra) < 1e-5
    ds, dH, dbw, dW = C.edge_abs_mean_backward(ga.cuda(), s.cuda(), H.cuda(), bw.cuda(),
                                               W.cuda(), True, True, True, True)
    _check_edge_grads((ds, dH, dbw, dW), ga, s, H, bw, W, torch.float32)


def test_edge_backward_partial_requests(C):
    s, H, bw, W, ga = _edge_inputs(100, 6, 10, 8, torch.float64, seed=3)
    d = [t.cuda() for t in (s, H, bw, W, ga)]
    ds, dH, dbw, dW = C.edge_abs_mean_backward(d[4], d[0], d[1], d[2], d[3],
                                               False, True, False, False)
    assert ds is None and dbw is None and dW is None and dH is not None
    ds, dH, dbw, dW = C.edge_abs_mean_backward(d[4], d[0], d[1], d[2], d[3],
                                               False, False, True, True)
    assert dH is None and dbw is not None and dW is not None


@pytest.mark.parametrize("shape", [(700, 8, 40, 11), (300, 7, 64, 11)])
def test_edge_backward_partial_requests_fp32(C, shape):
    """fp32 requests of some gradients only (narrow layers, whose full
    request takes the backward staged through LDS with 16-byte or scalar
    row stores; a one-sided request takes the input or the parameter
    kernel): the requested gradients hold the oracle bar, the others are not
    returned."""
    N, I, O, R = shape
    s, H, bw, W, ga = _edge_inputs(N, I, O, R, torch.float32, seed=I + O)
    d = [t.cuda() for t in (s, H, bw, W, ga)]
    for which in ((True, True, True, True), (True, False, False, False),
                  (False, True, False, False), (True, True, False, False),
                  (False, False, True, True), (True, False, False, True)):
        got = C.edge_abs_mean_backward(d[4], d[0], d[1], d[2], d[3], *which)
        assert all((g is None) == (not w) for g, w in zip(got, which)), which
        _check_edge_grads(got, ga, s, H, bw, W, torch.float32, which=which)


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
# and R + 1 at 2, 5, 12 and 16.
LINEAR_SHAPES = [(37, 5, 4, 4), (90, 3, 7, 6), (300, 7, 64, 11), (250, 4, 33, 11),
                 (1000, 9, 100, 15), (513, 3, 200, 11), (700, 2, 300, 8), (4097, 5, 512, 11),
                 (6000, 3, 64, 11), (2000, 8, 64, 11), (500, 12, 10, 3), (777, 16, 24, 14),
                 (90, 3, 20, 1)]


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
    _check_edge_grads((ds, dH, dbw, dW), ga, s, H, bw, W, torch.float32, D=gy)
    # a partial request leaves the other outputs unwritten and the rest equal
    ds2, dH2, dbw2, dW2 = C.edge_linear_backward(ga.cuda(), gy.cuda(), s.cuda(), H.cuda(),
                                                 bw.cuda(), W.cuda(), False, True, False, True)
    assert ds2 is None and dbw2 is None
    assert torch.equal(dH2, dH) and torch.equal(dW2, dW)
    # weight gradients only: the parameter kernel with grad_y added
    ds3, dH3, dbw3, dW3 = C.edge_linear_backward(ga.cuda(), gy.cuda(), s.cuda(), H.cuda(),
                                                 bw.cuda(), W.cuda(), False, False, True, True)
    assert ds3 is None and dH3 is None
    _check_edge_grads((None, None, dbw3, dW3), ga, s, H, bw, W, torch.float32, D=gy,
                      which=(False, False, True, True))


# (N, I, O, R) of the one-pass forward (128 x 128 blocks): partial sample
# and output blocks, a single block, several of each, outputs past 512, every
# k-step count (R + 1 = 2, 5, 8, 12, 15, 16), 16-byte staging (I % 4 == 0)
# and scalar staging with a partial last feature group (I % 4 != 0).
YLIN_SHAPES = [(37, 5, 4, 4), (300, 7, 64, 11), (1000, 9, 100, 15), (513, 3, 200, 11),
               (4097, 8, 512, 11), (777, 16, 130, 14), (90, 3, 20, 1), (129, 12, 257, 7),
               (2000, 4, 600, 4), (256, 6, 128, 11), (128, 1, 1, 3)]


@pytest.mark.parametrize("shape", YLIN_SHAPES)
def test_edge_linear_forward_matches_oracle(C, shape):
    """kan_hip_edge_linear_forward: the layer output y = s bw^T + H W^T and
    the edge statistic a = mean_n |phi| from one pass over phi, against the
    float64 products and the oracle's edge_abs_mean (fp32 1e-5 normwise);
    repeated calls are bit-identical; without a base branch as well."""
    N, I, O, R = shape
    print(f"edge linear forward {shape}", flush=True)
    s, H, bw, W, _ = _edge_inputs(N, I, O, R, torch.float32, seed=3 * N + O)
    assert C.edge_linear_forward_supported(H.cuda(), W.cuda())
    for base in (True, False):
        sd, bwd = (s.cuda(), bw.cuda()) if base else (None, None)
        y, a = C.edge_linear_forward(sd, H.cuda(), bwd, W.cuda())
        y2, a2 = C.edge_linear_forward(sd, H.cuda(), bwd, W.cuda())
        assert torch.equal(y, y2) and torch.equal(a, a2)
        ry = np64(H).reshape(N, I * R) @ np64(W).reshape(O, I * R).T
        if base:
            ry = ry + np64(s) @ np64(bw).T
        ra = ko.edge_abs_mean(np64(s) if base else None, np64(H), np64(bw) if base else None,
                              np64(W))
        assert normwise(np64(y), ry) < 1e-5, ("y", base)
        assert normwise(np64(a), ra) < 1e-5, ("a", base)


def test_edge_linear_supported_range(C):
    mk = lambda N, I, O, R, dt=torch.float32: (torch.empty(N, I, R, dtype=dt, device="cuda"),
                                               torch.empty(O, I, R, dtype=dt, device="cuda"))
    assert C.edge_linear_supported(*mk(10, 3, 512, 15))
    assert not C.edge_linear_supported(*mk(10, 3, 516, 11))   # O > 512
    assert C.edge_linear_supported(*mk(10, 3, 70, 11))
    assert not C.edge_linear_supported(*mk(10, 3, 64, 16))    # R + 1 > 16
    assert not C.edge_linear_supported(*mk(10, 3, 64, 11, torch.float64))
    assert C.edge_linear_forward_supported(*mk(10, 3, 1300, 15))
    assert not C.edge_linear_forward_supported(*mk(10, 3, 64, 16))    # R + 1 > 16
    assert not C.edge_linear_forward_supported(*mk(10, 3, 64, 11, torch.float64))


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


@pytest.mark.parametrize("widths,N", [([16, 64, 100, 12], 3000), ([8, 300, 6], 16384)])
@pytest.mark.parametrize("x_grad", [True, False])
@pytest.mark.parametrize("route", ["folded", "unfolded", "dense"])
def test_regularized_layers_match_oracle(C, monkeypatch, x_grad, route, widths, N):
    """KAN([16, 64, 100, 12]) at N = 3000 and KAN([8, 300, 6]) at N = 16384,
    fp32, forward_with_regularization + loss +
    backward through each route, every layer held to the fp64 oracle
    (tests/_netcheck.py, full mode: every element of the outputs, the
    parameter gradients and the input gradients, block by block, and the
    regulariser) at 1e-5 with sign flips of phi at fp32 rounding level
    counted and bounded term by term:
    * "folded": output and edge statistic through EdgeLinear (one folded
      native backward launch per layer; the weight-only branch for the first
      layer when x needs no gradient; the 300-wide layer's forward from one
      pass over phi, kan_hip_edge_linear_forward);
    * "unfolded": the separate native output products and edge backward,
      summed by autograd;
    * "dense": the PyTorch dense path (reg_impl="dense").
    All three meeting the same oracle bar shows that their differences are
    the counted flips."""
    from torchsplinekan_amd import KAN
    from torchsplinekan_amd import fused as fz
    print(f"regularised KAN({widths}) N={N} route={route} x_grad={x_grad}", flush=True)
    torch.manual_seed(1)
    net = KAN(widths, grid_size=7, backend="cuda").to("cuda")
    x = (torch.rand(N, widths[0], device="cuda") * 2.2 - 1.1).requires_grad_(x_grad)
    if route == "folded" and widths[1] >= 256:
        assert fz._one_pass_forward(N, widths[1], 7 + 3, x.device)
    if route == "unfolded":
        monkeypatch.setattr(fz, "edge_linear_applies", lambda *a: False)
    impl = "dense" if route == "dense" else "fused"
    with _netcheck.capture(net) as cap:
        y, r = net.forward_with_regularization(x, 1e-2, 1e-2, reg_impl=impl, chunk_size=256)
        (y.square().mean() + r).backward()
        torch.cuda.synchronize()
    assert all(l.last_backend == ("reference" if route == "dense" else "cuda")
               for l in net.layers)
    reg = _netcheck.check_layers(net, cap, 1e-2, 3, 1e-5,
                                 say=lambda m: print("  " + m, flush=True), full=True)
    assert abs(r.item() - reg) < 1e-5 * abs(reg)
    if x_grad:
        assert x.grad is not None


def test_regularized_layers_folded_backward_recorded(C):
    """create_graph through EdgeLinear (its recorded branch: the separate
    differentiable pieces): first and second derivatives with respect to the
    parameters against the dense path at 1e-5 (the dense path in fp32
    against itself in fp64 differs by at most 4e-7 on these quantities; the
    32,000 phi terms of this network leave an fp32 sign flip unlikely)."""
    from torchsplinekan_amd import KAN
    torch.manual_seed(2)
    net = KAN([6, 8, 4], grid_size=5, backend="cuda").to("cuda")
    x = torch.rand(400, 6, device="cuda") * 2.2 - 1.1
    f = _reg_grads(net, x.clone().requires_grad_(), "fused", create_graph=True)
    d = _reg_grads(net, x.clone().requires_grad_(), "dense", create_graph=True)
    errs = [normwise(np64(a), np64(b)) for a, b in zip(f, d)]
    print("  recorded fused vs dense:", " ".join(f"{e:.1e}" for e in errs), flush=True)
    assert max(errs) < 1e-5
