"""GPU parity at BASELINE.json's workloads themselves, built by the same
functions bench.py times (bench.build_c2 .. build_c5), against the fp64
oracle at the north star's fp32 bar (normwise relative 1e-5):

* c3: KANLinear 1024 -> 1024 G10 k3, N = 65536, x with grad: every element
  of y, dx, dcoef, dscaler and dbase_w (tests/_fullcheck.py: the oracle in
  row chunks; each tensor held to the bar block by block, so one faulty
  output tile of the c3 schedule cannot hide in the whole-tensor norm).
  The same step in float64: every element, block by block, at 1e-12.
* c5: KANLinear 4096 -> 256 G65 k3, N = 8192 (N I (G + 2k) = 2.38e9, past
  the reference's 32-bit guard): the same whole-tensor checks, exact zero
  basis rows outside the knot span, and every element of the edge statistic
  on the c5 basis (2.28e9 elements) and of its backward, block by block
  (tests/_fullcheck.py, check_edge_full).
* c4: KAN([256, 512, 512, 64]) G8 with update_grid knots on the Gaussian
  mixture, forward_with_regularization(1e-2, 1e-2, "auto") + MSE + backward:
  per layer, given its own device input, every element of its output, its
  parameter gradients and its input gradient, block by block
  (tests/_netcheck.py, full mode), and the regulariser from the oracle's
  edge means over all edges, with sign flips of phi at fp32 rounding level
  bounded term by term (tests/_slack.py); the network output on rows
  through the full oracle chain; layer 0's knots against the oracle's
  grid_from_samples.  The same in float64 at 1e-10.
* c2: KAN([784, 256, 10]) G5, N = 4096 + MSE: every output and gradient
  against the full oracle chain.

The matching reference tests hold the native backend to the reference
backend (tests/test_math_correctness.py:284-306); here the bar is the fp64
oracle.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kan_oracle as ko
from tests import _netcheck
from tests._util import normwise, np64

pytestmark = pytest.mark.gpu

TOL = 1e-5
# Bound for comparisons against the whole fp64 chain through several layers
# (not a kernel's parity: each layer is held to TOL given its own inputs).
CHAIN_TOL = 3e-5


@pytest.fixture(scope="module")
def bench():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    import bench as b
    return b


def _say(*a):
    print(*a, flush=True)


_params = _netcheck.params
basis_threaded = _netcheck.basis_threaded


def _check_whole_step(L, xd, td, x_cpu, k, tag, tol=TOL):
    """One training step of a single KANLinear (the bench's step); every
    element of its outputs against the oracle (tests/_fullcheck.py), each
    tensor block by block within tol."""
    from tests import _fullcheck
    for p in L.parameters():
        p.grad = None
    y = L(xd)
    F.mse_loss(y, td).backward()
    torch.cuda.synchronize()
    assert L.last_backend == "cuda"
    N, O = y.shape
    D = 2.0 * (np64(y) - np64(td)) / (N * O)
    errs = _fullcheck.check_layer_step(L, x_cpu, y.detach(), xd.grad, D, k,
                                       lambda m: _say(f"{tag}: {m}"))
    for name, (worst, block, whole) in errs.items():
        _say(f"{tag}: {name} whole-tensor {whole:.2e}, worst block {worst:.2e} at {block}")
    for name, (worst, block, whole) in errs.items():
        assert worst < tol, (name, worst, block)


@pytest.mark.timeout(900)
def test_c3_training_step_matches_oracle(bench):
    dev = torch.device("cuda", 0)
    L, xd, td, cpu = bench.build_c3(dev, 65536, need_dx=True)
    _say("c3: KANLinear 1024->1024 G10 k3 N=65536 fwd+MSE+bwd with dx, every element")
    _check_whole_step(L, xd, td, cpu[0], 3, tag="c3")


@pytest.mark.timeout(900)
def test_c3_fp64_training_step_matches_oracle(bench):
    """c3 in float64 (bench.py --dtype f64: the same draws cast after they
    are made), its three products on the fp64 MFMA tiles the cost model
    picks at this size: every element at the fp64 bar, 1e-12."""
    dev = torch.device("cuda", 0)
    L, xd, td, cpu = bench.build_c3(dev, 65536, need_dx=True, dtype=torch.float64)
    _say("c3-f64: KANLinear 1024->1024 G10 k3 N=65536 fp64 fwd+MSE+bwd with dx, every element")
    _check_whole_step(L, xd, td, cpu[0], 3, tag="c3-f64", tol=1e-12)


@pytest.mark.timeout(900)
def test_c5_kernel_limit_layer_full_size(bench):
    dev = torch.device("cuda", 0)
    L, x, target = bench.build_c5(dev, 8192)
    N, I = x.shape
    k = 3
    assert N * I * (L.grid_size + 2 * k) > 2 ** 31 - 1   # past the reference's guard
    xd, td = x.to(dev).requires_grad_(), target.to(dev)
    _say("c5: KANLinear 4096->256 G65 k3 N=8192 fwd+MSE+bwd with dx, every element")
    _check_whole_step(L, xd, td, x, k, tag="c5")
    # basis past 2^31 elements: exact zero rows outside [t_0, t_71], values on rows
    from torchsplinekan_amd import _C
    with torch.no_grad():
        Hg = _C.basis(xd.detach(), L.grid, k)
        assert Hg.numel() > 2 ** 31
        xg = xd.detach()
        out = (xg < L.grid[:, 0][None]) | (xg > L.grid[:, -1][None])
        frac = out.float().mean().item()
        _say(f"c5: {frac:.4f} of inputs outside the knot span")
        assert 0.004 < frac < 0.01
        assert int((Hg[out] != 0).sum()) == 0
        inside = ~out
        assert bool(((Hg.sum(-1) - 1.0).abs()[inside & (xg.abs() <= 1.0)] < 1e-5).all())
    rows = [0, 4095, N - 1]
    rH = ko.basis_dense(x[rows].double().numpy(), np64(L.grid), k)
    assert np.abs(np64(Hg[rows]) - rH).max() < 2e-6
    # edge statistic on the c5 basis and its backward (separate route: R + 1 = 69)
    s = torch.nn.functional.silu(xg)
    W = (L.spline_weight * L.spline_scaler.unsqueeze(-1)).detach()
    bw = L.base_weight.detach()
    a = _C.edge_abs_mean(s, Hg, bw, W)
    ga = torch.randn(a.shape, generator=torch.Generator().manual_seed(9)).to(dev)
    ds, dH, dbw, dW = _C.edge_abs_mean_backward(ga, s, Hg, bw, W, True, True, True, True)
    torch.cuda.synchronize()
    del Hg
    xs = x.detach().double().numpy()
    devres = {"a": a.cpu().numpy(), "ds": ds.cpu().numpy(), "dH": dH.cpu().numpy(),
              "dbw": dbw.cpu().numpy(), "dW": dW.cpu().numpy()}
    del a, ds, dH, dbw, dW
    from tests import _fullcheck
    res, n_amb = _fullcheck.check_edge_full(xs, np64(L.grid), k, np64(bw), np64(W), np64(ga),
                                            devres)
    O = W.shape[0]
    for name, (worst, block, whole) in res.items():
        _say(f"c5 edge: {name} every entry, whole {whole:.2e}, worst block {worst:.2e} at "
             f"{block} ({n_amb} of {N * O * I} terms ambiguous)")
        assert worst < TOL, name
    assert n_amb <= 1e-4 * N * O * I


@pytest.mark.timeout(1200)
def test_c4_regularised_network_matches_oracle(bench):
    dev = torch.device("cuda", 0)
    net, xd, td = bench.build_c4(dev, 16384)
    N = xd.shape[0]
    k = 3
    mu = 1e-2
    _say("c4: KAN([256,512,512,64]) G8 update_grid knots, forward_with_regularization")
    # layer 0's knots against the oracle's grid_from_samples on the same samples
    L0 = net.layers[0]
    rg = ko.grid_from_samples(np64(xd), 8, k, L0._ref.grid_eps)
    e = normwise(np64(L0.grid), rg)
    _say(f"c4: layer-0 knots vs grid_from_samples {e:.2e}")
    assert e < 1e-6
    # one training step (the bench's), each layer's input, output and regulariser captured
    with _netcheck.capture(net) as cap:
        for p in net.parameters():
            p.grad = None
        y, reg = net.forward_with_regularization(xd, mu, mu, reg_impl="auto")
        (F.mse_loss(y, td) + reg).backward()
        torch.cuda.synchronize()
    assert all(l.last_backend == "cuda" for l in net.layers) and len(cap) == 3
    # network output on rows through the full fp64 oracle chain (fp32 rounding
    # of the hidden activations carried through three layers: 8.8e-6 here);
    # each layer is held to TOL below, given its own device input
    rows = np.unique(np.linspace(0, N - 1, 32).astype(int))
    h = np64(xd)[rows]
    for layer in net.layers:
        grid, bw, sw, sc = _netcheck.params(layer)
        h, _ = ko.kan_forward(h, grid, bw, sw, sc, k)
    e = normwise(np64(y[rows]), h)
    _say(f"c4: network output rows through the fp64 chain from x {e:.2e}")
    assert e < CHAIN_TOL
    reg_total = _netcheck.check_layers(net, cap, mu, k, TOL, say=lambda m: _say("c4 " + m),
                                       full=True)
    e = abs(reg.item() - reg_total) / abs(reg_total)
    _say(f"c4: total regulariser {e:.2e}")
    assert e < TOL


@pytest.mark.timeout(1200)
def test_c4_regularised_network_fp64_matches_oracle(bench):
    """c4 in float64 (the edge statistic on the fp64 MFMA kernels, the layer
    products on the fp64 GEMM): every element of each layer's outputs and
    gradients against the oracle given its own device input, at 1e-10, with
    sign ambiguity bounded at float64's unit roundoff; the network output
    through the whole fp64 chain from x."""
    dev = torch.device("cuda", 0)
    net, xd, td = bench.build_c4(dev, 16384, torch.float64)
    N = xd.shape[0]
    k = 3
    mu = 1e-2
    tol = 1e-10
    _say("c4 fp64: KAN([256,512,512,64]) G8 update_grid knots, forward_with_regularization")
    with _netcheck.capture(net) as cap:
        for p in net.parameters():
            p.grad = None
        y, reg = net.forward_with_regularization(xd, mu, mu, reg_impl="auto")
        (F.mse_loss(y, td) + reg).backward()
        torch.cuda.synchronize()
    assert all(l.last_backend == "cuda" for l in net.layers) and len(cap) == 3
    rows = np.unique(np.linspace(0, N - 1, 32).astype(int))
    h = np64(xd)[rows]
    for layer in net.layers:
        grid, bw, sw, sc = _netcheck.params(layer)
        h, _ = ko.kan_forward(h, grid, bw, sw, sc, k)
    e = normwise(np64(y[rows]), h)
    _say(f"c4 fp64: network output rows through the fp64 chain from x {e:.2e}")
    assert e < tol
    reg_total = _netcheck.check_layers(net, cap, mu, k, tol, say=lambda m: _say("c4 fp64 " + m),
                                       unit=2.0 ** -53, full=True)
    e = abs(reg.item() - reg_total) / abs(reg_total)
    _say(f"c4 fp64: total regulariser {e:.2e}")
    assert e < tol


@pytest.mark.timeout(900)
def test_c2_network_matches_oracle(bench):
    """Each layer against the oracle given its own device input and the
    device's gradient of its output (all rows, all edges): outputs, dx and
    the three parameter gradients at 1e-5.  The whole fp64 chain from x is
    compared as well, at the propagation bound CHAIN_TOL: fp32 rounding of
    the hidden activations is carried through the later layer and its
    backward by any fp32 implementation (the chain's dx is 1.0e-5 here)."""
    dev = torch.device("cuda", 0)
    net, x, target = bench.build_c2(dev, 4096)
    xd, td = x.to(dev).requires_grad_(), target.to(dev)
    k = 3
    _say("c2: KAN([784,256,10]) G5 N=4096 fwd+MSE+bwd")
    cap = []

    def hook(module, inputs, out):
        if inputs[0].requires_grad:
            inputs[0].retain_grad()
        out.retain_grad()
        cap.append((inputs[0], out))

    handles = [l.register_forward_hook(hook) for l in net.layers]
    try:
        y = net(xd)
        F.mse_loss(y, td).backward()
        torch.cuda.synchronize()
    finally:
        for h in handles:
            h.remove()
    assert all(l.last_backend == "cuda" for l in net.layers) and len(cap) == 2
    chain = x.detach().double().numpy()
    for li, (layer, (xl, yl)) in enumerate(zip(net.layers, cap)):
        grid, bw, sw, sc = _params(layer)
        xs = np64(xl)
        H = basis_threaded(xs, grid, k)
        ry, _ = ko.kan_forward(xs, grid, bw, sw, sc, k, basis=H)
        chain, _ = ko.kan_forward(chain, grid, bw, sw, sc, k)
        D = np64(yl.grad)
        gx, gbw, gsw, gsc = ko.kan_backward(D, xs, grid, bw, sw, sc, k, basis=H)
        for name, got, ref in (("y", yl, ry), ("dx", xl.grad, gx),
                               ("dbase_w", layer.base_weight.grad, gbw),
                               ("dcoef", layer.spline_weight.grad, gsw),
                               ("dscaler", layer.spline_scaler.grad, gsc)):
            e = normwise(np64(got), ref)
            _say(f"c2 layer {li}: {name} {e:.2e}")
            assert e < TOL, (li, name)
    e = normwise(np64(y), chain)
    _say(f"c2: network output through the fp64 chain from x {e:.2e}")
    assert e < CHAIN_TOL
