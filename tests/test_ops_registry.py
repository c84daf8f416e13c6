"""The op registry of the boundary: torch.ops.spline_kan.kan_forward /
kan_backward with CPU, CUDA (ROCm device) and Meta kernels, as the
reference registers them (csrc/kan_ext.cpp:62-155).  CPU and device results
against the oracle; Meta / FakeTensor shapes and an FX trace for the shape
contract tracing relies on."""

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests._util import make_grid, normwise, np64


@pytest.fixture(scope="module")
def ops():
    from torchsplinekan_amd import _C  # noqa: F401  (registers the ops)
    return torch.ops.spline_kan


def _inputs(N, I, O, G, k, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(N, I, generator=g, dtype=torch.float64) * 2.2 - 1.1).to(dtype)
    grid = make_grid(I, G, k, "nonuniform", seed=seed, dtype=dtype)
    sw = (torch.randn(O, I, G + k, generator=g, dtype=torch.float64) * 0.1).to(dtype)
    bw = (torch.randn(O, I, generator=g, dtype=torch.float64) * 0.3).to(dtype)
    sc = (torch.rand(O, I, generator=g, dtype=torch.float64) + 0.5).to(dtype)
    D = torch.randn(N, O, generator=g, dtype=torch.float64).to(dtype)
    return x, grid, bw, sw, sc, D


def _check(ops, dev, dtype, has_base, has_scaler, tol):
    N, I, O, G, k = 70, 9, 5, 6, 3
    x, grid, bw, sw, sc, D = _inputs(N, I, O, G, k, dtype)
    empty = torch.empty(0, dtype=dtype, device=dev)
    d = lambda t: t.to(dev)
    y, H = ops.kan_forward(d(x), d(grid), d(bw) if has_base else empty, d(sw),
                           d(sc) if has_scaler else empty, k, has_scaler)
    assert H.shape == (N, I, G + k) and H.is_contiguous()
    a = lambda t, on: np64(t) if on else None
    ry, rH = ko.kan_forward(np64(x), np64(grid), a(bw, has_base), np64(sw), a(sc, has_scaler), k)
    assert normwise(np64(y), ry) < tol and normwise(np64(H), rH) < tol
    gx, gbw, gsw, gsc = ops.kan_backward(d(D), d(x), d(grid), d(bw) if has_base else empty,
                                         d(sw), d(sc) if has_scaler else empty, H, k, has_scaler)
    rgx, rgbw, rgsw, rgsc = ko.kan_backward(np64(D), np64(x), np64(grid), a(bw, has_base),
                                            np64(sw), a(sc, has_scaler), k, basis=rH)
    assert normwise(np64(gx), rgx) < tol and normwise(np64(gsw), rgsw) < tol
    assert (gbw is None) == (not has_base) and (gsc is None) == (not has_scaler)
    if has_base:
        assert normwise(np64(gbw), rgbw) < tol
    if has_scaler:
        assert normwise(np64(gsc), rgsc) < tol


@pytest.mark.parametrize("has_base,has_scaler", [(True, True), (False, True), (True, False)])
def test_cpu_ops_match_oracle(ops, has_base, has_scaler):
    _check(ops, "cpu", torch.float64, has_base, has_scaler, 1e-12)


def test_cpu_ops_validate_like_the_reference(ops):
    x, grid, bw, sw, sc, _ = _inputs(8, 4, 3, 5, 3, torch.float64)
    with pytest.raises(RuntimeError, match=r"spline_weight.size\(2\)"):
        ops.kan_forward(x, grid, bw, sw[:, :, :-1], sc, 3, True)


def test_meta_and_fake_shapes(ops):
    from torch._subclasses.fake_tensor import FakeTensorMode
    B, I, O, G, k = 6, 5, 4, 7, 2
    nk = G + 2 * k + 1
    m = lambda *s: torch.empty(*s, device="meta")
    y, H = ops.kan_forward(m(B, I), m(I, nk), m(O, I), m(O, I, G + k), m(O, I), k, True)
    assert y.shape == (B, O) and H.shape == (B, I, G + k) and y.device.type == "meta"
    gx, gbw, gsw, gsc = ops.kan_backward(m(B, O), m(B, I), m(I, nk), m(0), m(O, I, G + k), m(O, I),
                                         H, k, True)
    assert gx.shape == (B, I) and gbw is None and gsw.shape == (O, I, G + k) and gsc.shape == (O, I)
    with FakeTensorMode():
        f = lambda *s: torch.empty(*s, dtype=torch.float32)
        y, H = ops.kan_forward(f(B, I), f(I, nk), f(O, I), f(O, I, G + k), f(0), k, False)
        assert y.shape == (B, O) and H.shape == (B, I, G + k) and y.dtype == torch.float32
        out = ops.kan_backward(f(B, O), f(B, I), f(I, nk), f(O, I), f(O, I, G + k), f(0), H, k,
                               False)
        assert out[1].shape == (O, I) and out[3] is None


def test_fx_trace_records_the_ops(ops):
    from torch.fx.experimental.proxy_tensor import make_fx
    x, grid, bw, sw, sc, D = _inputs(16, 4, 3, 5, 3, torch.float64)

    def step(x, grid, bw, sw, sc, D):
        y, H = ops.kan_forward(x, grid, bw, sw, sc, 3, True)
        return y, ops.kan_backward(D, x, grid, bw, sw, sc, H, 3, True)

    gm = make_fx(step, tracing_mode="fake")(x, grid, bw, sw, sc, D)
    targets = {str(n.target) for n in gm.graph.nodes if n.op == "call_function"}
    assert "spline_kan.kan_forward.default" in targets
    assert "spline_kan.kan_backward.default" in targets
    y_ref, g_ref = step(x, grid, bw, sw, sc, D)
    y_fx, g_fx = gm(x, grid, bw, sw, sc, D)
    assert torch.equal(y_ref, y_fx) and all(torch.equal(a, b) for a, b in zip(g_ref, g_fx))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("has_base,has_scaler", [(True, True), (False, True), (True, False)])
def test_device_ops_match_oracle(ops, dtype, has_base, has_scaler):
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    print(f"torch.ops.spline_kan on device {dtype} base={has_base} scaler={has_scaler}",
          flush=True)
    _check(ops, "cuda", dtype, has_base, has_scaler, 1e-12 if dtype == torch.float64 else 1e-5)
