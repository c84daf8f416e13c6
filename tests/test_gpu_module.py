"""Module-level GPU behaviour of the native backend, after the reference's own
tests of the same API (tests/test_fused_regularization.py:58-219,
tests/test_math_correctness.py:180-360, tests/test_cuda.py:88-95,
tests/test_export.py:24-86, tests/test_grid_extension.py): every
regularisation implementation against the dense one across k, G and base
activations, the cross-layer gradient, the zero layer, no graph state kept on
modules, the fused path's memory bound, device movement, non-SiLU base
activations, the cubic second-derivative identity, the kernel limits and
their fallback, inference export, and grid extension on the device.

Tolerances are the reference tests' own: normwise 1e-10 (fp64) and 5e-5
(fp32) for fused against dense; 1e-12 / 1e-10 for native against the
reference backend in fp64.
"""

import gc
import io

import numpy as np
import pytest
import torch
import torch.nn as nn

from tests._util import make_grid, normwise, np64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from torchsplinekan_amd import _C
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return _C


def _grads(model, x, impl, mu=(0.7, 1.3), chunk=37, use_fwr=True):
    for p in model.parameters():
        p.grad = None
    xx = x.clone().requires_grad_()
    if use_fwr:
        y, r = model.forward_with_regularization(xx, *mu, reg_impl=impl, chunk_size=chunk)
    else:
        y = model(xx)
        r = model.regularization_loss(*mu, x=xx)
    (y.square().mean() + r).backward()
    return [y.detach(), r.detach(), xx.grad] + [p.grad.clone() for p in model.parameters()]


def _close(a, b, rtol):
    for u, v in zip(a, b):
        assert normwise(np64(u), np64(v)) < rtol


@pytest.mark.parametrize("k", [1, 2, 3])
@pytest.mark.parametrize("G", [3, 17, 60])
@pytest.mark.parametrize("act", [nn.SiLU, nn.Tanh])
def test_all_impls_match_dense_multilayer(C, k, G, act):
    from torchsplinekan_amd import KAN
    print(f"reg impls k={k} G={G} act={act.__name__}", flush=True)
    torch.manual_seed(k * 100 + G)
    m = KAN([4, 6, 3], grid_size=G, spline_order=k, base_activation=act,
            backend="cuda").double().cuda()
    x = (torch.rand(129, 4, dtype=torch.float64) * 2.6 - 1.3).cuda()  # beyond the knots too
    ref = _grads(m, x, None, use_fwr=False)
    for impl in ("dense", "checkpoint", "fused"):
        _close(_grads(m, x, impl), ref, 1e-10)


def test_fused_cross_layer_gradient_present(C):
    from torchsplinekan_amd import KAN
    torch.manual_seed(1)
    m = KAN([3, 4, 2], backend="cuda").double().cuda()
    x = torch.rand(40, 3, dtype=torch.float64, device="cuda") * 2 - 1
    h = m.layers[0](x)
    _, r_fused = m.layers[1].forward_with_regularization(h, 1.0, 1.0, reg_impl="fused")
    _, r_dense = m.layers[1].forward_with_regularization(h, 1.0, 1.0, reg_impl="dense")
    gf = torch.autograd.grad(r_fused, list(m.layers[0].parameters()), retain_graph=True)
    gd = torch.autograd.grad(r_dense, list(m.layers[0].parameters()))
    for a, b in zip(gf, gd):
        assert b.abs().max() > 1e-8
        assert torch.allclose(a, b, rtol=1e-10, atol=1e-14)


def test_fused_fp32_matches_dense(C):
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(2)
    m = KANLinear(64, 48, backend="cuda").cuda()
    x = torch.rand(777, 64, device="cuda") * 2 - 1
    _close(_grads(m, x, "fused"), _grads(m, x, "dense"), 5e-5)


def test_zero_layer_finite(C):
    from torchsplinekan_amd import KANLinear
    m = KANLinear(4, 3, backend="cuda").cuda()
    with torch.no_grad():
        m.base_weight.zero_()
        m.spline_weight.zero_()
    x = torch.randn(20, 4, device="cuda")
    _, r = m.forward_with_regularization(x, 1.0, 1.0, reg_impl="fused")
    r.backward()
    assert abs(r.item()) < 1e-30
    assert all(torch.isfinite(p.grad).all() for p in m.parameters())


def test_no_graph_state_cached_on_module(C):
    from torchsplinekan_amd import KAN
    m = KAN([4, 6, 2], backend="cuda").cuda()
    before = {k: type(v) for k, v in m.__dict__.items()}
    x = torch.randn(30, 4, device="cuda", requires_grad=True)
    y, r = m.forward_with_regularization(x, 1.0, 1.0, reg_impl="fused")
    (y.sum() + r).backward()
    for layer in m.layers:
        for k, v in layer.__dict__.items():
            if torch.is_tensor(v):
                assert v.grad_fn is None, k
        assert layer._waug_cache is None      # a training layer keeps no packed weight
    assert {k: type(v) for k, v in m.__dict__.items()} == before


def test_fused_peak_memory_much_lower_than_dense(C):
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(5)
    m = KANLinear(128, 128, backend="cuda").cuda()
    x = torch.rand(2048, 128, device="cuda") * 2 - 1
    peaks = {}
    for impl in ("dense", "fused"):
        for p in m.parameters():
            p.grad = None
        gc.collect()
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        y, r = m.forward_with_regularization(x, 1.0, 1.0, reg_impl=impl)
        (y.sum() + r).backward()
        torch.cuda.synchronize()
        peaks[impl] = torch.cuda.max_memory_allocated() - base
        del y, r
    phi_bytes = 2048 * 128 * 128 * 4
    assert peaks["dense"] > 2 * phi_bytes
    assert peaks["fused"] < 0.5 * phi_bytes


def test_device_movement(C):
    from torchsplinekan_amd import KANLinear
    layer = KANLinear(4, 4)
    x = torch.randn(10, 4)
    y_cpu = layer(x)
    assert layer.last_backend == "reference"
    layer_cuda = layer.cuda()
    y_cuda = layer_cuda(x.cuda())
    assert layer_cuda.last_backend == "cuda"
    assert torch.allclose(y_cpu.cuda(), y_cuda, atol=1e-5)
    assert torch.allclose(layer_cuda.cpu()(x), y_cpu, atol=1e-6)


def _clone_to(ref, backend, device, **kw):
    from torchsplinekan_amd import KANLinear
    m = KANLinear(ref.in_features, ref.out_features, grid_size=ref.grid_size,
                  spline_order=ref.spline_order, backend=backend, **kw).to(ref.grid.dtype)
    m.load_state_dict(ref.state_dict())
    return m.to(device)


@pytest.mark.parametrize("act", [nn.Tanh, nn.Identity, nn.GELU])
def test_native_executes_non_silu_activation(C, act):
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(4)
    ref = KANLinear(4, 3, base_activation=act, backend="reference").double()
    cu = _clone_to(ref, "cuda", "cuda", base_activation=act)
    x = torch.randn(10, 4, dtype=torch.float64) * 0.8
    y = cu(x.cuda())
    assert cu.last_backend == "cuda"
    assert torch.allclose(y.cpu(), ref(x), atol=1e-12)
    xc = x.cuda().requires_grad_()
    assert torch.autograd.gradcheck(lambda t: cu(t), (xc,), eps=1e-6, atol=1e-6)


def test_identity_base_gradient_matches_reference(C):
    torch.manual_seed(5)
    from torchsplinekan_amd import KANLinear
    ref = KANLinear(5, 2, base_activation=nn.Identity, backend="reference").double()
    cu = _clone_to(ref, "cuda", "cuda", base_activation=nn.Identity)
    x = torch.randn(12, 5, dtype=torch.float64) * 0.7
    for m, xx in ((ref, x), (cu, x.cuda())):
        m(xx).pow(2).sum().backward()
    cp = dict(cu.named_parameters())
    for n, p in ref.named_parameters():
        assert torch.allclose(p.grad, cp[n].grad.cpu(), atol=1e-10), n


def _away_from_knots(t, n, lo, hi):
    """n points in [lo, hi] at least 1e-3 from every knot of the row t."""
    xs = torch.linspace(lo, hi, 8 * n, dtype=torch.float64)
    d = (xs[:, None] - t[None].double()).abs().min(1).values
    return xs[d > 1e-3][::8][:n]


@pytest.mark.parametrize("backend", ["cuda", "reference"])
@pytest.mark.parametrize("uniform", [True, False])
def test_pure_spline_second_derivative_exact(C, backend, uniform):
    """A cubic spline reproduces x^3 - x exactly, so u_xx = 6x."""
    from torchsplinekan_amd import KANLinear
    from torchsplinekan_amd.reference_backend import curve2coeff
    k, G = 3, 6
    grid = make_grid(1, G, k, "uniform" if uniform else "nonuniform", seed=7)
    # interior knots span exactly [-1, 1], where the fit below is exact
    grid = -1 + 2 * (grid - grid[:, k:k + 1]) / (grid[:, k + G:k + G + 1] - grid[:, k:k + 1])
    layer = KANLinear(1, 1, grid_size=G, spline_order=k, backend=backend).double()
    layer._copy_grid_(grid.double())
    xs = torch.linspace(-1, 1, 400, dtype=torch.float64).unsqueeze(1)
    ys = (xs ** 3 - xs).t().unsqueeze(-1)
    with torch.no_grad():
        layer.base_weight.zero_()
        layer.spline_scaler.fill_(1.0)
        layer.spline_weight.copy_(curve2coeff(xs, ys, layer.grid, k))
    layer = layer.cuda()
    x = _away_from_knots(layer.grid[0].cpu(), 9, -0.95, 0.95).cuda().unsqueeze(1).requires_grad_()
    u = layer(x)
    ux = torch.autograd.grad(u.sum(), x, create_graph=True)[0]
    uxx = torch.autograd.grad(ux.sum(), x, create_graph=True)[0]
    assert layer.last_backend == backend
    assert torch.allclose(u, x ** 3 - x, atol=1e-9)
    assert torch.allclose(ux, 3 * x ** 2 - 1, atol=1e-8)
    assert torch.allclose(uxx, 6 * x, atol=1e-7)


@pytest.mark.parametrize("k", [1, 2, 3])
def test_native_matches_reference_on_nonuniform_grids(C, k):
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(10 + k)
    G = 7
    ref = KANLinear(3, 4, grid_size=G, spline_order=k, backend="reference").double()
    ref._copy_grid_(make_grid(3, G, k, "nonuniform", seed=20 + k).double())
    cu = _clone_to(ref, "cuda", "cuda")
    x = torch.stack([_away_from_knots(ref.grid[i], 30, -1.3, 1.3) for i in range(3)], 1)
    xr, xc = x.clone().requires_grad_(), x.cuda().requires_grad_()
    yr, yc = ref(xr), cu(xc)
    assert torch.allclose(yr, yc.cpu(), atol=1e-12)
    w = torch.randn_like(yr)
    yr.backward(w)
    yc.backward(w.cuda())
    assert torch.allclose(xr.grad, xc.grad.cpu(), atol=1e-10)
    cp = dict(cu.named_parameters())
    for n, p in ref.named_parameters():
        assert torch.allclose(p.grad, cp[n].grad.cpu(), atol=1e-10), n


def test_kernel_limits_and_fallback(C):
    from torchsplinekan_amd import KANLinear
    k = 3
    G = C.CUDA_MAX_DEG0_BASIS - 2 * k                       # exactly at the limit
    torch.manual_seed(11)
    ref = KANLinear(2, 2, grid_size=G, spline_order=k, backend="reference")
    cu = _clone_to(ref, "cuda", "cuda")
    x = torch.rand(64, 2) * 2 - 1
    assert torch.allclose(ref(x), cu(x.cuda()).cpu(), atol=1e-5)
    with pytest.raises(ValueError, match="CUDA kernel limit"):
        KANLinear(2, 2, grid_size=G + 1, spline_order=3, backend="cuda")
    big = KANLinear(2, 2, grid_size=200, backend="reference")
    auto = _clone_to(big, "auto", "cuda")
    assert auto.selected_backend == "reference"
    xx = torch.rand(32, 2) * 2 - 1
    assert torch.allclose(big(xx), auto(xx.cuda()).cpu(), atol=1e-5)
    assert auto.last_backend == "reference"
    # raw ops validate before launching
    Gr = 100
    xd = torch.rand(8, 2, device="cuda")
    grid = torch.linspace(-2, 2, Gr + 2 * k + 1, device="cuda").expand(2, -1).contiguous()
    args = (torch.zeros(2, 2, device="cuda"), torch.zeros(2, 2, Gr + k, device="cuda"),
            torch.ones(2, 2, device="cuda"), k, True)
    with pytest.raises(RuntimeError, match="G \\+ 2k"):
        C.kan_forward(xd, grid, *args)
    with pytest.raises(RuntimeError, match="G \\+ 2k"):
        C.kan_apply(xd, grid, *args)
    grid12 = torch.linspace(-2, 2, 12, device="cuda").expand(2, -1).contiguous()
    with pytest.raises(RuntimeError, match="spline_weight.size\\(2\\)"):
        C.kan_forward(xd, grid12, torch.zeros(2, 2, device="cuda"),
                      torch.zeros(2, 2, 7, device="cuda"), torch.ones(2, 2, device="cuda"), 3, True)
    torch.cuda.synchronize()


def _trained_like(model):
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        for p in model.parameters():
            p.add_(torch.randn(p.shape, generator=g, dtype=p.dtype).to(p.device) * 0.3)
    return model


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_export_preserves_function_grid_and_config(C, dtype):
    from torchsplinekan_amd import KAN
    torch.manual_seed(1)
    m = _trained_like(KAN([5, 7, 3], grid_size=6, base_activation=nn.Tanh).to("cuda", dtype))
    m.update_grid(torch.randn(200, 5, device="cuda", dtype=dtype) ** 3)
    sd_before = {k: v.clone() for k, v in m.state_dict().items()}
    e = m.export_inference()
    x = torch.randn(64, 5, device="cuda", dtype=dtype) * 1.5
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    with torch.no_grad():
        ye = e(x)
    assert torch.allclose(m(x), ye, atol=tol, rtol=tol)
    assert all(l.last_backend == "cuda" for l in e.layers)
    for k, v in m.state_dict().items():
        assert torch.equal(v, sd_before[k]), k
    for lo, le in zip(m.layers, e.layers):
        assert not hasattr(le, "spline_scaler") and le.enable_standalone_scale_spline is False
        assert torch.equal(lo.grid, le.grid)
        assert isinstance(le._ref.base_activation, nn.Tanh)
        assert le.backend == lo.backend
    assert not e.training and not any(p.requires_grad for p in e.parameters())


def test_export_save_load_roundtrip(C):
    from torchsplinekan_amd import KAN
    torch.manual_seed(2)
    m = _trained_like(KAN([4, 6, 2], grid_size=5).cuda())
    m.update_grid(torch.rand(100, 4, device="cuda") * 3 - 1)
    e = m.export_inference()
    buf = io.BytesIO()
    torch.save(e.state_dict(), buf)
    buf.seek(0)
    sd = torch.load(buf, map_location="cuda", weights_only=True)
    assert not any("spline_scaler" in k for k in sd)
    fresh = KAN([4, 6, 2], grid_size=5, enable_standalone_scale_spline=False).cuda()
    fresh.load_state_dict(sd)
    x = torch.randn(33, 4, device="cuda")
    assert torch.allclose(fresh(x), m(x), atol=1e-5)
    with pytest.raises(RuntimeError):
        KAN([4, 6, 2], grid_size=5).cuda().load_state_dict(sd)


def test_export_requires_grad_option_finetunes(C):
    from torchsplinekan_amd import KANLinear
    m = KANLinear(3, 2).cuda()
    e = m.export_inference(requires_grad=True)
    e(torch.randn(4, 3, device="cuda")).sum().backward()
    assert e.spline_weight.grad is not None and m.spline_weight.grad is None


def test_grid_extension_on_device(C):
    """tests/test_grid_extension.py of the reference on device tensors: the
    multilayer extension fits each layer on the inputs it actually sees,
    undersampled and constant-input fits stay finite, and the extended
    model trains with a fresh optimiser."""
    from torchsplinekan_amd import KAN
    torch.manual_seed(3)
    m = KAN([3, 5, 2], grid_size=4, backend="cuda").double().cuda()
    x = torch.rand(300, 3, dtype=torch.float64, device="cuda") * 2 - 1
    fine = m.extend_grid(8, x)
    assert all(l.grid_size == 8 for l in fine.layers)
    # nested uniform refinement (4 -> 8 keeps the old knots): the function is kept
    assert torch.allclose(fine(x), m(x), atol=1e-8)
    # each layer's refit used the hidden activations of the refined network's input
    h = m.layers[0](x)
    lo, hi = fine.layers[1].grid[:, 3], fine.layers[1].grid[:, 3 + 8]
    assert (lo <= h.amin(0) + 1e-9).all() or (hi >= h.amax(0) - 1e-9).all()
    # undersampled fit (fewer samples than coefficients) stays finite and bounded
    few = KAN([2, 2], grid_size=3, backend="cuda").double().cuda()
    xf = torch.rand(4, 2, dtype=torch.float64, device="cuda") * 2 - 1
    big = few.extend_grid(20, xf)
    assert all(torch.isfinite(p).all() for p in big.parameters())
    assert big(xf).abs().max() < 1e3
    # constant input: rank-deficient per-feature fit, still finite
    xc = torch.full((50, 2), 0.3, dtype=torch.float64, device="cuda")
    const = few.extend_grid(6, xc)
    assert all(torch.isfinite(p).all() for p in const.parameters())
    assert torch.allclose(const(xc), few(xc), atol=1e-6)
    # the extended model trains with a new optimiser
    opt = torch.optim.Adam(fine.parameters(), lr=1e-2)
    tgt = torch.randn(300, 2, dtype=torch.float64, device="cuda")
    losses = []
    for _ in range(5):
        opt.zero_grad()
        loss = ((fine(x) - tgt) ** 2).mean()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0]
