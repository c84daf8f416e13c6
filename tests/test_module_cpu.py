"""CPU tests of the module layer (KANLinear / KAN API, backend selection,
state_dict keys, error behaviour, reference backend and the CPU dispatch of
the raw ops) against the oracle.  Mirrors tests/test_reference.py and the
CPU parts of tests/test_cuda.py, tests/test_math_correctness.py:313-360 and
tests/test_fused_regularization.py of the reference."""

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import kan_oracle as ko
from tests._util import normwise, np64
from torchsplinekan_amd import KAN, KANLinear, _C
from torchsplinekan_amd import kan_linear as kl
from torchsplinekan_amd.reference_backend import compute_basis, compute_basis_derivative


def test_package_surface():
    for name in ("kan_forward", "kan_backward", "kan_apply", "set_basis_impl", "get_basis_impl",
                 "basis", "basis_grad", "edge_abs_mean", "edge_abs_mean_backward"):
        assert callable(getattr(_C, name)), name
    assert kl.CUDA_MAX_DEG0_BASIS == 71 and kl.CUDA_MAX_IN_FEATURES == 65535
    assert kl.native_config_supported(16, 65, 3) == (True, "")
    ok, reason = kl.native_config_supported(16, 66, 3)
    assert not ok and "72" in reason
    ok, reason = kl.native_config_supported(65536, 5, 3)
    assert not ok and "in_features" in reason


def test_reference_forward_matches_oracle_fp64():
    torch.manual_seed(0)
    L = KANLinear(16, 8, grid_size=5, spline_order=3, backend="reference").double()
    with torch.no_grad():
        L.spline_scaler.uniform_(0.5, 1.5)
    x = (torch.rand(32, 16, dtype=torch.float64) * 2.2 - 1.1).requires_grad_()
    y = L(x)
    assert L.last_backend == "reference"
    ry, H = ko.kan_forward(np64(x), np64(L.grid), np64(L.base_weight), np64(L.spline_weight),
                           np64(L.spline_scaler), 3)
    assert normwise(np64(y), ry) < 1e-14
    D = torch.randn(32, 8, dtype=torch.float64)
    y.backward(D)
    rgx, rgbw, rgsw, rgsc = ko.kan_backward(np64(D), np64(x), np64(L.grid), np64(L.base_weight),
                                            np64(L.spline_weight), np64(L.spline_scaler), 3,
                                            basis=H)
    for got, ref in [(x.grad, rgx), (L.base_weight.grad, rgbw), (L.spline_weight.grad, rgsw),
                     (L.spline_scaler.grad, rgsc)]:
        assert normwise(np64(got), ref) < 1e-12


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_raw_ops_cpu_dispatch_match_oracle(dtype):
    g = torch.Generator().manual_seed(1)
    N, I, O, G, k = 20, 5, 3, 4, 2
    grid = torch.from_numpy(ko.uniform_grid(I, G, k)).to(dtype)
    x = (torch.rand(N, I, generator=g, dtype=torch.float64) * 2 - 1).to(dtype)
    bw = torch.randn(O, I, generator=g, dtype=torch.float64).to(dtype)
    sw = torch.randn(O, I, G + k, generator=g, dtype=torch.float64).to(dtype)
    sc = (torch.rand(O, I, generator=g, dtype=torch.float64) + 0.5).to(dtype)
    y, H = _C.kan_forward(x, grid, bw, sw, sc, k, True)
    ry, rH = ko.kan_forward(np64(x), np64(grid), np64(bw), np64(sw), np64(sc), k)
    tol = 1e-13 if dtype == torch.float64 else 1e-6
    assert normwise(np64(y), ry) < tol and normwise(np64(H), rH) < tol
    D = torch.randn(N, O, generator=g, dtype=torch.float64).to(dtype)
    out = _C.kan_backward(D, x, grid, bw, sw, sc, H, k, True)
    ref = ko.kan_backward(np64(D), np64(x), np64(grid), np64(bw), np64(sw), np64(sc), k, basis=rH)
    for a, b in zip(out, ref):
        assert normwise(np64(a), b) < (1e-12 if dtype == torch.float64 else 1e-5)
    # kan_apply with autograd on CPU
    xx = x.clone().requires_grad_()
    _C.kan_apply(xx, grid, bw, sw, sc, k, True).backward(D)
    assert normwise(np64(xx.grad), ref[0]) < (1e-12 if dtype == torch.float64 else 1e-5)


def test_raw_op_validation_messages():
    grid = torch.from_numpy(ko.uniform_grid(4, 5, 3)).float()
    x = torch.rand(3, 4)
    empty = torch.empty(0)
    with pytest.raises(RuntimeError, match=r"spline_weight.size\(2\)"):
        _C.kan_forward(x, grid, empty, torch.zeros(2, 4, 7), empty, 3, False)
    with pytest.raises(RuntimeError, match="2-D"):
        _C.kan_forward(x[None], grid, empty, torch.zeros(2, 4, 8), empty, 3, False)
    with pytest.raises(RuntimeError, match="spline_order"):
        _C.kan_forward(x, grid, empty, torch.zeros(2, 4, 8), empty, 4, False)
    with pytest.raises(RuntimeError, match="FP32 and FP64"):
        _C.kan_forward(x.half(), grid.half(), empty, torch.zeros(2, 4, 8).half(), empty, 3, False)
    with pytest.raises(RuntimeError, match="base_weight must have shape"):
        _C.kan_forward(x, grid, torch.zeros(3, 4), torch.zeros(2, 4, 8), empty, 3, False)
    with pytest.raises(RuntimeError):
        _C.set_basis_impl(7)
    assert _C.get_basis_impl() == 1


def test_backend_selection_on_cpu():
    L = KANLinear(4, 3, backend="auto")
    assert L.selected_backend == "cuda"          # device inputs would run natively
    assert L.backend_for(torch.rand(2, 4)) == "reference"
    L(torch.rand(2, 4))
    assert L.last_backend == "reference"
    Lc = KANLinear(4, 3, backend="cuda")
    with pytest.raises(RuntimeError, match="CPU tensor"):
        Lc(torch.rand(2, 4))
    with pytest.raises(ValueError, match="CUDA kernel limit"):
        KANLinear(4, 3, grid_size=66, backend="cuda")
    La = KANLinear(4, 3, grid_size=66, backend="auto")
    assert La.selected_backend == "reference"
    with pytest.raises(ValueError):
        KANLinear(4, 3, backend="triton")
    with pytest.raises(ValueError):
        KANLinear(4, 4, spline_order=0)
    with pytest.raises(ValueError):
        KANLinear(4, 4, grid_size=-1)


def test_auto_falls_back_with_warning_when_library_missing(monkeypatch):
    """backend="auto" without the native library: device inputs go to the
    reference backend as in spline_kan/kan_linear.py:147-148, with one
    RuntimeWarning per process naming the missing library."""
    import types
    from torchsplinekan_amd import kan_linear as kl
    monkeypatch.setattr(kl, "_CUDA_EXT_LOADED", False)
    monkeypatch.setattr(kl, "_MISSING_WARNED", False)
    L = KANLinear(4, 3, backend="auto")
    assert L.selected_backend == "reference"
    dev_like = types.SimpleNamespace(is_cuda=True)
    with pytest.warns(RuntimeWarning, match="libkan_hip.so is not built"):
        assert L.backend_for(dev_like) == "reference"
    import warnings
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert L.backend_for(dev_like) == "reference"   # warned once only
    with pytest.raises(RuntimeError, match="could not be loaded"):
        KANLinear(4, 3, backend="cuda")


def test_state_dict_keys_and_roundtrip():
    L = KANLinear(4, 3, grid_size=5, backend="auto")
    keys = set(L.state_dict().keys())
    assert {"base_weight", "spline_weight", "spline_scaler", "grid", "_ref.base_weight",
            "_ref.spline_weight", "_ref.spline_scaler", "_ref.grid"} == keys
    L.update_grid(torch.randn(100, 4))
    L2 = KANLinear(4, 3, grid_size=5, backend="reference")
    L2.load_state_dict(L.state_dict())
    x = torch.randn(7, 4)
    assert torch.allclose(L(x), L2(x))
    assert torch.equal(L.grid, L._ref.grid)


def test_shapes_leading_dims_noncontiguous():
    L = KANLinear(8, 4, backend="reference")
    assert L(torch.randn(3, 5, 8)).shape == (3, 5, 4)
    x = torch.randn(10, 16)[:, ::2]
    assert not x.is_contiguous() and L(x).shape == (10, 4)
    assert KAN([16, 32, 8])(torch.randn(10, 16)).shape == (10, 8)
    with pytest.raises(ValueError):
        KAN([4])


def test_non_silu_activation_reference_matches_oracle_path():
    torch.manual_seed(3)
    L = KANLinear(5, 2, base_activation=nn.Tanh, backend="reference").double()
    x = torch.rand(9, 5, dtype=torch.float64) * 2 - 1
    H = ko.basis_dense(np64(x), np64(L.grid), 3)
    W = np64(L.spline_weight) * np64(L.spline_scaler)[:, :, None]
    ref = np.tanh(np64(x)) @ np64(L.base_weight).T + H.reshape(9, -1) @ W.reshape(2, -1).T
    assert normwise(np64(L(x)), ref) < 1e-14


@pytest.mark.parametrize("impl", ["dense", "checkpoint"])
def test_regularization_matches_oracle(impl):
    torch.manual_seed(4)
    L = KANLinear(6, 5, grid_size=4, backend="reference").double()
    x = torch.rand(40, 6, dtype=torch.float64) * 2.4 - 1.2
    y, r = L.forward_with_regularization(x, 0.3, 0.7, reg_impl=impl, chunk_size=16)
    assert L.last_backend == "reference"
    s = ko.silu(np64(x))
    H = ko.basis_dense(np64(x), np64(L.grid), 3)
    W = np64(L.spline_weight) * np64(L.spline_scaler)[:, :, None]
    a = ko.edge_abs_mean(s, H, np64(L.base_weight), W)
    assert abs(float(r) - ko.regularization_from_edge_means(a, 0.3, 0.7)) < 1e-12
    assert normwise(np64(L.edge_l1(x)), a) < 1e-13
    r.backward()
    # d reg / d base_weight through the chain rule of the oracle
    ga = ko.regularization_grad(a, 0.3, 0.7)
    _, _, dbw, dW = ko.edge_abs_mean_backward(ga, s, H, np64(L.base_weight), W)
    assert normwise(np64(L.base_weight.grad), dbw) < 1e-10
    assert normwise(np64(L.spline_weight.grad), dW * np64(L.spline_scaler)[:, :, None]) < 1e-10


def test_regularization_options_validation():
    L = KANLinear(3, 2, backend="reference")
    x = torch.rand(5, 3)
    with pytest.raises(ValueError):
        L.forward_with_regularization(x, reg_impl="bogus")
    with pytest.raises(RuntimeError):
        L.forward_with_regularization(x, reg_impl="fused")     # CPU tensor
    with pytest.raises(ValueError):
        L.forward_with_regularization(x, reg_impl="checkpoint", chunk_size=0)
    with pytest.raises(ValueError):
        L.regularization_loss(mode="bogus")
    with pytest.raises(ValueError):
        L._ref.regularization_loss(1.0, 1.0, x=None)
    r = L.regularization_loss(mode="coefficient")
    assert torch.isfinite(r)


def test_zero_layer_regulariser_is_finite():
    L = KANLinear(4, 4, backend="reference")
    with torch.no_grad():
        L.spline_weight.zero_()
        L.base_weight.zero_()
    x = torch.randn(20, 4)
    r = L.regularization_loss(x=x)
    assert abs(float(r)) < 1e-30
    r.backward()
    assert torch.isfinite(L.spline_weight.grad).all()


def test_composite_double_backward_cpu():
    L = KANLinear(3, 2, grid_size=3, backend="reference").double()
    x = (torch.randn(4, 3, dtype=torch.float64) * 0.4).requires_grad_()
    assert torch.autograd.gradcheck(L, (x,), eps=1e-6, atol=1e-4, rtol=1e-3)
    assert torch.autograd.gradgradcheck(L, (x,), eps=1e-6, atol=1e-3)
    # the raw autograd op on CPU: create_graph path
    grid, bw, sw, sc = L.grid, L.base_weight, L.spline_weight, L.spline_scaler

    def f(t):
        return _C.kan_apply(t, grid, bw, sw, sc, 3, True)

    assert torch.autograd.gradgradcheck(f, (x,), eps=1e-6, atol=1e-3)


def test_update_grid_behaviour():
    L = KANLinear(4, 4, backend="reference")
    with torch.no_grad():
        L.spline_scaler.fill_(2.0)
    before = L.spline_scaler.clone()
    L.update_grid(torch.randn(100, 4))
    assert torch.allclose(L.spline_scaler, before)
    assert not torch.isnan(L.spline_weight).any()
    with pytest.raises((ValueError, RuntimeError)):
        L.update_grid(torch.randn(0, 4))
    L.update_grid(torch.randn(10, 5, 4))


def test_basis_helpers_match_oracle():
    grid = torch.from_numpy(ko.uniform_grid(3, 7, 2))
    x = torch.rand(50, 3, dtype=torch.float64) * 2.6 - 1.3
    assert normwise(np64(compute_basis(x, grid, 2)), ko.basis_dense(np64(x), np64(grid), 2)) < 1e-15
    assert normwise(np64(compute_basis_derivative(x, grid, 2)),
                    ko.basis_derivative(np64(x), np64(grid), 2)) < 1e-14
    with pytest.raises(ValueError):
        compute_basis(x, grid, 4)


def test_select_keeps_the_chosen_edges():
    """KANLinear.select: all indices reproduce the layer; a subset of outputs
    and inputs equals the full layer evaluated with the dropped inputs'
    edges removed, restricted to the kept outputs."""
    torch.manual_seed(3)
    L = KANLinear(6, 5, grid_size=4, backend="reference").double()
    with torch.no_grad():
        L.spline_scaler.uniform_(0.5, 1.5)
        L.grid.add_(torch.linspace(0, 0.1, 6, dtype=torch.float64)[:, None])
        L._ref.grid.copy_(L.grid)
    x = torch.rand(40, 6, dtype=torch.float64) * 2 - 1
    full = L.select()
    assert torch.equal(full(x), L(x))
    oi, ii = torch.tensor([4, 1]), torch.tensor([0, 3, 5])
    sub = L.select(oi, ii)
    assert (sub.in_features, sub.out_features) == (3, 2)
    assert torch.equal(sub.grid, L.grid[ii]) and torch.equal(sub._ref.grid, L.grid[ii])
    masked = L.make_like()
    masked.load_state_dict(L.state_dict())
    drop = [i for i in range(6) if i not in ii.tolist()]
    with torch.no_grad():
        masked.base_weight[:, drop] = 0
        masked.spline_weight[:, drop] = 0
    assert torch.allclose(sub(x[:, ii]), masked(x)[:, oi], atol=1e-13)
    L.requires_grad_(False)
    assert not any(p.requires_grad for p in L.select(oi, ii).parameters())


def test_select_index_arguments():
    """select takes boolean masks as masks (not as 0/1 indices) and rejects
    out-of-range indices, masks of the wrong length and float indices."""
    torch.manual_seed(5)
    L = KANLinear(4, 3, grid_size=3, backend="reference").double()
    x = torch.rand(10, 4, dtype=torch.float64) * 2 - 1
    by_mask = L.select(torch.tensor([False, True, True]), torch.tensor([True, False, True, True]))
    by_index = L.select(torch.tensor([1, 2]), torch.tensor([0, 2, 3]))
    assert (by_mask.out_features, by_mask.in_features) == (2, 3)
    assert torch.equal(by_mask(x[:, [0, 2, 3]]), by_index(x[:, [0, 2, 3]]))
    assert L.select([True, False, True]).out_features == 2
    with pytest.raises(IndexError):
        L.select(torch.tensor([0, 3]))
    with pytest.raises(IndexError):
        L.select(None, [-1])
    with pytest.raises(ValueError):
        L.select(torch.tensor([True, False]))
    with pytest.raises(TypeError):
        L.select(torch.tensor([0.0, 1.0]))


@pytest.mark.parametrize("with_base", [True, False])
def test_chunked_edge_statistic_gradients(with_base):
    """reg_impl="checkpoint" statistic: value, all four first derivatives and
    second derivatives (gradgradcheck) against the dense phi formulation."""
    from torchsplinekan_amd.fused import edge_abs_mean_chunked
    from torchsplinekan_amd.reference_backend import compute_basis, edge_abs_mean_dense
    g = torch.Generator().manual_seed(11)
    N, I, O, G, k = 23, 3, 4, 4, 3
    x = (torch.rand(N, I, generator=g, dtype=torch.float64) * 2.6 - 1.3).requires_grad_()
    grid = torch.linspace(-1, 1, G + 1, dtype=torch.float64)
    h = grid[1] - grid[0]
    grid = torch.cat([grid[0] - h * torch.arange(k, 0, -1), grid,
                      grid[-1] + h * torch.arange(1, k + 1)]).repeat(I, 1)
    W = torch.randn(O, I, G + k, generator=g, dtype=torch.float64).requires_grad_()
    bw = torch.randn(O, I, generator=g, dtype=torch.float64).requires_grad_() if with_base else None
    s = torch.nn.functional.silu(x) if with_base else None

    def chunked(x_, W_, bw_):
        s_ = torch.nn.functional.silu(x_) if with_base else None
        return edge_abs_mean_chunked(s_, x_, grid, k, bw_, W_, 5)

    def dense(x_, W_, bw_):
        s_ = torch.nn.functional.silu(x_) if with_base else None
        return edge_abs_mean_dense(s_, compute_basis(x_, grid, k), bw_, W_)

    args = (x, W, bw) if with_base else (x, W)
    f_c = (lambda a, b, c: chunked(a, b, c)) if with_base else (lambda a, b: chunked(a, b, None))
    f_d = (lambda a, b, c: dense(a, b, c)) if with_base else (lambda a, b: dense(a, b, None))
    a_c, a_d = f_c(*args), f_d(*args)
    assert normwise(np64(a_c), np64(a_d)) < 1e-14
    ga = torch.randn(O, I, generator=g, dtype=torch.float64)
    gc = torch.autograd.grad(a_c, args, ga)
    gd = torch.autograd.grad(a_d, args, ga)
    for u, v in zip(gc, gd):
        assert normwise(np64(u), np64(v)) < 1e-12
    assert torch.autograd.gradgradcheck(f_c, args, (ga,))
