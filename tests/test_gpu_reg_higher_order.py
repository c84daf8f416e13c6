"""GPU parity of the native recorded backward of the edge statistic
(EdgeAbsMeanBackward and kan_hip_edge_abs_mean_double_backward): second
derivatives of the activation regulariser, mixed input x weight terms
included, on the device kernels at the fixed sign pattern.

Checked against (a) the dense differentiable formulas of the reference's
recorded path (spline_kan/fused.py:80-95), restated in float64 torch ops
on the same operands; (b) the reference's own tests of this path
(tests/test_fused_regularization.py:99-150): the closed-form mixed
derivative 0.5, gradcheck / gradgradcheck, and the joint Hessian-vector
product of fused against dense.  Tolerances: fp64 1e-12 normwise against
the dense formulas, the reference's rtol 1e-9 / atol 1e-10 for the joint
Hessian; fp32 1e-5 normwise.
"""

import pytest
import torch

from tests._util import normwise, np64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from torchsplinekan_amd import _C
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return _C


def _dense_double_backward(ga, s, H, bw, W, u):
    """Gradients of <u, (ds, dH, dbw, dW)> by autograd through the dense
    first-order formulas (sign pattern constant), in float64 on the CPU."""
    d = lambda t: None if t is None else t.detach().double().cpu().requires_grad_()
    ga, s, H, bw, W = d(ga), d(s), d(H), d(bw), d(W)
    n = H.shape[0]
    phi = torch.einsum("oir,nir->noi", W, H)
    if bw is not None:
        phi = s.unsqueeze(1) * bw.unsqueeze(0) + phi
    g = phi.sign().detach() * ga.unsqueeze(0) / n
    outs = [(g * bw.unsqueeze(0)).sum(1) if bw is not None else None,
            torch.einsum("noi,oir->nir", g, W),
            (g * s.unsqueeze(1)).sum(0) if bw is not None else None,
            torch.einsum("noi,nir->oir", g, H)]
    terms = [(o * uu.double().cpu()).sum() for o, uu in zip(outs, u)
             if o is not None and uu is not None]
    if not terms:
        return [None] * 5
    total = sum(terms)
    ins = [t for t in (ga, s, H, bw, W) if t is not None]
    grads = torch.autograd.grad(total, ins, allow_unused=True)
    it = iter(grads)
    return [next(it) if t is not None else None for t in (ga, s, H, bw, W)]


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 1e-5)])
@pytest.mark.parametrize("base", [True, False])
@pytest.mark.parametrize("n,I,O,R", [(37, 3, 5, 8), (5000, 4, 6, 13), (300, 9, 70, 4)])
def test_double_backward_matches_dense(C, dtype, tol, base, n, I, O, R):
    print(f"edge double backward n={n} I={I} O={O} R={R} base={base} {dtype}", flush=True)
    g = torch.Generator().manual_seed(n + O)
    mk = lambda *shape: torch.randn(*shape, generator=g, dtype=torch.float64).to(dtype).cuda()
    s, H, bw, W = mk(n, I), mk(n, I, R), mk(O, I), mk(O, I, R)
    ga = mk(O, I)
    if not base:
        s = bw = None
    u_full = [mk(n, I) if base else None, mk(n, I, R), mk(O, I) if base else None, mk(O, I, R)]
    for keep in ((0, 1, 2, 3), (1, 3), (0, 2), (2,), (1,)):
        u = [u_full[j] if j in keep else None for j in range(4)]
        got = C.edge_abs_mean_double_backward(ga, s, H, bw, W, *u, True, True, True, True, True)
        ref = _dense_double_backward(ga, s, H, bw, W, u)
        for name, a, b in zip(("ga", "s", "H", "bw", "W"), got, ref):
            if b is None or not b.abs().max() > 0:
                assert a is None or not a.abs().max() > 0, (keep, name)
                continue
            assert normwise(np64(a), np64(b)) < tol, (keep, name)


@pytest.mark.parametrize("has_base", [True, False])
def test_edge_stat_mixed_second_derivatives(C, has_base):
    """tests/test_fused_regularization.py:110-130 of the reference."""
    from torchsplinekan_amd import fused as fz
    opts = dict(device="cuda", dtype=torch.float64, requires_grad=True)
    H = torch.tensor([[[0.3, 0.7]], [[0.6, 0.4]]], **opts)
    W = torch.tensor([[[0.5, 0.9]]], **opts)
    if has_base:
        s = torch.tensor([[0.2], [0.4]], **opts)
        bw = torch.tensor([[0.8]], **opts)
        fn, inputs = fz.edge_abs_mean, (s, H, bw, W)
        a = fn(*inputs)
        dbw = torch.autograd.grad(a.sum(), bw, create_graph=True)[0]
        mixed = torch.autograd.grad(dbw.sum(), s)[0]
        assert torch.allclose(mixed, torch.full_like(s, 0.5))
    else:
        fn = lambda h, w: fz.edge_abs_mean(None, h, None, w)
        inputs = (H, W)
    assert torch.autograd.gradcheck(fn, inputs, eps=1e-6, atol=1e-6)
    assert torch.autograd.gradgradcheck(fn, inputs, eps=1e-6, atol=1e-6)


def test_second_order_runs_the_native_double_backward(C, monkeypatch):
    from torchsplinekan_amd import _C, fused as fz

    def boom(*a, **k):
        raise AssertionError("dense double backward used at second order")

    monkeypatch.setattr(_C, "_edge_double_backward_dense", boom)
    g = torch.Generator().manual_seed(0)
    mk = lambda *shape: torch.randn(*shape, generator=g, dtype=torch.float64).cuda().requires_grad_()
    s, H, bw, W = mk(40, 3), mk(40, 3, 6), mk(4, 3), mk(4, 3, 6)
    a = fz.edge_abs_mean(s, H, bw, W)
    grads = torch.autograd.grad(a.square().sum(), (s, H, bw, W), create_graph=True)
    hv = torch.autograd.grad(sum(t.sum() for t in grads), (s, H, bw, W))
    assert all(torch.isfinite(t).all() for t in hv)


def test_forward_with_regularization_fused_gradgradcheck(C):
    """tests/test_fused_regularization.py:95-107 of the reference."""
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(5)
    m = KANLinear(3, 2, grid_size=4, backend="cuda").double().cuda()
    x = (torch.rand(11, 3, dtype=torch.float64) * 1.8 - 0.9).cuda().requires_grad_()

    def f(t):
        y, r = m.forward_with_regularization(t, 0.5, 2.0, reg_impl="fused")
        return y.sum() + r

    assert torch.autograd.gradcheck(f, (x,), eps=1e-6, atol=1e-6)
    assert torch.autograd.gradgradcheck(f, (x,), eps=1e-6, atol=1e-5)


@pytest.mark.parametrize("scaler", [True, False])
def test_fused_multilayer_joint_hessian_matches_dense(C, scaler):
    """tests/test_fused_regularization.py:133-150 of the reference."""
    from torchsplinekan_amd import KAN
    torch.manual_seed(87)
    model = KAN([2, 3, 2], grid_size=4, backend="cuda",
                enable_standalone_scale_spline=scaler).double().cuda()
    x = torch.tensor([[0.19, -0.33], [0.71, 0.13]], device="cuda", dtype=torch.float64,
                     requires_grad=True)
    inputs = (x,) + tuple(model.parameters())
    directions = tuple(torch.randn_like(t) for t in inputs)
    hessians = []
    for impl in ("dense", "fused"):
        y, reg = model.forward_with_regularization(x, 0.7, 0.3, reg_impl=impl)
        grads = torch.autograd.grad(y.square().sum() + reg, inputs, create_graph=True)
        tangent = sum((g * v).sum() for g, v in zip(grads, directions))
        hessians.append(torch.autograd.grad(tangent, inputs))
    for dense, fused in zip(*hessians):
        assert torch.allclose(dense, fused, rtol=1e-9, atol=1e-10)
