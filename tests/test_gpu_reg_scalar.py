"""GPU parity of the native layer regulariser (kan_hip_edge_reg,
fused.EdgeRegularization): reg = mu1 * sum(a) + mu2 * entropy(a / sum(a)) of
one layer's edge means, against the fp64 oracle (oracle/kan_oracle.py,
regularization_from_edge_means, which follows
spline_kan/reference_backend.py:149-170), and its gradient and recorded
second derivative against autograd through the tensor expression of the
same formula (reference_backend.regularization_from_edge_means) in float64.
Covers one and many reduction blocks, zeros (the p clamp), an all-zero
layer (the total clamp) and run-to-run determinism.
"""

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko

pytestmark = pytest.mark.gpu

MU1, MU2 = 0.7, 0.3


@pytest.fixture(scope="module")
def fz():
    from torchsplinekan_amd import fused
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return fused


def _means(n, seed, zeros=0.0):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand(n, generator=g, dtype=torch.float64) ** 3  # spread over decades
    if zeros:
        a[torch.rand(n, generator=g) < zeros] = 0.0
    return a


def _tensor_expr(a, mu1=MU1, mu2=MU2):
    from torchsplinekan_amd.reference_backend import regularization_from_edge_means
    return regularization_from_edge_means(a, mu1, mu2)


@pytest.mark.parametrize("n", [1, 7, 1000, 64 * 512, 512 * 512, 1_000_003])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_value_matches_oracle(fz, n, dtype):
    print(f"edge regulariser n={n} {dtype}", flush=True)
    a = _means(n, seed=n, zeros=0.1)
    reg = fz.edge_regularization(a.to(dtype).cuda(), MU1, MU2)
    ref = ko.regularization_from_edge_means(a.to(dtype).double().numpy(), MU1, MU2)
    tol = 1e-6 if dtype == torch.float32 else 1e-13
    assert abs(float(reg) - ref) <= tol * abs(ref)


@pytest.mark.parametrize("n,zeros", [(1000, 0.0), (512 * 512, 0.2), (5, 0.6)])
def test_gradient_matches_autograd(fz, n, zeros):
    """float64: native backward against autograd through the tensor
    expression; float32: the same at the fp32 bar."""
    a = _means(n, seed=3 * n, zeros=zeros)
    for dtype, tol in ((torch.float64, 1e-12), (torch.float32, 1e-5)):
        ad = a.to(dtype).cuda().requires_grad_()
        (2.5 * fz.edge_regularization(ad, MU1, MU2)).backward()
        ar = a.double().cuda().requires_grad_()
        (2.5 * _tensor_expr(ar)).backward()
        err = (ad.grad.double() - ar.grad).abs().max() / ar.grad.abs().max()
        assert err <= tol, (dtype, float(err))


def test_all_zero_layer(fz):
    """T = 0: the total clamps to tiny, every p to tiny; value and gradient
    as through the tensor expression (finite)."""
    for dtype in (torch.float32, torch.float64):
        a = torch.zeros(300, dtype=dtype, device="cuda", requires_grad=True)
        reg = fz.edge_regularization(a, MU1, MU2)
        reg.backward()
        b = torch.zeros(300, dtype=dtype, device="cuda", requires_grad=True)
        ref = _tensor_expr(b)
        ref.backward()
        assert torch.isfinite(reg) and torch.isfinite(a.grad).all()
        assert float(reg) == pytest.approx(float(ref), rel=1e-6, abs=0.0)
        assert torch.allclose(a.grad, b.grad, rtol=1e-6, atol=0.0)


def test_deterministic(fz):
    a = _means(700_001, seed=11).float().cuda().requires_grad_()
    r1 = fz.edge_regularization(a, MU1, MU2)
    g1, = torch.autograd.grad(r1, a)
    r2 = fz.edge_regularization(a, MU1, MU2)
    g2, = torch.autograd.grad(r2, a)
    assert torch.equal(r1, r2) and torch.equal(g1, g2)


def test_recorded_backward(fz):
    """create_graph: the gradient as differentiable operations, so second
    derivatives match those through the tensor expression."""
    a = _means(2000, seed=5, zeros=0.1).cuda()
    v = torch.randn(2000, dtype=torch.float64, generator=torch.Generator().manual_seed(1)).cuda()

    def hvp(f):
        x = a.clone().requires_grad_()
        g, = torch.autograd.grad(f(x), x, create_graph=True)
        h, = torch.autograd.grad((g * v).sum(), x)
        return g.detach(), h

    g1, h1 = hvp(lambda x: fz.edge_regularization(x, MU1, MU2))
    g2, h2 = hvp(_tensor_expr)
    assert torch.allclose(g1, g2, rtol=1e-12, atol=0.0)
    assert (h1 - h2).abs().max() <= 1e-10 * h2.abs().max()
