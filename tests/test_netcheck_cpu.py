"""CPU check of the workload checker's full-layer mode (tests/_netcheck.py,
check_layers(full=True), which the c4 GPU tests use): a float64 regularised
KAN stepped on the CPU through the reference backend passes at 1e-12 with
float64's unit roundoff, and a fault of 1e-6 of a gradient's largest entry,
planted in one entry of one layer's dcoef, dscaler, dbase_w or input
gradient, fails it."""

import pytest
import torch
import torch.nn.functional as F

from tests import _netcheck

U64 = 2.0 ** -53


def _step(seed):
    from torchsplinekan_amd import KAN
    torch.manual_seed(seed)
    net = KAN([5, 7, 3], grid_size=5, backend="reference").double()
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(300, 5, generator=g, dtype=torch.float64) * 2.2 - 1.1).requires_grad_()
    t = torch.randn(300, 3, generator=g, dtype=torch.float64)
    with _netcheck.capture(net) as cap:
        y, reg = net.forward_with_regularization(x, 1e-2, 1e-2, reg_impl="auto")
        (F.mse_loss(y, t) + reg).backward()
    return net, cap, reg


def _check(net, cap):
    return _netcheck.check_layers(net, cap, 1e-2, 3, 1e-12, say=lambda m: None, unit=U64,
                                  full=True)


def test_full_mode_passes_a_correct_step():
    net, cap, reg = _step(0)
    total = _check(net, cap)
    assert abs(reg.item() - total) / abs(total) < 1e-12


@pytest.mark.parametrize("where", ["spline_weight", "spline_scaler", "base_weight", "x"])
def test_full_mode_fails_a_planted_fault(where):
    net, cap, _ = _step(1)
    with torch.no_grad():
        if where == "x":
            gr = cap[1][0].grad            # layer 1's input gradient
            gr[123, 4] += 1e-6 * gr.abs().max()
        else:
            gr = getattr(net.layers[1], where).grad
            idx = (2, 3, 1) if where == "spline_weight" else (2, 3)
            gr[idx] += 1e-6 * gr.abs().max()
    with pytest.raises(AssertionError):
        _check(net, cap)
