"""The whole-tensor checker of the full-size workload tests
(tests/_fullcheck.py), on the CPU: it passes a correct step (the reference
backend in float64) at a tight bar, and a fault planted in one block of one
gradient -- small enough to vanish in the whole-tensor norm -- fails its
blockwise bar."""

import numpy as np
import torch
import torch.nn.functional as F

from oracle import kan_oracle as ko
from tests import _fullcheck
from tests._util import np64
from torchsplinekan_amd import KANLinear


def test_block_error_finds_one_bad_tile():
    rng = np.random.default_rng(0)
    ref = rng.standard_normal((1024, 768))
    got = ref * (1 + 1e-8 * rng.standard_normal(ref.shape))
    worst, _, whole = _fullcheck.block_error(got, ref, 256, 256)
    assert worst < 1e-7 and whole < 1e-7
    got[512:768, 256:512] *= 1 + 3e-5          # one tile of 12, off by 3e-5
    worst, block, whole = _fullcheck.block_error(got, ref, 256, 256)
    assert whole < 1e-5 < worst and block == (512, 256)


def test_block_error_ragged_and_zero_blocks():
    ref = np.zeros((300, 70))
    ref[:256] = 1.0
    got = ref.copy()
    worst, _, _ = _fullcheck.block_error(got, ref, 256, 64)
    assert worst == 0.0
    got[290, 69] = 1e-3                           # in a ragged block of zeros
    worst, block, _ = _fullcheck.block_error(got, ref, 256, 64)
    assert worst > 1e-5 and block == (256, 64)


def _step(seed):
    torch.manual_seed(seed)
    L = KANLinear(40, 24, grid_size=6, backend="reference").double()
    with torch.no_grad():
        L.spline_scaler.uniform_(0.5, 1.5)
    x = (torch.rand(600, 40, dtype=torch.float64) * 2.4 - 1.2).float()
    xd = x.double().requires_grad_()
    t = torch.randn(600, 24, dtype=torch.float64)
    y = L(xd)
    F.mse_loss(y, t).backward()
    D = 2.0 * (np64(y) - np64(t)) / y.numel()
    return L, x, y.detach(), xd.grad, D


def test_check_layer_step_passes_and_catches():
    L, x, y, gx, D = _step(1)
    errs = _fullcheck.check_layer_step(L, x, y, gx, D, 3, lambda m: None, chunk=256)
    assert set(errs) == {"y", "dx", "dcoef", "dscaler", "dbase_w"}
    for name, (worst, _, _) in errs.items():
        assert worst < 1e-12, name
    with torch.no_grad():
        L.spline_weight.grad[16:24, 8:12] *= 1 + 1e-4   # one edge block of dcoef
    errs = _fullcheck.check_layer_step(L, x, y, gx, D, 3, lambda m: None, chunk=256)
    assert errs["dcoef"][0] > 1e-5
    assert errs["y"][0] < 1e-12 and errs["dbase_w"][0] < 1e-12


def test_edge_full_check_equals_the_oracle_and_finds_a_planted_fault():
    """check_edge_full (per feature, blockwise, slack taken off) reports
    errors at rounding level for the oracle's own statistic and backward,
    fed back as the device results, and fails a fault of 1e-4 of the
    largest entry planted in one entry of dH, ds, dW, dbw or a."""
    r = np.random.default_rng(3)
    N, I, O, G, k = 600, 7, 70, 6, 3
    x = r.uniform(-1.1, 1.1, size=(N, I))
    grid = ko.uniform_grid(I, G, k)
    W = r.normal(0, 0.2, size=(O, I, G + k))
    bw = r.normal(0, 0.3, size=(O, I))
    ga = r.normal(size=(O, I))
    H = ko.basis_dense(x, grid, k)
    s = ko.silu(x)
    ds, dH, dbw, dW = ko.edge_abs_mean_backward(ga, s, H, bw, W)
    dev = {"a": ko.edge_abs_mean(s, H, bw, W), "ds": ds, "dH": dH, "dbw": dbw, "dW": dW}
    res, n_amb = _fullcheck.check_edge_full(x, grid, k, bw, W, ga, dev, rows_per_block=64,
                                            outs_per_block=16)
    assert n_amb == 0
    for name, (worst, _, whole) in res.items():
        assert worst < 1e-13, name
    for name, idx in (("dH", (123, 4, 2)), ("ds", (321, 6)), ("dW", (33, 1, 5)),
                      ("dbw", (69, 0)), ("a", (7, 3))):
        bad = {key: v.copy() for key, v in dev.items()}
        bad[name][idx] += 1e-4 * np.abs(dev[name]).max()
        res, _ = _fullcheck.check_edge_full(x, grid, k, bw, W, ga, bad, rows_per_block=64,
                                            outs_per_block=16)
        assert res[name][0] > 1e-5, name
        assert all(res[other][0] < 1e-13 for other in res if other != name)
