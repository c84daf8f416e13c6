"""The oracle against golden vectors written by the reference implementation
itself (tests/golden/make_golden.py: compute_basis, compute_basis_derivative
and config 1 through ReferenceKANLayer), and, on the GPU, the native
kernels against the same vectors."""

import os

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests._util import normwise

GOLD = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                            "reference_vectors.npz"))
CASES = [(k, kind) for k in (1, 2, 3) for kind in ("uniform", "nonuniform", "repeated")]


@pytest.mark.parametrize("k,kind", CASES)
def test_oracle_basis_reproduces_reference_rounding(k, kind):
    tag = f"basis_k{k}_{kind}"
    grid, x = GOLD[tag + "_grid"], GOLD[tag + "_x"]
    # float32: bit-identical to the reference backend's rounding sequence
    assert np.array_equal(ko.basis_dense(x, grid, k), GOLD[tag + "_H32"])
    H64 = ko.basis_dense(x.astype(np.float64), grid.astype(np.float64), k)
    assert np.array_equal(H64, GOLD[tag + "_H64"])
    d64 = ko.basis_derivative(x.astype(np.float64), grid.astype(np.float64), k)
    assert np.allclose(d64, GOLD[tag + "_dH64"], atol=1e-13, rtol=0)


def _c1_oracle(dt):
    x, coef, bw, D = (GOLD["c1_x"].astype(dt), GOLD["c1_coef"].astype(dt),
                      GOLD["c1_bw"].astype(dt), GOLD["c1_D"].astype(dt))
    grid = GOLD["c1_grid64"].astype(dt)
    sc = np.ones(bw.shape, dtype=dt)
    y, H = ko.kan_forward(x, grid, bw, coef, sc, 3)
    return (y,) + ko.kan_backward(D, x, grid, bw, coef, sc, 3, basis=H)


def test_oracle_config1_matches_reference():
    assert np.array_equal(GOLD["c1_grid32"], ko.uniform_grid(16, 5, 3, dtype=np.float32))
    got = _c1_oracle(np.float64)
    names = ["y", "gx", "gbw", "gsw", "gsc"]
    for name, g in zip(names, got):
        assert normwise(g, GOLD[f"c1_{name}64"]) < 1e-12, name
        # the reference's float32 run is within the fp32 bar of the fp64 truth
        assert normwise(GOLD[f"c1_{name}32"], g) < 1e-5, name


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_native_config1_matches_reference_vectors(dtype):
    from torchsplinekan_amd import KANLinear
    tag = "32" if dtype == torch.float32 else "64"
    L = KANLinear(16, 8, grid_size=5, spline_order=3, backend="cuda").to(dtype)
    with torch.no_grad():
        L.spline_weight.copy_(torch.from_numpy(GOLD["c1_coef"]))
        L.base_weight.copy_(torch.from_numpy(GOLD["c1_bw"]))
        L.spline_scaler.fill_(1.0)
    L = L.cuda()
    x = torch.from_numpy(GOLD["c1_x"]).to("cuda", dtype).requires_grad_()
    D = torch.from_numpy(GOLD["c1_D"]).to("cuda", dtype)
    y = L(x)
    assert L.last_backend == "cuda"
    (y * D).sum().backward()
    got = [y, x.grad, L.base_weight.grad, L.spline_weight.grad, L.spline_scaler.grad]
    tol = 1e-5 if dtype == torch.float32 else 1e-12
    for name, g in zip(["y", "gx", "gbw", "gsw", "gsc"], got):
        assert normwise(g.detach().cpu().double().numpy(), GOLD[f"c1_{name}64"]) < tol, name


@pytest.mark.gpu
@pytest.mark.parametrize("k,kind", CASES)
def test_native_legacy_basis_bit_identical_to_reference_fp32(k, kind):
    from torchsplinekan_amd import _C
    tag = f"basis_k{k}_{kind}"
    grid = torch.from_numpy(GOLD[tag + "_grid"]).cuda()
    x = torch.from_numpy(GOLD[tag + "_x"]).cuda()
    try:
        _C.set_basis_impl(0)
        H0 = _C.basis(x, grid, k).cpu().numpy()
    finally:
        _C.set_basis_impl(1)
    H1 = _C.basis(x, grid, k).cpu().numpy()
    assert np.array_equal(H0, GOLD[tag + "_H32"])
    assert np.abs(H1 - GOLD[tag + "_H64"]).max() < 2e-6
    out = (GOLD[tag + "_x"] < GOLD[tag + "_grid"][:, 0][None]) | \
          (GOLD[tag + "_x"] > GOLD[tag + "_grid"][:, -1][None])
    assert (H1[out] == 0).all() and (GOLD[tag + "_H32"][out] == 0).all()
