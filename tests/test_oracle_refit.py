"""Pins the oracle's knot update and least-squares refit (grid_from_samples,
curve2coeff, fit_spline_coeffs, refit_gram, update_grid) and checks the
module's CPU paths against it.

What pins what:
  * golden vectors written by the reference itself (tests/golden/make_golden.py:
    ReferenceKANLayer.update_grid in float32/float64, fit_spline_coeffs);
  * exact recovery: curves that lie in the new spline space come back with
    their own coefficients;
  * minimum-norm optimality on a rank-deficient fit (A^T (A c - y) = 0 and
    c orthogonal to null(A));
  * the identity C coef^T = A^T y_old behind the refit Gram route.
On the exactly rank-deficient golden case the reference's torch.linalg.lstsq
(gelsy driver) returns coefficients that do not solve the least-squares
problem (their residual is checked below); the oracle, like the native path,
returns the minimum-norm least-squares solution there.
"""

import os

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko

GOLD = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                            "reference_vectors.npz"))


@pytest.mark.parametrize("tag,dt", [("32", np.float32), ("64", np.float64)])
def test_grid_from_samples_matches_reference_bit_for_bit(tag, dt):
    x = GOLD["ug_x"].astype(dt)
    grid = ko.grid_from_samples(x, 5, 3, float(GOLD["ug_grid_eps"]), 0.01)
    assert grid.dtype == dt
    assert np.array_equal(grid, GOLD["ug_grid" + tag])
    assert (np.diff(grid, axis=1) > 0).all()


def test_grid_from_samples_interior_closed_form():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(501, 4))
    G, k, eps, margin = 6, 2, 0.1, 0.05
    grid = ko.grid_from_samples(x, G, k, eps, margin)
    xs = np.sort(x, axis=0)
    lo, hi = xs[0] - margin, xs[-1] + margin
    for j in range(G + 1):
        q = min(max(j * (1 - eps) / G + eps / 2, 0.0), 1.0)
        quant = np.array([np.interp(q * 500, np.arange(501), xs[:, i]) for i in range(4)])
        expect = (1 - eps) * quant + eps * (lo + j / G * (hi - lo))
        assert np.allclose(grid[:, k + j], expect, rtol=0, atol=1e-14)
    step = (hi - lo) / G
    assert np.allclose(grid[:, 0], grid[:, k] - k * step, atol=1e-14)
    assert np.allclose(grid[:, -1], grid[:, k + G] + k * step, atol=1e-14)


@pytest.mark.parametrize("tag,dt,tol", [("32", np.float32, 1e-5), ("64", np.float64, 1e-12)])
def test_update_grid_matches_reference(tag, dt, tol):
    x, coef = GOLD["ug_x"].astype(dt), GOLD["ug_coef"].astype(dt)
    grid, sw = ko.update_grid(x, GOLD["ug_grid_old" + tag], coef, 5, 3,
                              float(GOLD["ug_grid_eps"]), 0.01)
    assert np.array_equal(grid, GOLD["ug_grid" + tag])
    ref = GOLD["ug_sw" + tag]
    assert np.abs(sw - ref).max() / np.abs(ref).max() < tol


def test_curve2coeff_recovers_curves_in_the_spline_space():
    rng = np.random.default_rng(0)
    G, k, I, O = 7, 3, 3, 4
    grid = ko.uniform_grid(I, G, k)
    x = rng.uniform(-1, 1, size=(400, I))
    c = rng.normal(size=(O, I, G + k))
    y = np.einsum("oir,bir->obi", c, ko.basis_dense(x, grid, k))
    assert np.abs(ko.curve2coeff(x, y, grid, k) - c).max() < 1e-10
    sw = ko.fit_spline_coeffs(x, y, grid, k, ridge=1e-14)
    assert np.abs(sw - c).max() < 1e-8


def test_curve2coeff_minimum_norm_on_rank_deficient_fit():
    x, g_old, coef, g_new = GOLD["rd_x"], GOLD["rd_grid_old"], GOLD["rd_coef"], GOLD["rd_grid"]
    y = np.einsum("oir,bir->obi", coef, ko.basis_dense(x, g_old, 2))
    grid, sw = ko.update_grid(x, g_old, coef, 4, 2, float(GOLD["ug_grid_eps"]), 0.05)
    assert np.array_equal(grid, g_new)
    A = ko.basis_dense(x, g_new, 2)
    for i in range(x.shape[1]):
        Ai, yi, ci = A[:, i, :], y[:, :, i].T, sw[:, i, :].T
        U, s, Vt = np.linalg.svd(Ai)
        null = Vt[(s > 1e-12 * s[0]).sum():]
        assert np.abs(Ai.T @ (Ai @ ci - yi)).max() < 1e-12           # normal equations
        assert np.abs(null @ ci).max() < 1e-12                       # no null-space part
        ref = GOLD["rd_sw"][:, i, :].T                               # gelsy's coefficients
        assert np.linalg.norm(Ai @ ref - yi) > 1e-3 > np.linalg.norm(Ai @ ci - yi)


def test_fit_spline_coeffs_matches_reference():
    y_old = np.einsum("oir,bir->obi", GOLD["fs_coef"],
                      ko.basis_dense(GOLD["fs_x"], GOLD["fs_grid_old"], 3))
    sw = ko.fit_spline_coeffs(GOLD["fs_x"], y_old, GOLD["fs_grid_new"], 3, 1e-12)
    ref = GOLD["fs_sw"]
    assert np.abs(sw - ref).max() / np.abs(ref).max() < 1e-12


def test_refit_gram_cross_term_gives_normal_equation_rhs():
    rng = np.random.default_rng(1)
    x = rng.uniform(-1.2, 1.2, size=(300, 3))
    g_old, g_new = ko.uniform_grid(3, 5, 3), ko.uniform_grid(3, 9, 3)
    coef = rng.normal(size=(2, 3, 8))
    G, C = ko.refit_gram(x, g_old, g_new, 3)
    A = ko.basis_dense(x, g_new, 3)
    y_old = np.einsum("oir,bir->obi", coef, ko.basis_dense(x, g_old, 3))
    assert np.abs(np.einsum("irs,ois->iro", C, coef) - np.einsum("bir,obi->iro", A, y_old)).max() < 1e-12
    assert np.allclose(G, np.transpose(G, (0, 2, 1)))
    assert (np.linalg.eigvalsh(G) > -1e-12).all()


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 1e-5)])
def test_module_cpu_update_grid_matches_oracle(dtype, tol):
    from torchsplinekan_amd import KANLinear
    g = torch.Generator().manual_seed(7)
    L = KANLinear(5, 3, grid_size=6, spline_order=3, backend="reference").to(dtype)
    with torch.no_grad():
        L.spline_weight.copy_(torch.randn(3, 5, 9, generator=g, dtype=dtype) * 0.1)
    x = torch.randn(300, 5, generator=g, dtype=dtype) * 0.6
    a = lambda t: t.detach().numpy()
    grid_ref, sw_ref = ko.update_grid(a(x), a(L.grid), a(L.spline_weight), 6, 3,
                                      L._ref.grid_eps, 0.02)
    L.update_grid(x, margin=0.02)
    assert np.array_equal(a(L.grid), grid_ref) and torch.equal(L.grid, L._ref.grid)
    assert np.abs(a(L.spline_weight) - sw_ref).max() / np.abs(sw_ref).max() < tol


def test_module_cpu_extend_grid_matches_oracle():
    from torchsplinekan_amd import KAN, KANLinear
    g = torch.Generator().manual_seed(8)
    L = KANLinear(4, 2, grid_size=5, spline_order=3, backend="reference").double()
    with torch.no_grad():
        L.spline_weight.copy_(torch.randn(2, 4, 8, generator=g, dtype=torch.float64) * 0.1)
    x = torch.rand(250, 4, generator=g, dtype=torch.float64) * 2 - 1
    new = L.extend_grid(10, x)
    assert new.grid_size == 10 and tuple(new.spline_weight.shape) == (2, 4, 13)
    a = lambda t: t.detach().numpy()
    y_old = np.einsum("oir,bir->obi", a(L.spline_weight), ko.basis_dense(a(x), a(L.grid), 3))
    ref = ko.fit_spline_coeffs(a(x), y_old, a(new.grid), 3, 1e-12)
    assert np.abs(a(new.spline_weight) - ref).max() / np.abs(ref).max() < 1e-12
    # uniform refinement of a uniform grid: old knots are a subset, the old
    # spline is exactly representable, so the refined layer reproduces it
    xt = torch.rand(64, 4, generator=g, dtype=torch.float64) * 2 - 1
    assert torch.allclose(new(xt), L(xt), atol=1e-9)
    # seeded: the second layer is refit on the hidden activations of x, and
    # the refined network reproduces the coarse one only where those samples
    # support every refined basis function (some random initialisations leave
    # a refined interval with too few samples)
    torch.manual_seed(0)
    net = KAN([4, 3, 2], grid_size=5, backend="reference").double()
    fine = net.extend_grid(10, x)
    assert fine.widths == [4, 3, 2] and all(l.grid_size == 10 for l in fine.layers)
    assert torch.allclose(fine(xt), net(xt), atol=1e-6)
