"""Pins the oracle's higher-order derivatives (basis_derivative_n,
silu_derivative, kan_edge_derivative), which the native create_graph path is
checked against, and runs the module's create_graph maths on the CPU.

What pins what:
  * q = 0 and q = 1 reproduce basis_dense / basis_derivative (the latter is
    pinned by the reference's golden vectors and finite differences);
  * central finite differences of order q - 1, away from knots, in float64;
  * exact polynomial derivatives: coefficients that reproduce x^3 (k = 3) or
    x^2 (k = 2) give 6x, 6 and 2 through the derivative rows;
  * derivative rows sum to zero inside [t_k, t_{G+k}] (partition of unity);
  * order > k is zero.
A dropped p factor, a shifted window index or a swapped term fails the
finite-difference and polynomial checks.
"""

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko


def _grid(I, G, k, kind, seed=0):
    g = ko.uniform_grid(I, G, k)
    if kind == "nonuniform":
        rng = np.random.default_rng(seed)
        steps = rng.uniform(0.5, 1.5, size=(I, g.shape[1] - 1)) * (g[0, 1] - g[0, 0])
        g = np.concatenate([np.full((I, 1), -1.0 - k * 0.3), steps], axis=1).cumsum(axis=1)
    return g


def _away_from_knots(x, grid, h):
    """Mask of points farther than 4h from every knot of their feature."""
    d = np.abs(x[:, :, None] - grid[None]).min(axis=2)
    return d > 4 * h


@pytest.mark.parametrize("k", [1, 2, 3])
def test_low_orders_are_basis_and_first_derivative(k):
    rng = np.random.default_rng(k)
    grid = _grid(3, 6, k, "nonuniform", seed=k)
    x = rng.uniform(grid[:, 0] - 0.1, grid[:, -1] + 0.1, size=(200, 3))
    assert np.array_equal(ko.basis_derivative_n(x, grid, k, 0), ko.basis_dense(x, grid, k))
    assert np.array_equal(ko.basis_derivative_n(x, grid, k, 1), ko.basis_derivative(x, grid, k))
    z = ko.basis_derivative_n(x, grid, k, k + 1)
    assert z.shape == (200, 3, 6 + k) and not z.any()


@pytest.mark.parametrize("k", [2, 3])
@pytest.mark.parametrize("kind", ["uniform", "nonuniform"])
def test_finite_differences_of_the_previous_order(k, kind):
    rng = np.random.default_rng(10 + k)
    grid = _grid(4, 7, k, kind, seed=k)
    x = rng.uniform(grid[:, k], grid[:, -k - 1], size=(400, 4))
    h = 1e-6
    keep = _away_from_knots(x, grid, h)
    for q in range(2, k + 1):
        fd = (ko.basis_derivative_n(x + h, grid, k, q - 1)
              - ko.basis_derivative_n(x - h, grid, k, q - 1)) / (2 * h)
        an = ko.basis_derivative_n(x, grid, k, q)
        scale = np.abs(an).max()
        assert np.abs((fd - an)[keep]).max() < 1e-5 * scale, q


def _coeffs_for(poly, grid, k):
    """Spline coefficients reproducing poly on the interior (least squares on
    dense interior samples; exact since poly lies in the spline space)."""
    t = np.linspace(0.0, 1.0, 400)[:, None]
    xs = grid[None, :, k] + t * (grid[None, :, -k - 1] - grid[None, :, k])
    A = ko.basis_dense(xs, grid, k)
    c = np.stack([np.linalg.lstsq(A[:, i, :], poly(xs[:, i]), rcond=None)[0]
                  for i in range(grid.shape[0])])
    return c  # [I, R]


@pytest.mark.parametrize("kind", ["uniform", "nonuniform"])
def test_polynomial_derivatives_are_exact(kind):
    k = 3
    grid = _grid(2, 8, k, kind, seed=5)
    c = _coeffs_for(lambda v: v ** 3, grid, k)
    x = np.random.default_rng(2).uniform(grid[:, k], grid[:, -k - 1], size=(300, 2))
    vals = [np.einsum("nir,ir->ni", ko.basis_derivative_n(x, grid, k, q), c) for q in range(4)]
    assert np.abs(vals[0] - x ** 3).max() < 1e-10
    assert np.abs(vals[1] - 3 * x ** 2).max() < 1e-9
    assert np.abs(vals[2] - 6 * x).max() < 1e-8
    assert np.abs(vals[3] - 6.0).max() < 1e-7
    k = 2
    grid = _grid(2, 6, k, kind, seed=6)
    c = _coeffs_for(lambda v: v ** 2 - 0.5 * v, grid, k)
    x = np.random.default_rng(3).uniform(grid[:, k], grid[:, -k - 1], size=(300, 2))
    d2 = np.einsum("nir,ir->ni", ko.basis_derivative_n(x, grid, k, 2), c)
    assert np.abs(d2 - 2.0).max() < 1e-8


@pytest.mark.parametrize("k", [1, 2, 3])
def test_derivative_rows_sum_to_zero_inside(k):
    grid = _grid(3, 9, k, "nonuniform", seed=k)
    x = np.random.default_rng(k).uniform(grid[:, k], grid[:, -k - 1], size=(500, 3))
    for q in range(1, k + 1):
        d = ko.basis_derivative_n(x, grid, k, q)
        assert np.abs(d.sum(-1)).max() < 1e-9 * max(1.0, np.abs(d).max())


def test_silu_derivatives():
    x = np.linspace(-6, 6, 1001)
    assert np.array_equal(ko.silu_derivative(x, 0), ko.silu(x))
    assert np.array_equal(ko.silu_derivative(x, 1), ko.silu_grad(x))
    h = 1e-5
    for q in (2, 3, 4):
        fd = (ko.silu_derivative(x + h, q - 1) - ko.silu_derivative(x - h, q - 1)) / (2 * h)
        assert np.abs(fd - ko.silu_derivative(x, q)).max() < 1e-8


def test_edge_derivative_sums_to_forward_and_differentiates():
    rng = np.random.default_rng(4)
    I, O, G, k = 3, 2, 5, 3
    grid = _grid(I, G, k, "uniform")
    x = rng.uniform(-0.9, 0.9, size=(50, I))
    sw = rng.normal(size=(O, I, G + k))
    bw = rng.normal(size=(O, I))
    sc = rng.uniform(0.5, 1.5, size=(O, I))
    y, _ = ko.kan_forward(x, grid, bw, sw, sc, k)
    assert np.abs(ko.kan_edge_derivative(x, grid, bw, sw, sc, k, 0).sum(2) - y).max() < 1e-12
    h = 1e-6
    keep = _away_from_knots(x, grid, h)[:, None, :]
    for q in (1, 2, 3):
        fd = (ko.kan_edge_derivative(x + h, grid, bw, sw, sc, k, q - 1)
              - ko.kan_edge_derivative(x - h, grid, bw, sw, sc, k, q - 1)) / (2 * h)
        an = ko.kan_edge_derivative(x, grid, bw, sw, sc, k, q)
        err = np.abs(fd - an) * keep
        assert err.max() < 1e-5 * np.abs(an).max(), q


def test_reference_backend_create_graph_matches_oracle():
    """The CPU (reference-backend) PINN derivatives of one layer: u_x and
    u_xx by autograd against the oracle's edge derivatives."""
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(0)
    L = KANLinear(3, 2, grid_size=6, spline_order=3, backend="reference").double()
    with torch.no_grad():
        L.spline_weight.normal_(0, 0.2)
    x = (torch.rand(40, 3, dtype=torch.float64) * 1.8 - 0.9).requires_grad_()
    u = L(x)
    ux = torch.autograd.grad(u.sum(), x, create_graph=True)[0]
    uxx = torch.autograd.grad(ux.sum(), x, create_graph=True)[0]
    a = lambda t: t.detach().numpy()
    args = (a(x), a(L.grid), a(L.base_weight), a(L.spline_weight), a(L.spline_scaler), 3)
    assert np.abs(a(ux) - ko.kan_edge_derivative(*args, 1).sum(1)).max() < 1e-12
    assert np.abs(a(uxx) - ko.kan_edge_derivative(*args, 2).sum(1)).max() < 1e-10
