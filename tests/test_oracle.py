"""Pins the CPU oracle (oracle/kan_oracle.py) against what the mathematics
fixes, so that a dropped term, a wrong sign or index or a transposed operand
in the oracle fails here:

* basis: exact rational Cox-de Boor (fractions.Fraction) on small grids;
  closed-form uniform B-splines for k = 1, 2, 3; partition of unity;
  non-negativity; at most k+1 non-zeros; exact zeros outside the knot span;
  two independent formulations (dense recurrence and local de Boor) agree;
* derivative: central finite differences; exact cubic reproduction x^3 - x;
* forward: brute-force loop over the definition;
* backward: finite differences of the forward for all four gradients;
* edge statistic: brute-force loop; finite-difference backward;
* regulariser: closed form on hand-computed values; finite differences;
  all-zero layer.

Mirrors the reference's invariant tests (tests/test_reference.py:10-23,
tests/test_local_basis.py:40-68, tests/test_math_correctness.py:205-236,
tests/test_corrections.py:195-249, tests/test_fused_regularization.py:110-162).
"""

import itertools
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests._util import make_grid, make_points


def _rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# basis
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("k", [1, 2, 3])
@pytest.mark.parametrize("kind", ["uniform", "nonuniform", "repeated"])
def test_basis_dense_matches_exact_rational(k, kind):
    G = 4
    grid = make_grid(2, G, k, kind, seed=7 + k).numpy()
    x = make_points(torch.from_numpy(grid), n=40, seed=k).numpy()
    H = ko.basis_dense(x, grid, k)
    for n in range(x.shape[0]):
        for i in range(x.shape[1]):
            exact = ko.basis_fraction(float(x[n, i]), [float(v) for v in grid[i]], k)
            assert np.allclose(H[n, i], [float(e) for e in exact], atol=1e-14, rtol=0)


def _uniform_closed_form(u, k):
    """Uniform B-spline pieces on one span, u in [0, 1): values of the k+1
    functions active on that span, lowest index first."""
    if k == 1:
        return [1 - u, u]
    if k == 2:
        return [(1 - u) ** 2 / 2, (-2 * u * u + 2 * u + 1) / 2, u * u / 2]
    return [(1 - u) ** 3 / 6, (3 * u ** 3 - 6 * u ** 2 + 4) / 6,
            (-3 * u ** 3 + 3 * u ** 2 + 3 * u + 1) / 6, u ** 3 / 6]


@pytest.mark.parametrize("k", [1, 2, 3])
def test_basis_uniform_closed_form(k):
    G = 6
    grid = make_grid(1, G, k, "uniform").numpy()
    h = 2.0 / G
    x = _rng(k).uniform(-1, 1, size=(500, 1))
    H = ko.basis_dense(x, grid, k)
    for n in range(x.shape[0]):
        m = int(np.floor((x[n, 0] - grid[0, 0]) / h + 1e-12))   # span t_m <= x < t_{m+1}
        m = min(m, grid.shape[1] - 2)
        u = (x[n, 0] - grid[0, m]) / h
        expect = np.zeros(G + k)
        for j, v in enumerate(_uniform_closed_form(u, k)):
            r = m - k + j
            if 0 <= r < G + k:
                expect[r] = v
        assert np.allclose(H[n, 0], expect, atol=1e-12)


@pytest.mark.parametrize("k", [1, 2, 3])
@pytest.mark.parametrize("G", [1, 4, 17])
def test_basis_invariants(k, G):
    grid = make_grid(3, G, k, "nonuniform", seed=G).numpy()
    x = make_points(torch.from_numpy(grid), n=800, seed=G).numpy()
    H = ko.basis_dense(x, grid, k)
    assert (H >= -1e-15).all()
    assert ((H != 0).sum(-1) <= k + 1).all()
    inner = (x >= grid[:, k][None]) & (x <= grid[:, k + G][None])
    assert np.allclose(H.sum(-1)[inner], 1.0, atol=1e-13)
    out = (x < grid[:, 0][None]) | (x > grid[:, -1][None])
    assert out.any() and (H[out] == 0).all()


@pytest.mark.parametrize("k", [1, 2, 3])
@pytest.mark.parametrize("kind", ["uniform", "nonuniform", "repeated"])
def test_local_and_dense_formulations_agree(k, kind):
    grid = make_grid(2, 9, k, kind, seed=k).numpy()
    x = make_points(torch.from_numpy(grid), n=150, seed=k + 1).numpy()
    assert np.allclose(ko.basis_local(x, grid, k), ko.basis_dense(x, grid, k), atol=1e-13, rtol=0)


def test_basis_nan_policy():
    grid = ko.uniform_grid(1, 5, 3)
    x = np.array([[np.nan]])
    # dense recurrence (reference backend): NaN propagates (0 * NaN)
    assert np.isnan(ko.basis_dense(x, grid, 3)).all()
    # local scheme (native path): NaN is out of range -> zero row
    assert (ko.basis_local(x, grid, 3) == 0).all()


# ---------------------------------------------------------------------------
# derivative
# ---------------------------------------------------------------------------

def _away_from_knots(grid, n, seed, margin=1e-3):
    x = _rng(seed).uniform(grid[:, 0].min(), grid[:, -1].max(), size=(n, grid.shape[0]))
    for i in range(grid.shape[0]):
        d = np.abs(x[:, i, None] - grid[i][None]).min(-1)
        x[d < margin, i] += 2 * margin
    return x


@pytest.mark.parametrize("k", [1, 2, 3])
def test_derivative_matches_finite_differences(k):
    grid = make_grid(2, 7, k, "nonuniform", seed=3).numpy()
    x = _away_from_knots(grid, 300, seed=k)
    d = ko.basis_derivative(x, grid, k)
    eps = 1e-6
    fd = (ko.basis_dense(x + eps, grid, k) - ko.basis_dense(x - eps, grid, k)) / (2 * eps)
    assert np.allclose(d, fd, atol=1e-6)


def test_cubic_reproduction_and_second_derivative():
    """u(x) = x^3 - x is a cubic spline on any knot vector; coefficients by
    least squares reproduce it exactly; u' = 3x^2 - 1 through the derivative."""
    k, G = 3, 8
    grid = ko.uniform_grid(1, G, k)
    xs = np.linspace(-1, 1, 200)[:, None]
    H = ko.basis_dense(xs, grid, k)[:, 0, :]
    c, *_ = np.linalg.lstsq(H, (xs ** 3 - xs)[:, 0], rcond=None)
    xt = _rng(0).uniform(-0.99, 0.99, size=(100, 1))
    assert np.allclose(ko.basis_dense(xt, grid, k)[:, 0, :] @ c, xt[:, 0] ** 3 - xt[:, 0], atol=1e-12)
    du = ko.basis_derivative(xt, grid, k)[:, 0, :] @ c
    assert np.allclose(du, 3 * xt[:, 0] ** 2 - 1, atol=1e-10)


# ---------------------------------------------------------------------------
# forward / backward
# ---------------------------------------------------------------------------

def _layer(N, I, O, G, k, seed, scaler=True, base=True):
    r = _rng(seed)
    grid = make_grid(I, G, k, "nonuniform", seed=seed).numpy()
    x = r.uniform(-1.2, 1.2, size=(N, I))
    sw = r.normal(0, 0.3, size=(O, I, G + k))
    bw = r.normal(0, 0.5, size=(O, I)) if base else None
    sc = r.uniform(0.5, 1.5, size=(O, I)) if scaler else None
    return x, grid, bw, sw, sc


@pytest.mark.parametrize("scaler,base", [(True, True), (False, True), (True, False)])
def test_forward_matches_brute_force(scaler, base):
    N, I, O, G, k = 7, 3, 4, 5, 2
    x, grid, bw, sw, sc = _layer(N, I, O, G, k, 1, scaler, base)
    y, H = ko.kan_forward(x, grid, bw, sw, sc, k)
    for n, o in itertools.product(range(N), range(O)):
        acc = 0.0
        for i in range(I):
            if base:
                acc += bw[o, i] * x[n, i] / (1 + np.exp(-x[n, i]))
            b = [float(v) for v in ko.basis_fraction(x[n, i], list(grid[i]), k)]
            s = sc[o, i] if scaler else 1.0
            acc += s * sum(sw[o, i, r] * b[r] for r in range(G + k))
        assert abs(y[n, o] - acc) < 1e-12


@pytest.mark.parametrize("scaler,base", [(True, True), (False, False)])
def test_backward_matches_finite_differences(scaler, base):
    N, I, O, G, k = 6, 3, 2, 4, 3
    x, grid, bw, sw, sc = _layer(N, I, O, G, k, 2, scaler, base)
    x = _away_from_knots(grid, N, seed=9)
    D = _rng(4).normal(size=(N, O))

    def loss(x_, bw_, sw_, sc_):
        return (ko.kan_forward(x_, grid, bw_, sw_, sc_, k)[0] * D).sum()

    gx, gbw, gsw, gsc = ko.kan_backward(D, x, grid, bw, sw, sc, k)
    eps = 1e-6
    args = [x, bw, sw, sc]
    grads = [gx, gbw, gsw, gsc]
    for a_idx in range(4):
        if args[a_idx] is None:
            assert grads[a_idx] is None
            continue
        base_arr = args[a_idx]
        fd = np.zeros_like(base_arr)
        for idx in np.ndindex(base_arr.shape):
            p = [a.copy() if a is not None else None for a in args]
            m = [a.copy() if a is not None else None for a in args]
            p[a_idx][idx] += eps
            m[a_idx][idx] -= eps
            fd[idx] = (loss(*p) - loss(*m)) / (2 * eps)
        assert np.allclose(grads[a_idx], fd, atol=1e-6), a_idx


def test_params_only_backward_equals_full_backward():
    N, I, O, G, k = 9, 4, 3, 5, 3
    x, grid, bw, sw, sc = _layer(N, I, O, G, k, 5)
    D = _rng(1).normal(size=(N, O))
    _, H = ko.kan_forward(x, grid, bw, sw, sc, k)
    full = ko.kan_backward(D, x, grid, bw, sw, sc, k, basis=H)
    part = ko.kan_backward_params(D, x, bw, sw, sc, H)
    for a, b in zip(full[1:], part):
        assert np.allclose(a, b, atol=1e-15)


# ---------------------------------------------------------------------------
# edge statistic and regulariser
# ---------------------------------------------------------------------------

def _edge(N, I, O, R, seed, base=True):
    r = _rng(seed)
    s = r.normal(size=(N, I)) if base else None
    H = r.uniform(size=(N, I, R))
    bw = r.normal(size=(O, I)) if base else None
    W = r.normal(size=(O, I, R))
    return s, H, bw, W


@pytest.mark.parametrize("base", [True, False])
def test_edge_abs_mean_matches_brute_force(base):
    N, I, O, R = 11, 3, 4, 5
    s, H, bw, W = _edge(N, I, O, R, 0, base)
    a = ko.edge_abs_mean(s, H, bw, W, chunk=4)
    for o, i in itertools.product(range(O), range(I)):
        tot = 0.0
        for n in range(N):
            phi = (s[n, i] * bw[o, i] if base else 0.0) + sum(H[n, i, r] * W[o, i, r]
                                                               for r in range(R))
            tot += abs(phi)
        assert abs(a[o, i] - tot / N) < 1e-13


@pytest.mark.parametrize("base", [True, False])
def test_edge_abs_mean_by_feature_matches_edge_abs_mean(base):
    N, I, O, R = 300, 7, 9, 6
    s, H, bw, W = _edge(N, I, O, R, 5, base)
    a = ko.edge_abs_mean(s, H, bw, W, chunk=64)
    b = ko.edge_abs_mean_by_feature(s, H, bw, W, workers=3)
    assert b.shape == a.shape and np.abs(a - b).max() < 1e-13 * np.abs(a).max()
    sub = ko.edge_abs_mean_by_feature(s, H, bw, W, features=[5, 0, 3], workers=2)
    assert np.abs(sub - a[:, [5, 0, 3]]).max() < 1e-13 * np.abs(a).max()


@pytest.mark.parametrize("base", [True, False])
def test_edge_backward_matches_finite_differences(base):
    N, I, O, R = 5, 2, 3, 4
    s, H, bw, W = _edge(N, I, O, R, 1, base)
    ga = _rng(2).normal(size=(O, I))
    ds, dH, dbw, dW = ko.edge_abs_mean_backward(ga, s, H, bw, W, chunk=2)
    eps = 1e-7
    args = [s, H, bw, W]
    grads = [ds, dH, dbw, dW]

    def f(*a):
        return (ko.edge_abs_mean(*a) * ga).sum()

    for a_idx in range(4):
        if args[a_idx] is None:
            assert grads[a_idx] is None
            continue
        fd = np.zeros_like(args[a_idx])
        for idx in np.ndindex(args[a_idx].shape):
            p = [a.copy() if a is not None else None for a in args]
            m = [a.copy() if a is not None else None for a in args]
            p[a_idx][idx] += eps
            m[a_idx][idx] -= eps
            fd[idx] = (f(*p) - f(*m)) / (2 * eps)
        assert np.allclose(grads[a_idx], fd, atol=1e-6), a_idx


def test_edge_sign_zero_contributes_nothing():
    s = np.zeros((3, 1))
    H = np.zeros((3, 1, 2))
    bw = np.ones((1, 1))
    W = np.ones((1, 1, 2))
    ds, dH, dbw, dW = ko.edge_abs_mean_backward(np.ones((1, 1)), s, H, bw, W)
    assert (ds == 0).all() and (dH == 0).all() and (dbw == 0).all() and (dW == 0).all()


def test_regulariser_closed_form_and_gradient():
    a = np.array([[0.1, 0.3], [0.2, 0.4]])
    A = 1.0
    p = a / A
    S = -(p * np.log(p)).sum()
    assert abs(ko.regularization_from_edge_means(a, 0.7, 0.3) - (0.7 * A + 0.3 * S)) < 1e-15
    g = ko.regularization_grad(a, 0.7, 0.3)
    eps = 1e-7
    fd = np.zeros_like(a)
    for idx in np.ndindex(a.shape):
        ap, am = a.copy(), a.copy()
        ap[idx] += eps
        am[idx] -= eps
        fd[idx] = (ko.regularization_from_edge_means(ap, 0.7, 0.3)
                   - ko.regularization_from_edge_means(am, 0.7, 0.3)) / (2 * eps)
    assert np.allclose(g, fd, atol=1e-7)


def test_regulariser_zero_layer_is_finite():
    a = np.zeros((3, 2))
    assert ko.regularization_from_edge_means(a, 1.0, 1.0) == pytest.approx(0.0, abs=1e-30)
    g = ko.regularization_grad(a, 0.0, 1.0)
    assert np.isfinite(g).all()


def test_uniform_grid_rounding_matches_fp32_formula():
    g = ko.uniform_grid(2, 10, 3, dtype=np.float32)
    r = np.arange(17, dtype=np.float32)
    expect = np.float32(-1) + ((r - np.float32(3)) * np.float32(2)) / np.float32(10)
    assert np.array_equal(g[0], expect) and np.array_equal(g[1], expect)
    assert g[0, 3] == np.float32(-1) and g[0, 13] == np.float32(1)


def test_fraction_basis_is_exact():
    b = ko.basis_fraction(Fraction(1, 3), [0, 1, 2, 3, 4], 3)
    assert b == [Fraction(1, 162)]
