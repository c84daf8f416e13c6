"""CPU checks of tests/_slack.py, the checker the workload-level GPU tests
use for regularised layers: with no ambiguous terms its gradients equal the
oracle's own (kan_backward / kan_backward_params plus edge_abs_mean_backward
chained through silu' and the basis derivative); ambiguous terms are
detected where |phi| is at rounding level and their slack bounds every
sign choice."""

import numpy as np

from oracle import kan_oracle as ko
from tests import _slack


def _layer(N=60, I=5, O=4, G=6, k=3, seed=0):
    r = np.random.default_rng(seed)
    x = r.uniform(-1.1, 1.1, size=(N, I))
    grid = ko.uniform_grid(I, G, k)
    sw = r.normal(0, 0.2, size=(O, I, G + k))
    bw = r.normal(0, 0.3, size=(O, I))
    sc = r.uniform(0.5, 1.5, size=(O, I))
    D = r.normal(size=(N, O))
    ga = r.normal(size=(O, I))
    return x, grid, bw, sw, sc, D, ga, k


def test_param_and_input_grads_equal_the_oracle_chain():
    x, grid, bw, sw, sc, D, ga, k = _layer()
    N, I = x.shape
    O = sw.shape[0]
    H = ko.basis_dense(x, grid, k)
    s = ko.silu(x)
    W = sw * sc[:, :, None]
    # oracle: linear layer gradients + edge statistic gradients, chained to x
    gx, gbw, gsw, gsc = ko.kan_backward(D, x, grid, bw, sw, sc, k, basis=H)
    ds, dH, dbw_e, dWe = ko.edge_abs_mean_backward(ga, s, H, bw, W)
    gbw = gbw + dbw_e
    gsw = gsw + sc[:, :, None] * dWe
    gsc = gsc + (sw * dWe).sum(2)
    gx = gx + ds * ko.silu_grad(x) + (dH * ko.basis_derivative(x, grid, k)).sum(2)
    edges = [(o, i) for o in range(O) for i in range(I)]
    res, n_amb = _slack.edge_param_grads(D, ga, s, H, bw, sw, sc, edges)
    assert n_amb == 0
    oo, ii = zip(*edges)
    for name, ref in (("spline_weight", gsw[oo, ii]), ("spline_scaler", gsc[oo, ii]),
                      ("base_weight", gbw[oo, ii])):
        got, slack = res[name]
        assert np.abs(got - ref).max() < 1e-13 and np.all(slack == 0)
    rows = [0, 7, N - 1]
    ref_x, slack_x, n_amb = _slack.edge_input_grads(D, ga, x, grid, k, s, H, bw, sw, sc, rows)
    assert n_amb == 0 and np.all(slack_x == 0)
    assert np.abs(ref_x - gx[rows]).max() < 1e-13


def test_without_statistic_or_output_term():
    x, grid, bw, sw, sc, D, ga, k = _layer(seed=1)
    H = ko.basis_dense(x, grid, k)
    s = ko.silu(x)
    gbw, gsw, gsc = ko.kan_backward_params(D, x, bw, sw, sc, H)
    res, _ = _slack.edge_param_grads(D, None, s, H, bw, sw, sc, [(1, 2), (3, 0)])
    assert np.abs(res["spline_weight"][0] - gsw[[1, 3], [2, 0]]).max() < 1e-13
    assert np.abs(res["base_weight"][0] - gbw[[1, 3], [2, 0]]).max() < 1e-13
    W = sw * sc[:, :, None]
    _, _, dbw, dW = ko.edge_abs_mean_backward(ga, s, H, bw, W)
    res, _ = _slack.edge_param_grads(None, ga, s, H, bw, sw, sc, [(1, 2)])
    assert np.abs(res["base_weight"][0] - dbw[1, 2]).max() < 1e-13
    assert np.abs(res["spline_weight"][0] - sc[1, 2] * dW[1, 2]).max() < 1e-13


def test_ambiguous_terms_are_found_and_bounded():
    """Plant phi = 0 exactly on one edge and sample (bw chosen to cancel the
    spline part there): that term is ambiguous, the oracle uses g = 0 for it,
    and any device sign choice stays within the slack."""
    x, grid, bw, sw, sc, D, ga, k = _layer(seed=2)
    H = ko.basis_dense(x, grid, k)
    s = ko.silu(x)
    n0, o0, i0 = 3, 1, 2
    W = sw * sc[:, :, None]
    bw = bw.copy()
    bw[o0, i0] = -(H[n0, i0] @ W[o0, i0]) / s[n0, i0]
    res, n_amb = _slack.edge_param_grads(D, ga, s, H, bw, sw, sc, [(o0, i0)])
    assert n_amb >= 1
    ref, slack = res["base_weight"]
    N = x.shape[0]
    for sign in (-1.0, 1.0):   # a device that took either sign at the planted term
        dev = ref + sign * ga[o0, i0] / N * s[n0, i0]
        assert _slack.within(dev, ref, slack, 0.0) <= 1e-15
    dev = ref + 3.0 * abs(ga[o0, i0]) / N * abs(s[n0, i0])   # beyond any sign choice
    assert _slack.within(dev, ref, slack, 0.0) > 0


def test_operand_grads_equal_the_oracle():
    x, grid, bw, sw, sc, D, ga, k = _layer(seed=3)
    H = ko.basis_dense(x, grid, k)
    s = ko.silu(x)
    ds, dH, _, _ = ko.edge_abs_mean_backward(ga, s, H, bw, sw)
    rows = [1, 4, 59]
    rds, sds, rdH, sdH, n_amb = _slack.edge_operand_grads(ga, s, H, bw, sw, rows)
    assert n_amb == 0 and np.all(sds == 0) and np.all(sdH == 0)
    assert np.abs(rds - ds[rows]).max() < 1e-13 and np.abs(rdH - dH[rows]).max() < 1e-13
    _, dH0, _, _ = ko.edge_abs_mean_backward(ga, None, H, None, sw)
    rds, _, rdH, _, _ = _slack.edge_operand_grads(ga, None, H, None, sw, rows)
    assert rds is None and np.abs(rdH - dH0[rows]).max() < 1e-13


def test_full_edge_backward_equals_the_oracle():
    x, grid, bw, sw, sc, D, ga, k = _layer(seed=4)
    H = ko.basis_dense(x, grid, k)
    s = ko.silu(x)
    ref = ko.edge_abs_mean_backward(ga, s, H, bw, sw)
    got, slack, n_amb = _slack.edge_backward_full(ga, s, H, bw, sw, chunk=7)
    assert n_amb == 0
    for a, b, sl in zip(got, ref, slack):
        assert np.abs(a - b).max() < 1e-13 and np.all(sl == 0)
    # with dL/dy: the linear layer's products added
    got, _, _ = _slack.edge_backward_full(ga, s, H, bw, sw, D=D, chunk=16)
    N, I, R = H.shape
    O = sw.shape[0]
    lin = (D @ bw, (D @ sw.reshape(O, I * R)).reshape(N, I, R), D.T @ s,
           (D.T @ H.reshape(N, I * R)).reshape(O, I, R))
    for a, b, l in zip(got, ref, lin):
        assert np.abs(a - (b + l)).max() < 1e-12
    got, slack, _ = _slack.edge_backward_full(ga, None, H, None, sw)
    assert got[0] is None and got[2] is None and slack[0] is None
    ref0 = ko.edge_abs_mean_backward(ga, None, H, None, sw)
    assert np.abs(got[1] - ref0[1]).max() < 1e-13 and np.abs(got[3] - ref0[3]).max() < 1e-13


def test_full_layer_grads_equal_the_sampled_helpers():
    """layer_grads_full (every edge and row, features in threads) equals the
    sampled helpers entry for entry, slack included, with and without the
    output term, the statistic and the base branch; a planted phi = 0 is
    found as ambiguous by both."""
    x, grid, bw, sw, sc, D, ga, k = _layer(N=50, I=6, O=5, seed=7)
    N, I = x.shape
    O = sw.shape[0]
    H = ko.basis_dense(x, grid, k)
    s = ko.silu(x)
    # plant phi[n0, o0, i0] = 0 exactly (base term cancels the spline term)
    n0, o0, i0 = 3, 2, 4
    bw = bw.copy()
    bw[o0, i0] = -(H[n0, i0] @ (sw[o0, i0] * sc[o0, i0])) / s[n0, i0]
    edges = [(o, i) for o in range(O) for i in range(I)]
    rows = list(range(N))
    for Dv, gav, base in ((D, ga, True), (None, ga, True), (D, None, True), (D, ga, False)):
        b = bw if base else None
        sv = s if base else None
        full, n_full = _slack.layer_grads_full(Dv, gav, x, grid, k, sv, H, b, sw, sc, workers=3)
        res, n_par = _slack.edge_param_grads(Dv, gav, sv, H, b, sw, sc, edges)
        assert n_full == n_par
        if gav is not None and base:
            assert n_full >= 1   # the planted term
        oo, ii = map(np.array, zip(*edges))
        for name, (ref, slack) in res.items():
            fr, fs = full[name]
            assert np.abs(fr[oo, ii] - ref).max() < 1e-13, name
            assert np.abs(fs[oo, ii] - slack).max() < 1e-13, name
        rx, sx, _ = _slack.edge_input_grads(Dv, gav, x, grid, k, sv, H, b, sw, sc, rows)
        assert np.abs(full["x"][0] - rx).max() < 1e-12
        assert np.abs(full["x"][1] - sx).max() < 1e-13
        assert ("base_weight" in full) == base


def test_slack_adjusted_differences():
    ref = np.array([1.0, -2.0, 3.0, 0.0])
    dev = np.array([1.5, -2.1, 2.0, 0.0])
    slack = np.array([0.2, 0.5, 0.0, 1.0])
    got = _slack.slack_adjusted(dev, ref, slack)
    assert np.allclose(got, [1.3, -2.0, 2.0, 0.0])

