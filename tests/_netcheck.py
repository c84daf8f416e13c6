"""Layer-by-layer oracle check of one training step of a regularised KAN
(forward_with_regularization + loss + backward) on the device.

capture(net) records, for every layer, its input, its output and its
regulariser as the step runs (gradients of hidden tensors retained).
check_layers() then holds each layer to the fp64 oracle given that layer's
own device input (exact float32 values) and the device's gradient of its
output:
  * outputs on sampled rows (full=True: every row);
  * the regulariser, from the oracle's edge means over every edge;
  * parameter gradients on sampled edges over all samples, and the input
    gradient on sampled rows (full=True: every edge and row, block by
    block), through both the layer output and the edge statistic, with sign
    flips of phi at the device's rounding level bounded term by term
    (tests/_slack.py).
Each link of the chain is checked, so the whole backward is: the gradient
a layer receives is the previous check's input gradient.
"""

import contextlib
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from oracle import kan_oracle as ko
from tests import _slack
from tests._util import normwise, np64

WORKERS = max(1, min(16, os.cpu_count() or 1))


def basis_threaded(x, grid, k, chunk=32):
    """ko.basis_dense over feature chunks in threads (numpy releases the GIL)."""
    I = x.shape[1]
    parts = [(i, min(i + chunk, I)) for i in range(0, I, chunk)]
    with ThreadPoolExecutor(WORKERS) as ex:
        cols = list(ex.map(lambda p: ko.basis_dense(x[:, p[0]:p[1]], grid[p[0]:p[1]], k), parts))
    return np.concatenate(cols, axis=1)


def edge_means_threaded(s, H, bw, W):
    """ko.edge_abs_mean_by_feature with one BLAS thread per worker (the
    per-feature products are small; nested BLAS threads would oversubscribe)."""
    from threadpoolctl import threadpool_limits
    with threadpool_limits(limits=1, user_api="blas"):
        return ko.edge_abs_mean_by_feature(s, H, bw, W, workers=WORKERS)


def sample_edges(O, I, n, seed):
    r = np.random.default_rng(seed)
    e = {(0, 0), (O - 1, I - 1)}
    while len(e) < min(n, O * I):
        e.add((int(r.integers(O)), int(r.integers(I))))
    return sorted(e)


def params(layer):
    return (np64(layer.grid), np64(layer.base_weight), np64(layer.spline_weight),
            np64(layer.spline_scaler))


@contextlib.contextmanager
def capture(net):
    """Records (input, output, regulariser) of every layer's
    forward_with_regularization while the block runs."""
    cap = []
    for layer in net.layers:
        orig = layer.forward_with_regularization

        def wrapped(x, *a, _orig=orig, **kw):
            if x.requires_grad:
                x.retain_grad()
            y, r = _orig(x, *a, **kw)
            if y.requires_grad:
                y.retain_grad()
            cap.append((x, y, r))
            return y, r

        layer.forward_with_regularization = wrapped
    try:
        yield cap
    finally:
        for layer in net.layers:
            del layer.forward_with_regularization


def check_layers(net, cap, mu, k, tol, n_rows=32, n_edges=48, n_xrows=12, say=print,
                 amb_frac=1e-4, unit=_slack.U32, full=False):
    """Per-layer checks of a captured step (see the module docstring); returns
    the oracle's total regulariser.  Every check asserts against `tol`;
    `unit` is the device's unit roundoff (2^-24 float32, 2^-53 float64).
    full=True checks every row of y and dx and every edge of the parameter
    gradients instead of samples, block by block (_full_layer)."""
    reg_total = 0.0
    for li, (layer, (xl, yl, rl)) in enumerate(zip(net.layers, cap)):
        grid, bw, sw, sc = params(layer)
        x = np64(xl)
        N = x.shape[0]
        O, I = bw.shape
        s = ko.silu(x)
        H = basis_threaded(x, grid, k)
        if full:
            reg_total += _full_layer(li, layer, xl, yl, rl, x, s, H, mu, k, tol, say, amb_frac,
                                     unit)
            del H
            continue
        rows = np.unique(np.linspace(0, N - 1, n_rows).astype(int))
        ry, _ = ko.kan_forward(x[rows], grid, bw, sw, sc, k)
        e = normwise(np64(yl[rows]), ry)
        say(f"layer {li} ({I}->{O}): y rows {e:.2e}")
        assert e < tol
        W = sw * sc[:, :, None]
        a = edge_means_threaded(s, H, bw, W)
        r_ref = ko.regularization_from_edge_means(a, mu, mu)
        reg_total += r_ref
        r_dev = rl.item()
        e = abs(r_dev - r_ref) / abs(r_ref)
        say(f"layer {li}: regulariser {r_dev:.8g} vs {r_ref:.8g} ({e:.2e})")
        assert e < tol
        ga = ko.regularization_grad(a, mu, mu)
        D = np64(yl.grad)
        edges = sample_edges(O, I, n_edges, seed=li)
        res, n_amb = _slack.edge_param_grads(D, ga, s, H, bw, sw, sc, edges, unit=unit)
        oo, ii = map(list, zip(*edges))
        for name, key, got in (("dbase_w", "base_weight", layer.base_weight.grad[oo, ii]),
                               ("dcoef", "spline_weight", layer.spline_weight.grad[oo, ii]),
                               ("dscaler", "spline_scaler", layer.spline_scaler.grad[oo, ii])):
            ref, slack = res[key]
            e = _slack.within(np64(got), ref, slack, tol)
            say(f"layer {li}: {name} on {len(edges)} edges {e:.2e} "
                f"({n_amb} of {len(edges) * N} terms ambiguous)")
            assert e < tol, name
        assert n_amb <= max(3, amb_frac * len(edges) * N)
        if xl.requires_grad:
            xrows = rows[:n_xrows]
            ref, slack, n_amb = _slack.edge_input_grads(D, ga, x, grid, k, s, H, bw, sw, sc,
                                                        xrows, unit=unit)
            e = _slack.within(np64(xl.grad[xrows]), ref, slack, tol)
            say(f"layer {li}: dx on {len(xrows)} rows {e:.2e} "
                f"({n_amb} of {len(xrows) * O * I} terms ambiguous)")
            assert e < tol
            assert n_amb <= max(3, amb_frac * len(xrows) * O * I)
        del H
    return reg_total


def _full_layer(li, layer, xl, yl, rl, x, s, H, mu, k, tol, say, amb_frac, unit):
    """check_layers for one layer over every row and edge: y and dx in
    256 x 256 blocks, dcoef in 64-output x 16-feature blocks, dscaler and
    dbase_w in 64 x 64 blocks, each block's normwise error within tol after
    the slack of ambiguous signs (tests/_slack.py) is taken off entry by
    entry.  Returns the oracle's regulariser of the layer."""
    from tests._fullcheck import block_error
    grid, bw, sw, sc = params(layer)
    N = x.shape[0]
    O, I = bw.shape
    R = sw.shape[2]
    y_ref, _ = ko.kan_forward(x, grid, bw, sw, sc, k, basis=H)
    e, blk, whole = block_error(np64(yl), y_ref, 256, 256)
    say(f"layer {li} ({I}->{O}): y every row, whole {whole:.2e}, worst block {e:.2e} at {blk}")
    assert e < tol
    W = sw * sc[:, :, None]
    a = edge_means_threaded(s, H, bw, W)
    r_ref = ko.regularization_from_edge_means(a, mu, mu)
    e = abs(rl.item() - r_ref) / abs(r_ref)
    say(f"layer {li}: regulariser {rl.item():.8g} vs {r_ref:.8g} ({e:.2e})")
    assert e < tol
    ga = ko.regularization_grad(a, mu, mu)
    D = np64(yl.grad)
    res, n_amb = _slack.layer_grads_full(D, ga, x, grid, k, s, H, bw, sw, sc,
                                         need_dx=xl.requires_grad, unit=unit, workers=WORKERS)
    checks = [("dbase_w", layer.base_weight.grad, "base_weight", (64, 64)),
              ("dcoef", layer.spline_weight.grad, "spline_weight", (64, 16 * R)),
              ("dscaler", layer.spline_scaler.grad, "spline_scaler", (64, 64))]
    if xl.requires_grad:
        checks.append(("dx", xl.grad, "x", (256, 256)))
    for name, got, key, (bm, bn) in checks:
        ref, slack = res[key]
        adj = _slack.slack_adjusted(np64(got), ref, slack)
        e, blk, whole = block_error(adj.reshape(ref.shape[0], -1), ref.reshape(ref.shape[0], -1),
                                    bm, bn)
        say(f"layer {li}: {name} every entry, whole {whole:.2e}, worst block {e:.2e} at {blk} "
            f"({n_amb} of {N * O * I} terms ambiguous)")
        assert e < tol, name
    assert n_amb <= max(3, amb_frac * N * O * I)
    return r_ref

