"""Whole-tensor oracle check of one training step of a single KANLinear at
full workload size (c3, c5): every element of y, dx, dcoef, dscaler and
dbase_w against the fp64 oracle, in sample chunks that bound host memory.

The oracle's kan_forward / kan_backward run per chunk of rows; y and dx are
row-local, and the parameter gradients are sums over samples, so the chunks'
parameter gradients add up to the whole batch's.  Each tensor is compared
block by block (normwise relative error of every block, the worst block
reported): a fault confined to one output tile of a kernel's schedule shows
in its block even where the whole-tensor norm would dilute it.
"""

import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from oracle import kan_oracle as ko
from tests._netcheck import WORKERS, basis_threaded
from tests._util import np64


def deriv_threaded(x, grid, k, chunk=32):
    """ko.basis_derivative over feature chunks in threads."""
    I = x.shape[1]
    parts = [(i, min(i + chunk, I)) for i in range(0, I, chunk)]
    with ThreadPoolExecutor(WORKERS) as ex:
        cols = list(ex.map(lambda p: ko.basis_derivative(x[:, p[0]:p[1]], grid[p[0]:p[1]], k),
                           parts))
    return np.concatenate(cols, axis=1)


def _block_sums(a2, bm, bn):
    """Sum of squares of a 2-D array over blocks of bm x bn (ragged edges
    form smaller blocks)."""
    sq = np.square(a2)
    rows = np.add.reduceat(sq, np.arange(0, a2.shape[0], bm), axis=0)
    return np.add.reduceat(rows, np.arange(0, a2.shape[1], bn), axis=1)


def block_error(got, ref, bm, bn):
    """(worst blockwise normwise relative error, its block index, whole-tensor
    error).  A block whose reference norm is below 1 % of the root-mean-square
    block norm is measured against that floor instead."""
    got = np.asarray(got, dtype=np.float64).reshape(got.shape[0], -1)
    ref = np.asarray(ref, dtype=np.float64).reshape(ref.shape[0], -1)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), "non-finite values"
    num = _block_sums(got - ref, bm, bn)
    den = _block_sums(ref, bm, bn)
    floor = 1e-4 * den.mean()          # (1 % of the RMS block norm)^2
    err = np.sqrt(num / np.maximum(den, floor))
    worst = np.unravel_index(int(np.argmax(err)), err.shape)
    whole = float(np.sqrt(num.sum() / den.sum()))
    return float(err[worst]), (int(worst[0]) * bm, int(worst[1]) * bn), whole


def check_layer_step(layer, x_cpu, y_dev, gx_dev, D, k, say, chunk=None):
    """Errors of every output of one layer step against the oracle.

    layer: the KANLinear after backward (its .grad fields filled); x_cpu the
    float32 input on the host; y_dev / gx_dev the device output and input
    gradient (gx_dev may be None); D the float64 gradient of the loss with
    respect to y.  Returns {name: (worst block error, block, whole error)}."""
    t0 = time.time()
    grid = np64(layer.grid)
    bw, sw, sc = np64(layer.base_weight), np64(layer.spline_weight), np64(layer.spline_scaler)
    x = x_cpu.detach().double().numpy()
    N, I = x.shape
    O, _, R = sw.shape
    if chunk is None:       # about 1 GB of float64 basis per chunk
        chunk = max(256, min(4096, (1 << 27) // (I * R)))
    y_got = np64(y_dev)
    gx_got = np64(gx_dev) if gx_dev is not None else None
    y_ref = np.empty((N, O))
    gx_ref = np.empty((N, I)) if gx_dev is not None else None
    gbw = np.zeros((O, I))
    gsw = np.zeros_like(sw)
    gsc = np.zeros((O, I))
    for n0 in range(0, N, chunk):
        n1 = min(n0 + chunk, N)
        xc = x[n0:n1]
        H = basis_threaded(xc, grid, k)
        y_ref[n0:n1] = ko.kan_forward(xc, grid, bw, sw, sc, k, basis=H)[0]
        if gx_ref is not None:
            dB = deriv_threaded(xc, grid, k)
            cx, cbw, csw, csc = ko.kan_backward(D[n0:n1], xc, grid, bw, sw, sc, k, basis=H,
                                                basis_deriv=dB)
            gx_ref[n0:n1] = cx
        else:
            cbw, csw, csc = ko.kan_backward_params(D[n0:n1], xc, bw, sw, sc, H)
        gbw += cbw
        gsw += csw
        gsc += csc
        if (n0 // chunk) % 4 == 3:
            say(f"oracle rows {n1}/{N}, {time.time() - t0:.1f} s")
    say(f"oracle over {N} rows in {time.time() - t0:.1f} s")
    out = {"y": block_error(y_got, y_ref, 256, 256)}
    if gx_ref is not None:
        out["dx"] = block_error(gx_got, gx_ref, 256, 256)
    out["dcoef"] = block_error(np64(layer.spline_weight.grad).reshape(O, I * R),
                               gsw.reshape(O, I * R), 64, 16 * R)
    out["dscaler"] = block_error(np64(layer.spline_scaler.grad), gsc, 64, 64)
    out["dbase_w"] = block_error(np64(layer.base_weight.grad), gbw, 64, 64)
    return out


def check_edge_full(x, grid, k, bw, W, ga, dev, extra=16, unit=None, rows_per_block=256,
                    outs_per_block=64):
    """Every element of the edge statistic a [O, I] and of its backward
    (ds [N, I], dH [N, I, R], dbw [O, I], dW [O, I, R]) against the oracle,
    one input feature at a time: the oracle's basis of that feature from x,
    phi = [s_i | H_i] [bw_i | W_i]^T, g = ga sign(phi) / N with 0 on the
    set of ambiguous signs, and each entry's slack for those signs taken off
    (tests/_slack.py).  dev holds the device results as host arrays under
    "a", "ds", "dH", "dbw", "dW".  Each tensor is held block by block: a
    block is one feature's rows_per_block samples (ds, dH) or outs_per_block
    outputs (a, dbw, dW), with the floor of block_error.  Features run in
    threads with one BLAS thread each, so nothing of size [N, I, R] is formed
    on the host beyond dev itself.  -> ({name: (worst block error,
    (first row or output of the block, feature), whole-tensor error)},
    ambiguous count)."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits
    from tests import _slack
    unit = _slack.U32 if unit is None else unit
    N, I = x.shape
    O, _, R = W.shape
    c = _slack.rounding_factor(R, extra) * unit
    bsz = {"a": outs_per_block, "ds": rows_per_block, "dH": rows_per_block,
           "dbw": outs_per_block, "dW": outs_per_block}
    extent = {"a": O, "ds": N, "dH": N, "dbw": O, "dW": O}
    num = {name: np.zeros((-(-extent[name] // bs), I)) for name, bs in bsz.items()}
    den = {name: np.zeros_like(num[name]) for name in bsz}

    def blocks(a2, bs):
        """Sums of squares of a over blocks of bs leading indices."""
        rows = np.square(a2).reshape(a2.shape[0], -1).sum(1)
        return np.add.reduceat(rows, np.arange(0, a2.shape[0], bs))

    def one(i):
        Hi = ko.basis_dense(x[:, i:i + 1], grid[i:i + 1], k)[:, 0, :]
        si = ko.silu(x[:, i])
        Wi, bwi = W[:, i, :], bw[:, i]
        sb = np.outer(si, bwi)
        phi = Hi @ Wi.T + sb
        mag = np.abs(Hi) @ np.abs(Wi).T + np.abs(sb)
        amb = np.abs(phi) <= c * mag
        S = np.sign(phi)
        S[amb] = 0.0
        g = S * (ga[:, i] / N)[None, :]
        gA = amb * (np.abs(ga[:, i]) / N)[None, :]
        refs = {"a": (np.abs(phi).sum(0) / N, 0.0, dev["a"][:, i]),
                "ds": (g @ bwi, gA @ np.abs(bwi), dev["ds"][:, i]),
                "dH": (g @ Wi, gA @ np.abs(Wi), dev["dH"][:, i, :]),
                "dbw": (g.T @ si, gA.T @ np.abs(si), dev["dbw"][:, i]),
                "dW": (g.T @ Hi, gA.T @ np.abs(Hi), dev["dW"][:, i, :])}
        for name, (ref, slack, got) in refs.items():
            adj = _slack.slack_adjusted(np.asarray(got, dtype=np.float64), ref, slack)
            num[name][:, i] = blocks(adj - ref, bsz[name])
            den[name][:, i] = blocks(ref, bsz[name])
        return int(amb.sum())

    with threadpool_limits(limits=1, user_api="blas"):
        with ThreadPoolExecutor(WORKERS) as ex:
            n_amb = sum(ex.map(one, range(I)))
    out = {}
    for name, bs in bsz.items():
        floor = 1e-4 * den[name].mean()
        err = np.sqrt(num[name] / np.maximum(den[name], floor))
        w = np.unravel_index(int(np.argmax(err)), err.shape)
        whole = float(np.sqrt(num[name].sum() / den[name].sum()))
        out[name] = (float(err[w]), (int(w[0]) * bs, int(w[1])), whole)
    return out, n_amb

