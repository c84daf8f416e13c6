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
