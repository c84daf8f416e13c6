"""CPU oracle for the KANLinear hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of torch-spline-kan's
KANLinear path (B-spline basis, its derivative, the SiLU + spline forward,
the analytic first-order backward, the fused mean|phi| edge statistic and
the entropy regulariser).  It is the checker the GPU kernels are compared
with; it is never the thing measured or shipped.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``torchsplinekan_amd``) never imports it.

Each function cites the reference file:line it follows (paths relative to
the torch-spline-kan source tree).  Every function computes in the dtype of
its inputs (float32 or float64) with the same elementwise operation order
as the reference, so float64 calls are the high-precision truth and float32
calls reproduce the reference backend's rounding of elementwise work.

How each function is pinned (tests/test_oracle.py):
  basis_dense       exact rational Cox-de Boor (fractions.Fraction) on small
                    grids; closed-form uniform B-splines for k = 1, 2, 3;
                    partition of unity, non-negativity, support, zeros out
                    of range; golden vectors written by the reference's own
                    compute_basis (tests/golden/), matched bit for bit in
                    float32 and exactly in float64.
  basis_local       agreement with basis_dense to 1e-13 in float64 over
                    uniform, nonuniform and repeated-knot grids, including
                    points on every knot and out of range.
  basis_derivative  central finite differences of basis_dense in float64
                    away from knots; exact cubic reproduction (x^3 - x).
  basis_derivative_n
                    q = 0, 1 identical to basis_dense / basis_derivative;
                    central finite differences of order q - 1 away from
                    knots; exact reproduction of polynomial derivatives
                    (6x and 6 for x^3, 2 for x^2 at k = 2); derivative rows
                    sum to zero inside the knot span (partition of unity);
                    zeros for q > k (tests/test_oracle_derivs.py).
  silu_derivative   q = 0, 1 identical to silu / silu_grad; central finite
                    differences of order q - 1.
  kan_edge_derivative
                    q = 0 summed over inputs equals kan_forward; central
                    finite differences of order q - 1 (all edges).
  kan_forward       brute-force per-(n,o) loop over the definition; config-1
                    golden vectors of the reference (tests/test_golden.py).
  kan_backward      finite differences of kan_forward (all four gradients);
                    config-1 golden vectors.
  edge_abs_mean     brute-force per-(n,o,i) loop.
  edge_abs_mean_by_feature
                    agreement with edge_abs_mean to 1e-13 in float64 (with
                    and without the base branch, on a feature subset).
  edge_abs_mean_backward
                    finite differences of edge_abs_mean away from phi = 0.
  regularization_from_edge_means (+ _grad)
                    closed form on hand-computed inputs; finite differences;
                    all-zero layer gives 0 with a finite zero gradient.
  grid_from_samples golden vectors of the reference's update_grid knots
                    (float32 bit-exact, float64); interior knots against the
                    quantile/uniform closed form; strictly increasing rows.
  curve2coeff       exact recovery of coefficients of curves that lie in the
                    new spline space; minimum-norm optimality conditions
                    (A^T(Ac - y) = 0, c orthogonal to null(A)) on a
                    rank-deficient case; golden vectors of update_grid.
  fit_spline_coeffs exact recovery (ridge -> 0) and the regularised normal
                    equations' residual; golden vectors of the reference's
                    fit_spline_coeffs.
  refit_gram        C coef^T against A^T y_old formed from the dense old curves.
"""

from fractions import Fraction

import numpy as np

__all__ = [
    "uniform_grid",
    "basis_dense",
    "basis_local",
    "basis_derivative",
    "basis_derivative_n",
    "silu",
    "silu_derivative",
    "kan_edge_derivative",
    "silu_grad",
    "kan_forward",
    "kan_backward",
    "kan_backward_params",
    "edge_abs_mean",
    "edge_abs_mean_by_feature",
    "edge_abs_mean_backward",
    "regularization_from_edge_means",
    "regularization_grad",
    "basis_fraction",
    "grid_from_samples",
    "refit_gram",
    "curve2coeff",
    "fit_spline_coeffs",
    "update_grid",
]


# ---------------------------------------------------------------------------
# knots
# ---------------------------------------------------------------------------

def uniform_grid(in_features, grid_size, spline_order, lo=-1.0, hi=1.0, dtype=np.float64):
    """Extended uniform knot rows [I, G+2k+1]: t_r = lo + ((r - k)(hi - lo))/G,
    evaluated in float32 in that order and then cast, as the reference builds
    the grid buffer (_build_uniform_grid, spline_kan/reference_backend.py:327-332)."""
    G, k = grid_size, spline_order
    r = np.arange(G + 2 * k + 1, dtype=np.float32)
    row = np.float32(lo) + ((r - np.float32(k)) * np.float32(hi - lo)) / np.float32(G)
    return np.repeat(row[None, :], in_features, axis=0).astype(dtype)


# ---------------------------------------------------------------------------
# basis
# ---------------------------------------------------------------------------

def _guarded_div(num, den):
    """num / den where den != 0, else 0 (den broadcast against num)."""
    nz = den != 0
    safe = np.where(nz, den, np.ones_like(den))
    return np.where(nz, num / safe, np.zeros_like(num))


def basis_dense(x, grid, k, chunk=1 << 14):
    """B-spline basis [N, I, G+k] by the dense Cox-de Boor recurrence.

    Follows compute_basis, spline_kan/reference_backend.py:62-94:
    degree 0 is the half-open indicator [t_r, t_{r+1}) with the last interval
    closed on the right; level d combines alpha*B_r + beta*B_{r+1} with
    alpha = (x - t_r)/(t_{r+d} - t_r), beta = (t_{r+d+1} - x)/(t_{r+d+1} - t_{r+1}),
    a zero denominator giving a zero coefficient.  The elementwise operation
    order is the reference's, so results carry its rounding in the input
    dtype.  Processed in sample chunks to bound memory.
    """
    x = np.asarray(x)
    grid = np.asarray(grid)
    dt = x.dtype
    N, I = x.shape
    nk = grid.shape[1]
    R = nk - k - 1
    out = np.empty((N, I, R), dtype=dt)
    t = grid[None, :, :].astype(dt)
    tl, tr = t[:, :, :-1], t[:, :, 1:]
    for n0 in range(0, N, chunk):
        xe = x[n0:n0 + chunk, :, None]
        b = ((xe >= tl) & (xe < tr)).astype(dt)
        last = ((xe >= tl[:, :, -1:]) & (xe <= tr[:, :, -1:])).astype(dt)
        b = np.concatenate([b[:, :, :-1], last], axis=-1)
        for d in range(1, k + 1):
            n = b.shape[-1] - 1
            t0, td = t[:, :, :n], t[:, :, d:d + n]
            t1, td1 = t[:, :, 1:1 + n], t[:, :, d + 1:d + 1 + n]
            den_l = td - t0
            den_r = td1 - t1
            alpha = _guarded_div(xe - t0, np.broadcast_to(den_l, (xe.shape[0],) + den_l.shape[1:]))
            beta = _guarded_div(td1 - xe, np.broadcast_to(den_r, (xe.shape[0],) + den_r.shape[1:]))
            b = alpha * b[:, :, :n] + beta * b[:, :, 1:n + 1]
        out[n0:n0 + chunk] = b
    return out


def _find_span(t, x):
    """Span m with t[m] <= x < t[m+1]; x == t[-1] gives the last span of
    non-zero length; -1 for x outside [t[0], t[-1]] or NaN.
    Follows find_span, csrc/kan_cuda.cu:207-221."""
    nk = len(t)
    if not (x >= t[0]) or x > t[nk - 1]:
        return -1
    if x == t[nk - 1]:
        m = nk - 2
        while m > 0 and t[m] == t[nk - 1]:
            m -= 1
        return m
    lo, hi = 0, nk - 1
    while hi - lo > 1:
        mid = (lo + hi) >> 1
        if t[mid] <= x:
            lo = mid
        else:
            hi = mid
    return lo


def _local_values(t, m, x, deg):
    """The deg+1 functions B_{m-deg+j, deg}(x), j = 0..deg, by the triangular
    scheme of Piegl & Tiller (The NURBS Book, algorithm A2.2) with clamped knot
    reads and zero-denominator guards.  Follows local_basis,
    csrc/kan_cuda.cu:230-271."""
    nk = len(t)
    dt = type(x)

    def T(idx):
        return t[0 if idx < 0 else (nk - 1 if idx > nk - 1 else idx)]

    v = [dt(1)] + [dt(0)] * deg
    for d in range(1, deg + 1):
        saved = dt(0)
        for j in range(d):
            rgt = T(m + j + 1) - x
            lft = x - T(m + 1 - d + j)
            dd = rgt + lft
            tmp = v[j] / dd if dd != 0 else dt(0)
            v[j] = saved + rgt * tmp
            saved = lft * tmp
        v[d] = saved
    return v


def basis_local(x, grid, k):
    """B-spline basis [N, I, G+k] from the span search plus the k+1 active
    values (csrc/kan_cuda.cu:207-312), zero rows out of range and for NaN.
    Scalar loops: for small inputs only."""
    x = np.asarray(x)
    grid = np.asarray(grid).astype(x.dtype)
    N, I = x.shape
    nk = grid.shape[1]
    R = nk - k - 1
    out = np.zeros((N, I, R), dtype=x.dtype)
    for n in range(N):
        for i in range(I):
            t = grid[i]
            xv = x[n, i]
            m = _find_span(t, xv)
            if m < 0:
                continue
            v = _local_values(t, m, xv, k)
            for j in range(k + 1):
                r = m - k + j
                if 0 <= r < R:
                    out[n, i, r] = v[j]
    return out


def basis_derivative(x, grid, k, chunk=1 << 14):
    """dB_{r,k}/dx [N, I, G+k] = k (B_{r,k-1}/(t_{r+k}-t_r) - B_{r+1,k-1}/(t_{r+k+1}-t_{r+1})),
    zero-denominator terms dropped.  Follows compute_basis_derivative,
    spline_kan/reference_backend.py:99-125 (and csrc/kan_cpu.cpp:88-131)."""
    x = np.asarray(x)
    dt = x.dtype
    grid = np.asarray(grid).astype(dt)
    nk = grid.shape[1]
    R = nk - k - 1
    lower = basis_dense(x, grid, k - 1, chunk=chunk)
    t = grid[None]
    d1 = t[:, :, k:k + R] - t[:, :, :R]
    d2 = t[:, :, k + 1:k + 1 + R] - t[:, :, 1:1 + R]
    shp = (x.shape[0],) + d1.shape[1:]
    term1 = _guarded_div(lower[:, :, :R], np.broadcast_to(d1, shp))
    term2 = _guarded_div(lower[:, :, 1:R + 1], np.broadcast_to(d2, shp))
    return dt.type(k) * (term1 - term2)


def basis_derivative_n(x, grid, k, q, chunk=1 << 14):
    """q-th derivative D^q B_{r,k}(x) [N, I, G+k] (q >= 0).

    q = 0 is basis_dense and q = 1 is basis_derivative, operation for
    operation.  For q >= 1: the degree k-q basis, then q steps of the
    derivative recurrence for p = k-q+1 .. k,
        D^j B_{r,p} = p (D^(j-1) B_{r,p-1}/(t_{r+p}-t_r) - D^(j-1) B_{r+1,p-1}/(t_{r+p+1}-t_{r+1})),
    zero-denominator terms dropped.  q > k gives zeros (a degree-k piecewise
    polynomial).  This is the derivative autograd takes through the
    differentiable recurrences of compute_basis / compute_basis_derivative
    (spline_kan/reference_backend.py:69-125) when the reference records its
    backward (kan_backward_composite, csrc/kan_cpu.cpp:301-345; create_graph
    uses in tests/test_math_correctness.py:232-260)."""
    x = np.asarray(x)
    dt = x.dtype
    grid = np.asarray(grid).astype(dt)
    nk = grid.shape[1]
    R = nk - k - 1
    if q == 0:
        return basis_dense(x, grid, k, chunk=chunk)
    if q > k:
        return np.zeros((x.shape[0], x.shape[1], R), dtype=dt)
    cur = basis_dense(x, grid, k - q, chunk=chunk)
    t = grid[None]
    for p in range(k - q + 1, k + 1):
        n = nk - p - 1
        d1 = t[:, :, p:p + n] - t[:, :, :n]
        d2 = t[:, :, p + 1:p + 1 + n] - t[:, :, 1:1 + n]
        shp = (x.shape[0],) + d1.shape[1:]
        term1 = _guarded_div(cur[:, :, :n], np.broadcast_to(d1, shp))
        term2 = _guarded_div(cur[:, :, 1:n + 1], np.broadcast_to(d2, shp))
        cur = dt.type(p) * (term1 - term2)
    return cur


def silu_derivative(x, q):
    """q-th derivative of silu(x) = x sigmoid(x), q = 0..4, with s = sigmoid(x):
    q=1  s (1 + x (1 - s))              (silu_grad; csrc/kan_cpu.cpp:279-281)
    q=2  s (1 - s) (2 + x (1 - 2s))
    q=3  s (1 - s) (3 (1 - 2s) + x (1 - 6s + 6s^2))
    q=4  s (1 - s) (4 (1 - 6s + 6s^2) + x (1 - 2s) (1 - 12s + 12s^2))
    (from s' = s (1 - s))."""
    x = np.asarray(x)
    if q == 0:
        return silu(x)
    if q == 1:
        return silu_grad(x)
    s = 1.0 / (1.0 + np.exp(-x))
    if q == 2:
        return s * (1 - s) * (2 + x * (1 - 2 * s))
    if q == 3:
        return s * (1 - s) * (3 * (1 - 2 * s) + x * (1 - 6 * s + 6 * s * s))
    if q == 4:
        return s * (1 - s) * (4 * (1 - 6 * s + 6 * s * s)
                              + x * (1 - 2 * s) * (1 - 12 * s + 12 * s * s))
    raise ValueError("silu_derivative: q must be 0..4")


def kan_edge_derivative(x, grid, base_weight, spline_weight, spline_scaler, k, q):
    """phi^(q)[n, o, i] = bw[o,i] silu^(q)(x[n,i]) + sum_r Weff[o,i,r] D^q B_r(x[n,i]):
    the q-th x-derivative of every edge function of the layer (the terms whose
    sum over i is kan_forward for q = 0).  Dense [N, O, I]; small sizes only."""
    W = _eff_weight(np.asarray(spline_weight), spline_scaler)
    Hq = basis_derivative_n(x, grid, k, q)
    phi = np.einsum("oir,nir->noi", W, Hq)
    if base_weight is not None:
        phi = phi + np.asarray(base_weight)[None] * silu_derivative(x, q)[:, None, :]
    return phi


def basis_fraction(xv, knots, k):
    """Exact rational B-spline values [B_{0,k}(x) .. B_{R-1,k}(x)] of one
    point on one knot row by the Cox-de Boor definition (degree 0 half-open,
    last interval closed; zero denominators give zero).  Brute force on
    fractions.Fraction, used to pin basis_dense."""
    xv = Fraction(xv)
    t = [Fraction(v) for v in knots]
    n0 = len(t) - 1
    b = []
    for r in range(n0):
        inside = t[r] <= xv < t[r + 1]
        if r == n0 - 1:
            inside = t[r] <= xv <= t[r + 1]
        b.append(Fraction(1) if inside else Fraction(0))
    for d in range(1, k + 1):
        nb = []
        for r in range(len(b) - 1):
            dl = t[r + d] - t[r]
            dr = t[r + d + 1] - t[r + 1]
            a = (xv - t[r]) / dl if dl != 0 else Fraction(0)
            c = (t[r + d + 1] - xv) / dr if dr != 0 else Fraction(0)
            nb.append(a * b[r] + c * b[r + 1])
        b = nb
    return b


# ---------------------------------------------------------------------------
# forward / backward
# ---------------------------------------------------------------------------

def silu(x):
    """x * sigmoid(x) = x / (1 + exp(-x))."""
    return x / (x.dtype.type(1) + np.exp(-x))


def silu_grad(x):
    """d silu/dx = sigma(x) (1 + x (1 - sigma(x))) (csrc/kan_cpu.cpp:245-246)."""
    one = x.dtype.type(1)
    sg = one / (one + np.exp(-x))
    return sg * (one + x * (one - sg))


def _eff_weight(sw, scaler):
    return sw if scaler is None else sw * scaler[:, :, None]


def kan_forward(x, grid, base_weight, spline_weight, spline_scaler, k, basis=None):
    """(y [N, O], H [N, I, R]) with
    y = silu(x) base_weight^T + H (spline_weight * spline_scaler)^T.
    base_weight None: no base branch; spline_scaler None: no scaler.
    Follows kan_forward_cpu, csrc/kan_cpu.cpp:136-188."""
    N, I = x.shape
    O, _, R = spline_weight.shape
    H = basis_dense(x, grid, k) if basis is None else basis
    W = _eff_weight(spline_weight, spline_scaler)
    y = H.reshape(N, I * R) @ W.reshape(O, I * R).T
    if base_weight is not None:
        y = silu(x) @ base_weight.T + y
    return y, H


def kan_backward(D, x, grid, base_weight, spline_weight, spline_scaler, k, basis=None,
                 basis_deriv=None):
    """Analytic first-order backward -> (gx, gbw | None, gsw, gscaler | None):
      gbw     = D^T silu(x)
      DtH     = D^T H;  gsw = scaler * DtH;  gscaler = sum_r sw * DtH
      gx      = sum_r (D W)[n,i,r] dB_r/dx(x[n,i]) + (D bw) * silu'(x)
    Follows kan_backward_cpu, csrc/kan_cpu.cpp:193-290."""
    N, I = x.shape
    O, _, R = spline_weight.shape
    H = basis_dense(x, grid, k) if basis is None else basis
    gbw = D.T @ silu(x) if base_weight is not None else None
    DtH = (D.T @ H.reshape(N, I * R)).reshape(O, I, R)
    if spline_scaler is not None:
        gsw = spline_scaler[:, :, None] * DtH
        gsc = (spline_weight * DtH).sum(axis=2)
    else:
        gsw, gsc = DtH, None
    W = _eff_weight(spline_weight, spline_scaler)
    DW = (D @ W.reshape(O, I * R)).reshape(N, I, R)
    dB = basis_derivative(x, grid, k) if basis_deriv is None else basis_deriv
    gx = (DW * dB).sum(axis=2)
    if base_weight is not None:
        gx = gx + (D @ base_weight) * silu_grad(x)
    return gx, gbw, gsw, gsc


def kan_backward_params(D, x, base_weight, spline_weight, spline_scaler, basis):
    """Parameter gradients only (x without requires_grad) ->
    (gbw | None, gsw, gscaler | None), the same formulas as kan_backward
    (csrc/kan_cpu.cpp:219-241)."""
    N, I = x.shape
    O, _, R = spline_weight.shape
    gbw = D.T @ silu(x) if base_weight is not None else None
    DtH = (D.T @ basis.reshape(N, I * R)).reshape(O, I, R)
    if spline_scaler is not None:
        return gbw, spline_scaler[:, :, None] * DtH, (spline_weight * DtH).sum(axis=2)
    return gbw, DtH, None


# ---------------------------------------------------------------------------
# edge statistic and regulariser
# ---------------------------------------------------------------------------

def _phi_chunk(s, H, bw, W):
    """phi [n, O, I] = s[n,i] bw[o,i] + sum_r H[n,i,r] W[o,i,r] for a sample chunk."""
    phi = np.einsum("nir,oir->noi", H, W, optimize=True)
    if bw is not None:
        phi = s[:, None, :] * bw[None, :, :] + phi
    return phi


def edge_abs_mean(s, H, bw, W, chunk=256):
    """a[o,i] = (1/N) sum_n |s[n,i] bw[o,i] + sum_r H[n,i,r] W[o,i,r]| [O, I],
    chunked over samples (s, bw None: no base branch).  Follows
    edge_abs_mean_dense, spline_kan/reference_backend.py:128-146, and the
    statistic of csrc/kan_reg_cuda.cu:1-10."""
    N = H.shape[0]
    acc = np.zeros(W.shape[:2], dtype=np.float64 if H.dtype == np.float64 else H.dtype)
    for n0 in range(0, N, chunk):
        sc = s[n0:n0 + chunk] if s is not None else None
        acc += np.abs(_phi_chunk(sc, H[n0:n0 + chunk], bw, W)).sum(axis=0)
    return acc / H.dtype.type(N)


def edge_abs_mean_by_feature(s, H, bw, W, features=None, workers=8):
    """The statistic of edge_abs_mean, one input feature at a time: column i
    of a is (1/N) sum_n |[s_i | H_i] [bw_i | W_i]^T|, a [N, R+1] x [R+1, O]
    product per feature, the features spread over `workers` threads (numpy
    releases the GIL in the products and reductions).  Same arithmetic as
    edge_abs_mean (spline_kan/reference_backend.py:128-146) in a form whose
    cost is a few seconds at a network layer of 16384 samples x 512 x 512
    edges.  `features` selects columns (default all) -> a [O, len(features)]."""
    from concurrent.futures import ThreadPoolExecutor
    N, I, R = H.shape
    feats = list(range(I)) if features is None else list(features)
    dt = np.float64 if H.dtype == np.float64 else H.dtype

    def column(i):
        A = H[:, i, :]
        B = W[:, i, :]
        if bw is not None:
            A = np.concatenate([s[:, i:i + 1], A], axis=1)
            B = np.concatenate([bw[:, i:i + 1], B], axis=1)
        return np.abs(A @ B.T).sum(axis=0, dtype=dt)

    with ThreadPoolExecutor(max(1, workers)) as ex:
        cols = list(ex.map(column, feats))
    out = np.stack(cols, axis=1) if cols else np.zeros((W.shape[0], 0), dtype=dt)
    return out / dt(N)


def edge_abs_mean_backward(ga, s, H, bw, W, chunk=256):
    """Gradients of edge_abs_mean given grad_a [O, I] -> (ds | None, dH, dbw | None, dW),
    with g[n,o,i] = ga[o,i] sign(phi[n,o,i]) / N and sign(0) = 0:
      ds = sum_o g bw,  dH = sum_o g W,  dbw = sum_n g s,  dW = sum_n g H.
    Follows csrc/kan_reg_cuda.cu:25-28, 81-107 and 113-176."""
    N = H.shape[0]
    dt = H.dtype
    inv_n = dt.type(1) / dt.type(N)
    dH = np.empty_like(H)
    ds = np.empty_like(s) if s is not None else None
    dW = np.zeros_like(W)
    dbw = np.zeros_like(bw) if bw is not None else None
    for n0 in range(0, N, chunk):
        sc = s[n0:n0 + chunk] if s is not None else None
        Hc = H[n0:n0 + chunk]
        g = np.sign(_phi_chunk(sc, Hc, bw, W)) * (ga * inv_n)[None]
        dH[n0:n0 + chunk] = np.einsum("noi,oir->nir", g, W, optimize=True)
        dW += np.einsum("noi,nir->oir", g, Hc, optimize=True)
        if bw is not None:
            ds[n0:n0 + chunk] = (g * bw[None]).sum(axis=1)
            dbw += (g * sc[:, None, :]).sum(axis=0)
    return ds, dH, dbw, dW


def regularization_from_edge_means(a, reg_act, reg_entropy):
    """mu1 * A + mu2 * S with A = sum a, p = max(a / max(A, tiny), tiny),
    S = -sum p log p; tiny = smallest normal number of a's dtype.
    Follows spline_kan/reference_backend.py:149-170."""
    tiny = np.finfo(a.dtype).tiny
    A = a.sum()
    p = np.maximum(a / max(A, tiny), tiny)
    S = -(p * np.log(p)).sum()
    return reg_act * A + reg_entropy * S


def regularization_grad(a, reg_act, reg_entropy):
    """d(regularization_from_edge_means)/da [O, I], the derivative of the
    clamped formula (clamp passes gradient only where it is inactive)."""
    tiny = np.finfo(a.dtype).tiny
    A = a.sum()
    A_safe = max(A, tiny)
    q = a / A_safe
    p = np.maximum(q, tiny)
    dS_dp = -(np.log(p) + 1.0)
    dS_dq = np.where(q >= tiny, dS_dp, 0.0)
    # q = a / A_safe: dq_j/da_i = delta_ij / A_safe - a_j / A_safe^2 (when A > tiny)
    g = dS_dq / A_safe
    if A > tiny:
        g = g - (dS_dq * a).sum() / (A_safe * A_safe)
    return reg_act * np.ones_like(a) + reg_entropy * g


# ---------------------------------------------------------------------------
# knot update and least-squares refit (update_grid, extend_grid)
# ---------------------------------------------------------------------------

def grid_from_samples(x, G, k, grid_eps, margin=0.01):
    """Knot rows [I, G+2k+1] adapted to samples x [B, I]: G+1 interior knots
    (1 - grid_eps) * quantile + grid_eps * uniform over the margin-widened
    range, then k outer knots per side spaced (range)/G.  Quantiles are the
    linear interpolation between sorted samples at positions
    q * (B - 1), q = clamp(j (1 - grid_eps)/G + grid_eps/2, 0, 1).
    Follows spline_kan/reference_backend.py:384-439 (elementwise operation
    order kept; in the dtype of x)."""
    dt = x.dtype.type
    B = x.shape[0]
    xs = np.sort(x, axis=0)
    lo = xs[0] - dt(margin)
    hi = xs[-1] + dt(margin)
    # torch.linspace(0, 1, G+1): first half start + i*step, second half end - (n-1-i)*step
    step = dt(1.0) / dt(G)
    u = np.array([dt(i) * step if i < (G + 1) // 2 else dt(1.0) - dt(G - i) * step
                  for i in range(G + 1)], dtype=x.dtype)
    uniform = lo[None] + u[:, None] * (hi - lo)[None]
    q = (np.arange(G + 1, dtype=x.dtype) * dt((1.0 - grid_eps) / G) + dt(grid_eps / 2.0))
    q = np.clip(q, dt(0.0), dt(1.0))
    pos = q * dt(B - 1)
    i_lo = np.clip(pos.astype(np.int64), 0, B - 1)
    i_hi = np.clip(i_lo + 1, 0, B - 1)
    w = (pos - i_lo.astype(x.dtype))[:, None]
    quant = (dt(1.0) - w) * xs[i_lo] + w * xs[i_hi]
    inner = dt(1.0 - grid_eps) * quant + dt(grid_eps) * uniform
    ext = (hi - lo) / dt(G)
    left = inner[0][None] - np.arange(k, 0, -1, dtype=x.dtype)[:, None] * ext[None]
    right = inner[-1][None] + np.arange(1, k + 1, dtype=x.dtype)[:, None] * ext[None]
    return np.ascontiguousarray(np.concatenate([left, inner, right], axis=0).T)


def refit_gram(x, grid_old, grid_new, k):
    """Per-feature normal matrix G[i] = A_i^T A_i [I, Rn, Rn] and cross term
    C[i] = A_i^T Bold_i [I, Rn, Ro] in float64, with A / Bold the bases of
    x on grid_new / grid_old.  C[i] coef[o, i, :] equals the reference's
    A_i^T y_old for y_old[o, b, i] = sum_s coef[o, i, s] Bold[b, i, s]
    (spline_kan/reference_backend.py:199-202, 483-484)."""
    A = basis_dense(x, grid_new, k).astype(np.float64)
    Bo = basis_dense(x, grid_old, k).astype(np.float64)
    return np.einsum("bir,bis->irs", A, A), np.einsum("bir,bis->irs", A, Bo)


def curve2coeff(x, y, grid, k):
    """Minimum-norm least-squares coefficients [O, I, R] of the curves
    y [O, B, I] at x [B, I] on `grid`, per feature in float64, with the
    basis evaluated in the dtype of x (spline_kan/reference_backend.py:218-265;
    numpy's lstsq returns the same minimum-norm solution as torch's gelsy
    driver, with rank cut eps * max(B, R))."""
    A = basis_dense(x, grid, k).astype(np.float64)
    Y = y.astype(np.float64)
    O, I, R = Y.shape[0], A.shape[1], A.shape[2]
    out = np.zeros((O, I, R), dtype=np.float64)
    for i in range(I):
        sol = np.linalg.lstsq(A[:, i, :], Y[:, :, i].T, rcond=None)[0]    # [R, O]
        out[:, i, :] = sol.T
    return out.astype(x.dtype)


def fit_spline_coeffs(x, y, grid, k, ridge=1e-12):
    """Ridge-regularised normal-equation coefficients [O, I, R] with the
    basis in float64: Cholesky of A^T A + lam * (tr(A^T A)/R) I, lam = ridge,
    raised 1e3-fold (up to three times) while the factorisation fails, then a
    general solve (spline_kan/reference_backend.py:173-215)."""
    A = basis_dense(x.astype(np.float64), grid.astype(np.float64), k)
    Y = y.astype(np.float64)
    R = A.shape[-1]
    AtA = np.einsum("bir,bis->irs", A, A)
    Aty = np.einsum("bir,obi->iro", A, Y)
    scale = np.maximum(np.trace(AtA, axis1=1, axis2=2), 1e-300) / R
    lam = ridge
    sol = None
    for _ in range(4):
        M = AtA + (lam * scale)[:, None, None] * np.eye(R)[None]
        try:
            L = np.linalg.cholesky(M)
        except np.linalg.LinAlgError:
            lam *= 1e3
            continue
        z = np.linalg.solve(L, Aty)
        sol = np.linalg.solve(np.transpose(L, (0, 2, 1)), z)
        break
    if sol is None:
        sol = np.stack([np.linalg.lstsq(M[i], Aty[i], rcond=None)[0] for i in range(M.shape[0])])
    return np.transpose(sol, (2, 0, 1)).astype(x.dtype)


def update_grid(x, grid, spline_weight, G, k, grid_eps, margin=0.01):
    """(new_grid, new_spline_weight) of ReferenceKANLayer.update_grid: the
    old unscaled curves y_old = sum_r coef * H_old at x, refitted on
    grid_from_samples by curve2coeff (spline_kan/reference_backend.py:443-493)."""
    H_old = basis_dense(x, grid, k)
    y_old = np.einsum("oir,bir->obi", spline_weight, H_old).astype(x.dtype)
    new_grid = grid_from_samples(x, G, k, grid_eps, margin)
    return new_grid, curve2coeff(x, y_old, new_grid, k)
