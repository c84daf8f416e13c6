"""Oracle gradients of a regularised KAN layer with an explicit bound for the
terms whose sign fp32 cannot decide.

The edge statistic's backward uses g = ga sign(phi) / n.  Where |phi| is
within the rounding error of the device's float32 evaluation of phi, the
device may take the other sign (or zero) than the float64 oracle; nothing
else about the result depends on that choice.  These helpers compute, in
float64 from the oracle's functions:

* the rounding bound beta[n, o, i] = c u (|s bw| + sum_r |H W|), u = 2^-24,
  c = 2 (R + 1 + 16): the dot product of R + 1 terms in any order (gamma_{R+1})
  plus the device's own rounding of s = silu(x) and of the basis values
  (a few ulps each), doubled;
* the ambiguous set A = {|phi| <= beta}, whose terms get g = 0 in the oracle;
* per gradient entry, the slack: the largest change any sign choice on A can
  make, sum over A of |ga| / n times |operand|.

A device gradient passes when |device - oracle| <= tol max|oracle| + slack,
elementwise: the sign flips are accounted for exactly where they occur and
every other term is held to the tolerance.  The number of ambiguous terms is
returned so that tests can assert it is small.
"""

import numpy as np

from oracle import kan_oracle as ko

U32 = 2.0 ** -24


def rounding_factor(R, extra=16):
    """c of the bound beta = c u sum|terms|: twice gamma_{R+1}'s count plus
    `extra` ulps for operands the device computes itself (16 for s and H
    evaluated from x on the device; 0 when device and oracle share the
    operands exactly, as the raw edge ops do)."""
    return 2.0 * (R + 1 + extra)


def edge_terms(s, H, bw, W, n_idx, o_idx, i_idx):
    """phi and sum |terms| for index arrays broadcast against each other
    (s [N, I] or None, H [N, I, R], bw [O, I] or None, W [O, I, R])."""
    Hn = H[n_idx, i_idx]                  # [..., R]
    Wo = W[o_idx, i_idx]                  # [..., R]
    phi = (Hn * Wo).sum(-1)
    mag = np.abs(Hn * Wo).sum(-1)
    if bw is not None:
        sb = s[n_idx, i_idx] * bw[o_idx, i_idx]
        phi = phi + sb
        mag = mag + np.abs(sb)
    return phi, mag


def edge_param_grads(D, ga, s, H, bw, sw, sc, edges, extra=16, unit=U32):
    """Parameter gradients of y = s bw^T + <H, sw*sc> and of the edge
    statistic together, for sampled edges [(o, i), ...], over all samples:
    -> dict name -> (ref [E, ...], slack [E, ...]) for "spline_weight"
    [E, R], "spline_scaler" [E], "base_weight" [E], and the count of
    ambiguous terms.  D [N, O] = dL/dy (None: no output term), ga [O, I]
    = dL/da (None: no statistic); `unit` is the device's unit roundoff."""
    N, I, R = H.shape
    W = sw * sc[:, :, None]
    c = rounding_factor(R, extra) * unit
    out = {k: ([], []) for k in ("spline_weight", "spline_scaler", "base_weight")}
    n_amb = 0
    nn_ = np.arange(N)
    for o, i in edges:
        g = np.zeros(N) if D is None else D[:, o].copy()
        gA = np.zeros(N)
        if ga is not None:
            phi, mag = edge_terms(s, H, bw, W, nn_, np.full(N, o), np.full(N, i))
            amb = np.abs(phi) <= c * mag
            n_amb += int(amb.sum())
            S = np.sign(phi)
            S[amb] = 0.0
            g += ga[o, i] * S / N
            gA = np.abs(ga[o, i]) * amb / N
        Hi = H[:, i, :]
        dWe, slW = Hi.T @ g, np.abs(Hi).T @ gA
        out["spline_weight"][0].append(sc[o, i] * dWe)
        out["spline_weight"][1].append(abs(sc[o, i]) * slW)
        out["spline_scaler"][0].append(sw[o, i] @ dWe)
        out["spline_scaler"][1].append(np.abs(sw[o, i]) @ slW)
        if bw is not None:
            out["base_weight"][0].append(s[:, i] @ g)
            out["base_weight"][1].append(np.abs(s[:, i]) @ gA)
    res = {k: (np.array(v[0]), np.array(v[1])) for k, v in out.items() if v[0]}
    return res, n_amb


def edge_input_grads(D, ga, x, grid, k, s, H, bw, sw, sc, rows, extra=16, unit=U32):
    """Gradient with respect to the layer input x for sampled rows, through
    the layer output and the edge statistic: dx[n, i] = silu'(x)
    sum_o g bw + sum_r dB_r(x) sum_o g W, g = D[n, o] + ga sign(phi) / N
    -> (ref [len(rows), I], slack [len(rows), I], ambiguous count); `unit`
    is the device's unit roundoff."""
    N, I, R = H.shape
    W = sw * sc[:, :, None]
    O = W.shape[0]
    c = rounding_factor(R, extra) * unit
    xr = x[rows]
    dB = ko.basis_derivative(xr, grid, k)           # [n, I, R]
    sp = ko.silu_grad(xr)                           # [n, I]
    ref, slack = [], []
    n_amb = 0
    oo = np.arange(O)[:, None]
    ii = np.arange(I)[None, :]
    for j, n in enumerate(rows):
        g = np.zeros((O, I)) if D is None else np.repeat(D[n][:, None], I, axis=1)
        gA = np.zeros((O, I))
        if ga is not None:
            phi, mag = edge_terms(s, H, bw, W, np.full((O, I), n), np.broadcast_to(oo, (O, I)),
                                  np.broadcast_to(ii, (O, I)))
            amb = np.abs(phi) <= c * mag
            n_amb += int(amb.sum())
            S = np.sign(phi)
            S[amb] = 0.0
            g = g + ga * S / N
            gA = np.abs(ga) * amb / N
        gW = np.einsum("oi,oir->ir", g, W)
        sW = np.einsum("oi,oir->ir", gA, np.abs(W))
        r = (dB[j] * gW).sum(-1)
        sl = (np.abs(dB[j]) * sW).sum(-1)
        if bw is not None:
            r = r + sp[j] * (g * bw).sum(0)
            sl = sl + np.abs(sp[j]) * (gA * np.abs(bw)).sum(0)
        ref.append(r)
        slack.append(sl)
    return np.array(ref), np.array(slack), n_amb


def edge_operand_grads(ga, s, H, bw, W, rows, n_total=None, extra=16):
    """Gradients of the edge statistic with respect to its sample operands on
    sampled rows: ds[n, i] = sum_o g bw, dH[n, i, r] = sum_o g W, with
    g = ga sign(phi) / N -> (ds_ref, ds_slack, dH_ref, dH_slack, ambiguous
    count); ds entries are None without a base branch.  s and H may hold
    only some rows of the statistic's samples: N is then n_total."""
    N, I, R = H.shape
    N = N if n_total is None else n_total
    O = W.shape[0]
    c = rounding_factor(R, extra) * U32
    oo = np.broadcast_to(np.arange(O)[:, None], (O, I))
    ii = np.broadcast_to(np.arange(I)[None, :], (O, I))
    ds, dss, dH, dHs = [], [], [], []
    n_amb = 0
    for n in rows:
        phi, mag = edge_terms(s, H, bw, W, np.full((O, I), n), oo, ii)
        amb = np.abs(phi) <= c * mag
        n_amb += int(amb.sum())
        S = np.sign(phi)
        S[amb] = 0.0
        g = ga * S / N
        gA = np.abs(ga) * amb / N
        dH.append(np.einsum("oi,oir->ir", g, W))
        dHs.append(np.einsum("oi,oir->ir", gA, np.abs(W)))
        if bw is not None:
            ds.append((g * bw).sum(0))
            dss.append((gA * np.abs(bw)).sum(0))
    arr = lambda v: np.array(v) if v else None
    return arr(ds), arr(dss), np.array(dH), np.array(dHs), n_amb


def edge_backward_full(ga, s, H, bw, W, D=None, chunk=256, extra=16, unit=U32):
    """All four gradients of the edge statistic (plus, with D = dL/dy, of the
    layer output y = s bw^T + <H, W>) with their slack, chunked over samples
    like ko.edge_abs_mean_backward: -> (ds, dH, dbw, dW) refs, the same four
    slacks (ds / dbw None without a base branch) and the ambiguous count.
    `unit` is the device's unit roundoff (2^-24 for float32, 2^-53 for
    float64)."""
    N, I, R = H.shape
    c = rounding_factor(R, extra) * unit
    dH, sH = np.empty_like(H), np.empty_like(H)
    dW, sW = np.zeros_like(W), np.zeros_like(W)
    hb = bw is not None
    ds = np.empty_like(s) if hb else None
    sds = np.empty_like(s) if hb else None
    dbw = np.zeros_like(bw) if hb else None
    sbw = np.zeros_like(bw) if hb else None
    n_amb = 0
    aW, abw = np.abs(W), (np.abs(bw) if hb else None)
    for n0 in range(0, N, chunk):
        Hc = H[n0:n0 + chunk]
        sc = s[n0:n0 + chunk] if hb else None
        phi = np.einsum("nir,oir->noi", Hc, W, optimize=True)
        mag = np.einsum("nir,oir->noi", np.abs(Hc), aW, optimize=True)
        if hb:
            sb = sc[:, None, :] * bw[None]
            phi = phi + sb
            mag = mag + np.abs(sb)
        amb = np.abs(phi) <= c * mag
        n_amb += int(amb.sum())
        S = np.sign(phi)
        S[amb] = 0.0
        g = S * (ga / N)[None]
        if D is not None:
            g = g + D[n0:n0 + chunk, :, None]
        gA = amb * (np.abs(ga) / N)[None]
        dH[n0:n0 + chunk] = np.einsum("noi,oir->nir", g, W, optimize=True)
        sH[n0:n0 + chunk] = np.einsum("noi,oir->nir", gA, aW, optimize=True)
        dW += np.einsum("noi,nir->oir", g, Hc, optimize=True)
        sW += np.einsum("noi,nir->oir", gA, np.abs(Hc), optimize=True)
        if hb:
            ds[n0:n0 + chunk] = (g * bw[None]).sum(axis=1)
            sds[n0:n0 + chunk] = (gA * abw[None]).sum(axis=1)
            dbw += (g * sc[:, None, :]).sum(axis=0)
            sbw += (gA * np.abs(sc)[:, None, :]).sum(axis=0)
    return (ds, dH, dbw, dW), (sds, sH, sbw, sW), n_amb


def layer_grads_full(D, ga, x, grid, k, s, H, bw, sw, sc, need_dx=True, extra=16, unit=U32,
                     workers=16):
    """Every gradient of one regularised layer step, over all samples and
    edges, with its slack: the layer output y = s bw^T + <H, sw*sc> with
    D = dL/dy [N, O] (None: no output term) and its edge statistic with
    ga = dL/da [O, I] (None: no statistic).  Feature by feature (the [N, O]
    tensors of phi, its rounding bound, g = D + ga sign(phi) / N with 0 on
    the ambiguous set, and the slack weight |ga| / N on that set, contracted
    with the feature's operands), features in threads with one BLAS thread
    each.  -> ({name: (ref, slack)} for "base_weight" [O, I] (with a base
    branch), "spline_weight" [O, I, R], "spline_scaler" [O, I] and, with
    need_dx, "x" [N, I]; the ambiguous count)."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits
    N, I, R = H.shape
    O = sw.shape[0]
    W = sw * sc[:, :, None]
    c = rounding_factor(R, extra) * unit
    hb = bw is not None
    out = {"spline_weight": (np.empty((O, I, R)), np.empty((O, I, R))),
           "spline_scaler": (np.empty((O, I)), np.empty((O, I)))}
    if hb:
        out["base_weight"] = (np.empty((O, I)), np.empty((O, I)))
    if need_dx:
        out["x"] = (np.empty((N, I)), np.empty((N, I)))
        sp = ko.silu_grad(x)

    def one(i):
        Hi, Wi = H[:, i, :], W[:, i, :]
        aH, aW = np.abs(Hi), np.abs(Wi)
        g = np.zeros((N, O)) if D is None else D.copy()
        gA = np.zeros((N, O))
        n_amb = 0
        if ga is not None:
            phi = Hi @ Wi.T
            mag = aH @ aW.T
            if hb:
                sb = np.outer(s[:, i], bw[:, i])
                phi += sb
                mag += np.abs(sb)
            amb = np.abs(phi) <= c * mag
            n_amb = int(amb.sum())
            S = np.sign(phi)
            S[amb] = 0.0
            g += S * (ga[:, i] / N)[None, :]
            gA = amb * (np.abs(ga[:, i]) / N)[None, :]
        dWi, sWi = g.T @ Hi, gA.T @ aH
        out["spline_weight"][0][:, i] = sc[:, i, None] * dWi
        out["spline_weight"][1][:, i] = np.abs(sc[:, i, None]) * sWi
        out["spline_scaler"][0][:, i] = (sw[:, i, :] * dWi).sum(1)
        out["spline_scaler"][1][:, i] = (np.abs(sw[:, i, :]) * sWi).sum(1)
        if hb:
            out["base_weight"][0][:, i] = g.T @ s[:, i]
            out["base_weight"][1][:, i] = gA.T @ np.abs(s[:, i])
        if need_dx:
            dB = ko.basis_derivative(x[:, i:i + 1], grid[i:i + 1], k)[:, 0, :]
            r = (dB * (g @ Wi)).sum(1)
            sl = (np.abs(dB) * (gA @ aW)).sum(1)
            if hb:
                r += sp[:, i] * (g @ bw[:, i])
                sl += np.abs(sp[:, i]) * (gA @ np.abs(bw[:, i]))
            out["x"][0][:, i] = r
            out["x"][1][:, i] = sl
        return n_amb

    with threadpool_limits(limits=1, user_api="blas"):
        with ThreadPoolExecutor(max(1, workers)) as ex:
            n_amb = sum(ex.map(one, range(I)))
    return out, n_amb


def slack_adjusted(dev, ref, slack):
    """dev with each entry's difference from ref shrunk by its slack (to ref
    itself where |dev - ref| <= slack), for blockwise error measures."""
    dev = np.asarray(dev, dtype=np.float64)
    d = dev - ref
    return ref + np.sign(d) * np.maximum(np.abs(d) - slack, 0.0)


def within(dev, ref, slack, tol):
    """max over entries of (|dev - ref| - slack) / max|ref| (<= tol passes)."""
    dev = np.asarray(dev, dtype=np.float64)
    scale = np.abs(ref).max()
    if scale == 0.0:
        return float(np.max(np.abs(dev) - slack, initial=0.0))
    return float(np.max((np.abs(dev - ref) - slack) / scale, initial=0.0))
