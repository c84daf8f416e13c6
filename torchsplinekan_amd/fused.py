"""Memory-lean building blocks of forward + activation regularisation
(mirrors spline_kan/fused.py).

The regulariser needs the per-edge L1 norm (KAN paper eq. 19)

    a[o, i] = mean_n | s[n,i] bw[o,i] + sum_r H[n,i,r] W[o,i,r] |

with s = base_activation(x), H the B-spline basis of x and W the effective
spline weight.  ``EdgeAbsMean`` evaluates it on the gfx950 kernels without
storing the [N, O, I] edge tensor; its backward recomputes phi to get
sign(phi).  ``NativeBasis`` evaluates H on the device; its backward contracts
the incoming gradient with dB/dx in registers.  When the backward itself is
recorded (create_graph=True), NativeBasis's backward is the native
DerivContract (differentiable to any order on the device kernels) and
EdgeAbsMean's is the native EdgeAbsMeanBackward, whose own backward runs the
double-backward kernels at the fixed sign pattern; higher-order derivatives
stay exact without the dense [N, O, I] tensors of the reference's recorded
path (fused.py:43-102 of the reference).
"""

from typing import Optional

import torch

from .reference_backend import compute_basis, compute_basis_derivative

try:
    from . import _C
    HAS_FUSED_KERNELS = bool(getattr(_C, "HAS_FUSED_KERNELS", False))
except (ImportError, OSError):  # library not built
    _C = None
    HAS_FUSED_KERNELS = False


class NativeBasis(torch.autograd.Function):
    """H = basis(x) [B, I, R] on the device kernels."""

    @staticmethod
    def forward(ctx, x, grid, k: int):
        ctx.k = k
        ctx.save_for_backward(x, grid)
        return _C.basis(x, grid, k)

    @staticmethod
    def backward(ctx, gH):
        x, grid = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None
        if torch.is_grad_enabled():
            # recorded backward: the native contraction, itself differentiable
            return _C.deriv_contract(x, grid, gH, ctx.k, 1), None, None
        return _C.basis_grad(x.contiguous(), grid, ctx.k, gH.contiguous()), None, None


class NativeBasisSilu(torch.autograd.Function):
    """(s, H) = (silu(x), basis(x)) from one device pass over x, the two
    operands forward_with_regularization's native path takes from
    base_activation and the native basis separately
    (spline_kan/kan_linear.py:380-381).  The backward adds both inputs'
    contributions, sum_r gH dB_r/dx + gs silu'(x), in one pass as well;
    recorded backwards (create_graph) use the differentiable pieces."""

    @staticmethod
    def forward(ctx, x, grid, k: int):
        ctx.k = k
        ctx.save_for_backward(x, grid)
        return _C.basis_silu(x, grid, k)

    @staticmethod
    def backward(ctx, gs, gH):
        x, grid = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None
        B, I = x.shape
        if gs is None:
            gs = x.new_zeros(B, I)
        if gH is None:
            gH = x.new_zeros(B, I, grid.shape[1] - ctx.k - 1)
        if torch.is_grad_enabled():
            # recorded backward: spline and SiLU terms in one differentiable native call
            return _C.deriv_contract(x, grid, gH, ctx.k, 1, gs), None, None
        return _C.basis_silu_grad(x, grid, ctx.k, gH, gs), None, None


class EdgeAbsMean(torch.autograd.Function):
    """a[o,i] = mean_n |s*bw + <H, W>| without materialising [N, O, I]."""

    @staticmethod
    def forward(ctx, s, H, bw, W):
        has_base = bw is not None
        empty = H.new_empty(0)
        ctx.has_base = has_base
        ctx.save_for_backward(s if has_base else empty, H, bw if has_base else empty, W)
        return _C.edge_abs_mean(s if has_base else empty, H, bw if has_base else empty, W)

    @staticmethod
    def backward(ctx, ga):
        s, H, bw, W = ctx.saved_tensors
        has_base = ctx.has_base
        need_s, need_H, need_bw, need_W = ctx.needs_input_grad
        if torch.is_grad_enabled():
            # Recorded backward: a differentiable native function of the
            # saved tensors themselves (mixed input x weight terms kept),
            # whose own backward runs the native double-backward kernels.
            ds, dH, dbw, dW = _C.EdgeAbsMeanBackward.apply(
                ga, s if has_base else None, H, bw if has_base else None, W)
            return (ds if need_s and has_base else None, dH if need_H else None,
                    dbw if need_bw and has_base else None, dW if need_W else None)
        ds, dH, dbw, dW = _C.edge_abs_mean_backward(
            ga, s, H, bw, W, bool(need_s and has_base), bool(need_H),
            bool(need_bw and has_base), bool(need_W))
        return (ds if need_s and has_base else None, dH if need_H else None,
                dbw if need_bw and has_base else None, dW if need_W else None)


_CU_COUNT = {}


def _one_pass_forward(B: int, O: int, R: int, device) -> bool:
    """Whether EdgeLinear's forward takes y and a from one pass over phi
    (_C.edge_linear_forward, 128 x 128 sample x output blocks) rather than
    the edge statistic's kernel plus the engine's two output products:
    where the blocks fill the chip once (one per CU).  A sweep at G = 8
    (in_features 64-512, out_features 64-1024, N 2048-65536) found the one
    pass faster in every such case (time ratio 0.58-0.99; 512->512 at
    N = 16384: 1.56 -> 1.19 ms) and slower in nearly every other (512->64
    at N = 16384, 128 blocks: 0.28 -> 0.85 ms).  Its workspace (one partial
    row of the statistic per 128 samples, ceil(B / 128) * I * O values)
    grows with the batch, so it is taken only while that stays within the
    size of the basis H [B, I, R] the layer holds anyway (O <= 128 R)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    nblk = -(-B // 128)
    return nblk * -(-O // 128) >= _CU_COUNT[idx] and nblk * O <= B * R


class EdgeLinear(torch.autograd.Function):
    """(y, a) of one regularised layer from the same operands:
    y = s bw^T + H W^T (flattened over I and R) and a = mean_n |phi|.
    The reference builds them separately (two F.linear calls and EdgeAbsMean,
    spline_kan/kan_linear.py:384-387), so autograd runs the linear layer's
    gradient products, the edge statistic's backward and the sums of the two.
    Every one of those gradients is a contraction of
    g' = ga sign(phi) / n + dL/dy, so here a single native launch
    (_C.edge_linear_backward: dL/dy added to g inside the fused edge kernel)
    returns all four (only the weight gradients: the parameter kernel with
    dL/dy added the same way).  Recorded backwards (create_graph) use the
    separate differentiable pieces.  The forward of a wide layer takes y and
    a from one pass over phi as well (_C.edge_linear_forward: y is the sum
    over features of the edge values whose absolute means a holds)."""

    @staticmethod
    def forward(ctx, s, H, bw, W):
        B, I, R = H.shape
        O = W.shape[0]
        if _one_pass_forward(B, O, R, H.device) and _C.edge_linear_forward_supported(H, W):
            y, a = _C.edge_linear_forward(s, H, bw, W)
        else:
            y = _C.matmul(s, bw.t()) + _C.matmul(H.reshape(B, I * R), W.reshape(O, I * R).t())
            a = _C.edge_abs_mean(s, H, bw, W)
        ctx.save_for_backward(s, H, bw, W)
        return y, a

    @staticmethod
    def backward(ctx, gy, ga):
        s, H, bw, W = ctx.saved_tensors
        need_s, need_H, need_bw, need_W = ctx.needs_input_grad
        B, I, R = H.shape
        O = W.shape[0]
        if gy is None:
            gy = H.new_zeros(B, O)
        if ga is None:
            ga = H.new_zeros(O, I)
        H2, W2 = H.reshape(B, I * R), W.reshape(O, I * R)
        if torch.is_grad_enabled():
            # recorded backward: differentiable native pieces (as the
            # separate F.linear + EdgeAbsMean path records them)
            mm = _C.NativeMatmul.apply
            ds, dH, dbw, dW = _C.EdgeAbsMeanBackward.apply(ga, s, H, bw, W)
            ds = ds + mm(gy, bw) if need_s else None
            dH = dH + mm(gy, W2).reshape(B, I, R) if need_H else None
            dbw = dbw + mm(gy.t(), s) if need_bw else None
            dW = dW + mm(gy.t(), H2).reshape(O, I, R) if need_W else None
            return ds, dH, dbw, dW
        return _C.edge_linear_backward(ga, gy, s, H, bw, W, bool(need_s), bool(need_H),
                                       bool(need_bw), bool(need_W))


def _regularization_grad(a: torch.Tensor, g: torch.Tensor, mu1: float, mu2: float) -> torch.Tensor:
    """g * d reg / d a as differentiable tensor operations (the gradient that
    autograd takes through regularization_from_edge_means, clamps included:
    tc = max(T, tiny), m = [a / tc >= tiny], c = [T >= tiny],
    U = sum (log p + 1) m a, d reg / d a = mu1 + mu2 (c U / tc^2 - (log p + 1) m / tc))."""
    tiny = torch.finfo(a.dtype).tiny
    total = a.sum()
    tc = total.clamp(min=tiny)
    q = a / tc
    m = (q >= tiny).to(a.dtype)
    lp1 = q.clamp(min=tiny).log() + 1
    u = (lp1 * m * a).sum()
    c = (total >= tiny).to(a.dtype)
    return g * (mu1 + mu2 * (c * ((u / tc) / tc) - lp1 * m / tc))


class EdgeRegularization(torch.autograd.Function):
    """The layer regulariser mu1 * sum(a) + mu2 * entropy(a / sum(a)) from its
    edge means on the device: three native launches forward and one backward
    (kan_hip_edge_reg) in place of the ATen expression's ten and twenty
    (spline_kan/reference_backend.py:149-170).  A recorded backward
    (create_graph) takes the gradient as differentiable tensor operations."""

    @staticmethod
    def forward(ctx, a, mu1: float, mu2: float):
        reg, ws = _C.edge_regularization(a, mu1, mu2)
        ctx.save_for_backward(a)
        ctx.ws, ctx.mu = ws, (float(mu1), float(mu2))
        return reg

    @staticmethod
    def backward(ctx, g):
        a, = ctx.saved_tensors
        mu1, mu2 = ctx.mu
        if torch.is_grad_enabled():
            return _regularization_grad(a, g, mu1, mu2), None, None
        return _C.edge_regularization_backward(g, a, mu1, mu2, ctx.ws), None, None


def edge_regularization(a: torch.Tensor, mu1: float, mu2: float) -> torch.Tensor:
    """Regulariser of one layer's edge means a on the device (see
    EdgeRegularization)."""
    return EdgeRegularization.apply(a, mu1, mu2)


def edge_linear_applies(s: Optional[torch.Tensor], H: torch.Tensor, bw: Optional[torch.Tensor],
                        W: torch.Tensor) -> bool:
    """Whether edge_linear covers this layer: a base branch, and operands the
    folded native backward supports (float32, O <= 512, R + 1 <= 16;
    _C.edge_linear_supported)."""
    return (s is not None and bw is not None and _C is not None and H.is_cuda
            and _C.edge_linear_supported(H, W))


def edge_linear(s: torch.Tensor, H: torch.Tensor, bw: torch.Tensor, W: torch.Tensor):
    """(y [B, O], a [O, I]) of a regularised layer (see EdgeLinear)."""
    return EdgeLinear.apply(s, H, bw, W)


def native_basis(x: torch.Tensor, grid: torch.Tensor, k: int) -> torch.Tensor:
    return NativeBasis.apply(x, grid, k)


def native_basis_silu(x: torch.Tensor, grid: torch.Tensor, k: int):
    """(silu(x), basis(x)) of a device input in one pass (NativeBasisSilu)."""
    return NativeBasisSilu.apply(x, grid, k)


def edge_abs_mean(s: Optional[torch.Tensor], H: torch.Tensor, bw: Optional[torch.Tensor],
                  W: torch.Tensor) -> torch.Tensor:
    return EdgeAbsMean.apply(s, H, bw, W)


def native_linear(s: torch.Tensor, bw: torch.Tensor, H2: torch.Tensor,
                  W2: torch.Tensor) -> torch.Tensor:
    """Layer output s bw^T + H2 W2^T of the fused regularisation path, the two
    products the reference takes with F.linear (spline_kan/kan_linear.py:
    384-385), on the MFMA contraction engine (NativeMatmul: gradients are
    engine products as well, the long sample reductions split over K and
    summed in a fixed order)."""
    y = _C.NativeMatmul.apply(s, bw.t())
    return y + _C.NativeMatmul.apply(H2, W2.t())


class ChunkedEdgeAbsMean(torch.autograd.Function):
    """a[o, i] = mean_n |phi[n, o, i]| on any device with at most `chunk`
    samples' worth of phi (and of the basis) alive at once.  The forward
    accumulates sum_n |phi| chunk by chunk under no_grad and keeps only its
    inputs.  The backward visits the chunks again: it evaluates the chunk's
    basis, takes g = sign(phi) ga / N, and forms the four gradients in closed
    form (dW = sum_n g H, dbw = sum_n g s, ds = sum_o g bw, dx = sum_r
    (sum_o g W) dB_r/dx).  Those are differentiable operations on the saved
    inputs, so a recorded backward (create_graph) can be differentiated again;
    sign(phi) is constant almost everywhere and enters as data.  The reference
    bounds memory the same way through activation checkpointing
    (spline_kan/fused.py:114-137)."""

    @staticmethod
    def forward(ctx, x, s, bw, W, grid, k: int, chunk: int):
        N = x.shape[0]
        total = W.new_zeros(W.shape[:2])
        for lo in range(0, N, chunk):
            hi = min(lo + chunk, N)
            phi = _chunk_phi(x[lo:hi], None if s is None else s[lo:hi], grid, k, bw, W)
            total += phi.abs().sum(0)
        ctx.k, ctx.chunk = k, chunk
        ctx.save_for_backward(x, s, bw, W, grid)
        return total / N

    @staticmethod
    def backward(ctx, ga):
        x, s, bw, W, grid = ctx.saved_tensors
        k, chunk, N = ctx.k, ctx.chunk, x.shape[0]
        need_x, need_s, need_bw, need_W = ctx.needs_input_grad[:4]
        has_base = bw is not None
        dx, ds, dbw, dW = [], [], None, None
        for lo in range(0, N, chunk):
            hi = min(lo + chunk, N)
            xc = x[lo:hi]
            sc = s[lo:hi] if has_base else None
            Hc = compute_basis(xc, grid, k)
            with torch.no_grad():
                sgn = _chunk_phi(xc, sc, grid, k, bw, W, Hc).sign()
            g = sgn * (ga / N)                                           # [n, O, I]
            if need_W:
                part = torch.einsum("noi,nir->oir", g, Hc)
                dW = part if dW is None else dW + part
            if need_bw and has_base:
                part = torch.einsum("noi,ni->oi", g, sc)
                dbw = part if dbw is None else dbw + part
            if need_s and has_base:
                ds.append(torch.einsum("noi,oi->ni", g, bw))
            if need_x:
                gH = torch.einsum("noi,oir->nir", g, W)
                if k >= 1:
                    dx.append((gH * compute_basis_derivative(xc, grid, k)).sum(-1))
                else:                        # piecewise constant basis: dB/dx = 0
                    dx.append(torch.zeros_like(xc))
        return (torch.cat(dx) if need_x else None,
                torch.cat(ds) if need_s and has_base else None,
                dbw, dW, None, None, None)


def _chunk_phi(xc, sc, grid, k, bw, W, Hc=None):
    """phi [n, O, I] of a sample chunk: sc bw + <basis(xc), W>."""
    if Hc is None:
        Hc = compute_basis(xc, grid, k)
    phi = torch.einsum("nir,oir->noi", Hc, W)
    if bw is not None:
        phi = phi + sc[:, None, :] * bw[None]
    return phi


def edge_abs_mean_chunked(s: Optional[torch.Tensor], x: torch.Tensor, grid: torch.Tensor, k: int,
                          bw: Optional[torch.Tensor], W: torch.Tensor,
                          chunk_size: int) -> torch.Tensor:
    """Low-memory edge statistic on any device (reg_impl="checkpoint"):
    ChunkedEdgeAbsMean over chunks of chunk_size samples."""
    return ChunkedEdgeAbsMean.apply(x, s if bw is not None else None, bw, W, grid, k,
                                    chunk_size)
