"""Pure-PyTorch B-spline KAN layer: the ``backend="reference"`` path.

This is the backend a KANLinear uses for CPU inputs (``backend="auto"``) or
when asked explicitly; it mirrors spline_kan/reference_backend.py of
torch-spline-kan (same functions, argument meanings and results).  Device
tensors never reach it silently: the native backend either runs the HIP
kernels or raises.

Conventions (reference_backend.py:1-22 of the reference):
  extended knots  t_r = a + (r - k)(b - a)/G,  r = 0..G+2k  (per feature row)
  basis count     R = G + k
  degree 0        B_{r,0}(x) = [t_r <= x < t_{r+1}], last interval closed
  recurrence      B_{r,d} = (x - t_r)/(t_{r+d} - t_r) B_{r,d-1}
                          + (t_{r+d+1} - x)/(t_{r+d+1} - t_{r+1}) B_{r+1,d-1}
                  with zero denominators contributing zero
  edge function   phi_{o,i}(u) = bw[o,i] act(u) + scaler[o,i] sum_r coef[o,i,r] B_r(u)
"""

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F


def _guarded_ratio(num: torch.Tensor, den: torch.Tensor) -> torch.Tensor:
    """num / den where den != 0, else 0 (den broadcast against num)."""
    nz = den != 0
    return torch.where(nz, num / torch.where(nz, den, torch.ones_like(den)),
                       torch.zeros_like(num))


def compute_basis(x: torch.Tensor, grid: torch.Tensor, k: int) -> torch.Tensor:
    """B-spline basis [B, I, G+k] of x [B, I] on knot rows grid [I, G+2k+1].

    Cox-de Boor recurrence (spline_kan/reference_backend.py:32-96): the
    degree-d level combines alpha*B_r + beta*B_{r+1} with
    alpha = (x - t_r)/(t_{r+d} - t_r), beta = (t_{r+d+1} - x)/(t_{r+d+1} - t_{r+1}).
    """
    if k not in (0, 1, 2, 3):
        raise ValueError(f"spline_order must be 0, 1, 2, or 3, got {k}")
    xe = x.unsqueeze(-1)                       # [B, I, 1]
    t = grid.unsqueeze(0)                      # [1, I, nk]
    lo, hi = t[..., :-1], t[..., 1:]
    cur = ((xe >= lo) & (xe < hi)).to(x.dtype)
    closed_last = ((xe >= lo[..., -1:]) & (xe <= hi[..., -1:])).to(x.dtype)
    cur = torch.cat([cur[..., :-1], closed_last], dim=-1)
    for d in range(1, k + 1):
        n = cur.shape[-1] - 1
        t_r, t_rd = t[..., :n], t[..., d:d + n]
        t_r1, t_rd1 = t[..., 1:1 + n], t[..., d + 1:d + 1 + n]
        alpha = _guarded_ratio(xe - t_r, t_rd - t_r)
        beta = _guarded_ratio(t_rd1 - xe, t_rd1 - t_r1)
        cur = alpha * cur[..., :n] + beta * cur[..., 1:n + 1]
    return cur


def compute_basis_derivative(x: torch.Tensor, grid: torch.Tensor, k: int) -> torch.Tensor:
    """dB_{r,k}/dx [B, I, G+k] from differentiable ops (so it can itself be
    differentiated): k*(B_{r,k-1}/(t_{r+k}-t_r) - B_{r+1,k-1}/(t_{r+k+1}-t_{r+1}))
    (spline_kan/reference_backend.py:99-125)."""
    if k < 1:
        raise ValueError("compute_basis_derivative requires spline_order >= 1")
    lower = compute_basis(x, grid, k - 1)      # [B, I, R+1]
    R = grid.shape[1] - k - 1
    t = grid.unsqueeze(0)
    d1 = t[..., k:k + R] - t[..., :R]
    d2 = t[..., k + 1:k + 1 + R] - t[..., 1:1 + R]
    return k * (_guarded_ratio(lower[..., :R], d1) - _guarded_ratio(lower[..., 1:R + 1], d2))


def edge_abs_mean_dense(s: Optional[torch.Tensor], H: torch.Tensor,
                        base_weight: Optional[torch.Tensor],
                        eff_weight: torch.Tensor) -> torch.Tensor:
    """a[o, i] = mean_n |s[n,i] bw[o,i] + sum_r H[n,i,r] W[o,i,r]|, through the
    materialised edge tensor phi [N, O, I] (any order of autograd)
    (spline_kan/reference_backend.py:128-146)."""
    spline = torch.einsum("oir,nir->noi", eff_weight, H)
    if base_weight is None:
        return spline.abs().mean(dim=0)
    phi = s.unsqueeze(1) * base_weight.unsqueeze(0) + spline
    return phi.abs().mean(dim=0)


def regularization_from_edge_means(a: torch.Tensor, regularize_activation: float,
                                   regularize_entropy: float) -> torch.Tensor:
    """mu1 * sum(a) + mu2 * entropy(a / sum(a)), with the smallest normal
    number as clamp so that an all-zero layer gives a finite zero gradient
    (KAN paper eqs. 20-21; spline_kan/reference_backend.py:149-170)."""
    total = a.sum()
    tiny = torch.finfo(a.dtype).tiny
    p = (a / total.clamp(min=tiny)).clamp(min=tiny)
    entropy = -(p * p.log()).sum()
    return regularize_activation * total + regularize_entropy * entropy


def curve2coeff(x_samples: torch.Tensor, y_samples: torch.Tensor, grid: torch.Tensor,
                k: int) -> torch.Tensor:
    """Least-squares spline coefficients [O, I, R] reproducing y [O, B, I] at
    x [B, I], solved per feature in float64 on the CPU with the minimum-norm
    solution for rank-deficient systems (spline_kan/reference_backend.py:218-265)."""
    A = compute_basis(x_samples, grid, k).to(device="cpu", dtype=torch.float64)   # [B, I, R]
    Y = y_samples.to(device="cpu", dtype=torch.float64)                            # [O, B, I]
    O, I, R = Y.shape[0], A.shape[1], A.shape[2]
    out = torch.zeros(O, I, R, dtype=torch.float64)
    for i in range(I):
        sol = torch.linalg.lstsq(A[:, i, :], Y[:, :, i].t()).solution             # [R, O]
        out[:, i, :] = sol.t()
    return out.to(dtype=x_samples.dtype, device=x_samples.device)


def ridge_solve(gram: torch.Tensor, rhs: torch.Tensor, ridge: float) -> torch.Tensor:
    """Solutions [I, R, M] of (G_i + lam * mean(diag G_i) * Id) X_i = rhs_i for a
    batch of symmetric positive semi-definite G [I, R, R] (float64).

    lam runs through the ladder ridge, 1e3 ridge, 1e6 ridge, 1e9 ridge and
    stops at the first rung where every G_i's shifted matrix factors by
    Cholesky; the batch shares one lam.  If none does, the top rung's systems
    are solved by least squares.  This is the shift schedule of the
    reference's fit (spline_kan/reference_backend.py:197-215)."""
    if ridge <= 0:
        raise ValueError(f"ridge must be positive, got {ridge}")
    R = gram.shape[-1]
    mean_diag = torch.diagonal(gram, dim1=-2, dim2=-1).sum(-1).clamp(min=1e-300) / R
    shifted = gram
    for rung in range(4):
        lam = ridge * 1e3 ** rung
        shifted = gram + torch.diag_embed((lam * mean_diag)[:, None].expand(-1, R))
        factor, info = torch.linalg.cholesky_ex(shifted)
        if int(info.count_nonzero()) == 0:
            return torch.cholesky_solve(rhs, factor)
    return torch.linalg.lstsq(shifted, rhs).solution


def fit_spline_coeffs(x_samples: torch.Tensor, y_samples: torch.Tensor, grid: torch.Tensor,
                      k: int, ridge: float = 1e-12) -> torch.Tensor:
    """Ridge-regularised least-squares coefficients [O, I, R] of the curves
    y [O, B, I] sampled at x [B, I] on the knot rows `grid`, in float64 on
    the samples' device: per feature, the normal equations A^T A c = A^T y of
    the float64 basis A [B, R], solved by ridge_solve
    (spline_kan/reference_backend.py:173-215)."""
    if ridge <= 0:
        raise ValueError(f"ridge must be positive, got {ridge}")
    basis = compute_basis(x_samples.double(), grid.double(), k).transpose(0, 1)   # [I, B, R]
    curves = y_samples.double().permute(2, 1, 0)                                 # [I, B, O]
    gram = basis.transpose(1, 2) @ basis                                         # [I, R, R]
    coeffs = ridge_solve(gram, basis.transpose(1, 2) @ curves, ridge)            # [I, R, O]
    return coeffs.permute(2, 0, 1).to(dtype=x_samples.dtype)


class ReferenceKANLayer(nn.Module):
    """Pure-PyTorch B-spline KAN layer (owns all parameters and the knot grid).

    Mirrors spline_kan.reference_backend.ReferenceKANLayer: same constructor,
    parameter names/shapes, initialisation recipe, forward and regulariser.
    """

    def __init__(self, in_features: int, out_features: int, grid_size: int = 5,
                 spline_order: int = 3, scale_noise: float = 0.1, scale_base: float = 1.0,
                 scale_spline: float = 1.0, enable_standalone_scale_spline: bool = True,
                 base_activation: nn.Module = nn.SiLU, grid_eps: float = 0.02,
                 grid_range: Tuple[float, float] = (-1.0, 1.0)) -> None:
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.grid_size = grid_size
        self.spline_order = spline_order
        self.scale_noise = scale_noise
        self.scale_base = scale_base
        self.scale_spline = scale_spline
        self.enable_standalone_scale_spline = enable_standalone_scale_spline
        self.grid_eps = grid_eps
        self.grid_range = grid_range
        self.base_activation = base_activation() if isinstance(base_activation, type) \
            else base_activation
        self.register_buffer("grid", self._uniform_grid(grid_range[0], grid_range[1]))
        R = grid_size + spline_order
        self.base_weight = nn.Parameter(torch.empty(out_features, in_features))
        self.spline_weight = nn.Parameter(torch.empty(out_features, in_features, R))
        if enable_standalone_scale_spline:
            self.spline_scaler = nn.Parameter(torch.empty(out_features, in_features))
        self.reset_parameters()

    def _uniform_grid(self, a: float, b: float) -> torch.Tensor:
        G, k = self.grid_size, self.spline_order
        r = torch.arange(G + 2 * k + 1, dtype=torch.float32)
        row = a + (r - k) * (b - a) / G
        return row.unsqueeze(0).repeat(self.in_features, 1)

    def reset_parameters(self) -> None:
        """Kaiming-uniform base weights (times scale_base), spline coefficients
        uniform in +-scale_noise/sqrt(R), scaler = scale_spline
        (spline_kan/reference_backend.py:338-352)."""
        nn.init.kaiming_uniform_(self.base_weight, a=math.sqrt(5))
        R = self.grid_size + self.spline_order
        with torch.no_grad():
            self.base_weight.mul_(self.scale_base)
            noise = (torch.rand_like(self.spline_weight) - 0.5) * 2.0
            self.spline_weight.copy_(noise * self.scale_noise / math.sqrt(R))
            if self.enable_standalone_scale_spline:
                self.spline_scaler.fill_(self.scale_spline)

    def effective_spline_weight(self) -> torch.Tensor:
        """spline_weight * spline_scaler[..., None] (or spline_weight without scaler)."""
        if self.enable_standalone_scale_spline:
            return self.spline_weight * self.spline_scaler.unsqueeze(-1)
        return self.spline_weight

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        xf = x.reshape(-1, self.in_features)
        H = compute_basis(xf, self.grid, self.spline_order)
        y = F.linear(self.base_activation(xf), self.base_weight) + F.linear(
            H.reshape(xf.shape[0], -1),
            self.effective_spline_weight().reshape(self.out_features, -1))
        return y.reshape(lead + (self.out_features,))

    @torch.no_grad()
    def grid_from_samples(self, x_flat: torch.Tensor, G: int, margin: float = 0.01) -> torch.Tensor:
        """Knot rows [I, G+2k+1] adapted to the samples: G+1 interior knots from
        a (1-grid_eps) quantile + grid_eps uniform mixture over the
        margin-widened range, k outer knots per side spaced (range)/G
        (spline_kan/reference_backend.py:384-439)."""
        B = x_flat.shape[0]
        k = self.spline_order
        dt, dev = x_flat.dtype, x_flat.device
        xs, _ = x_flat.sort(dim=0)
        lo, hi = xs[0] - margin, xs[-1] + margin                       # [I]
        frac_u = torch.linspace(0.0, 1.0, G + 1, device=dev, dtype=dt)
        uniform = lo[None] + frac_u[:, None] * (hi - lo)[None]          # [G+1, I]
        q = (torch.arange(G + 1, dtype=dt, device=dev) * ((1.0 - self.grid_eps) / G)
             + self.grid_eps / 2.0).clamp(0.0, 1.0)
        pos = q * (B - 1)
        i_lo = pos.long().clamp(0, B - 1)
        i_hi = (i_lo + 1).clamp(0, B - 1)
        w = (pos - i_lo.to(dt)).unsqueeze(-1)
        quant = (1.0 - w) * xs[i_lo] + w * xs[i_hi]                      # [G+1, I]
        inner = (1.0 - self.grid_eps) * quant + self.grid_eps * uniform
        step = (hi - lo) / G
        left = inner[0][None] - torch.arange(k, 0, -1, device=dev, dtype=dt)[:, None] * step[None]
        right = inner[-1][None] + torch.arange(1, k + 1, device=dev, dtype=dt)[:, None] * step[None]
        return torch.cat([left, inner, right], dim=0).t().contiguous()

    def check_update_grid_args(self, x: torch.Tensor, margin: float) -> torch.Tensor:
        """Argument checks of update_grid in the reference's order
        (spline_kan/reference_backend.py:464-477); returns x as [B, I]."""
        if margin <= 0:
            raise ValueError(f"margin must be positive, got {margin}")
        if not (0.0 < self.grid_eps < 1.0):
            raise ValueError(f"grid_eps must be in (0, 1), got {self.grid_eps}")
        xf = x.reshape(-1, self.in_features)
        if xf.shape[0] < 2:
            raise ValueError(f"update_grid requires at least 2 samples, got {xf.shape[0]}")
        return xf

    @torch.no_grad()
    def update_grid(self, x: torch.Tensor, margin: float = 0.01) -> None:
        """Moves the knots to the sample distribution and refits the unscaled
        spline coefficients to the old curves by least squares; grid and
        coefficients are replaced together (spline_kan/reference_backend.py:442-493)."""
        xf = self.check_update_grid_args(x, margin)
        k = self.spline_order
        H_old = compute_basis(xf, self.grid, k)
        y_old = torch.einsum("oir,bir->obi", self.spline_weight, H_old)
        new_grid = self.grid_from_samples(xf, self.grid_size, margin)
        coef = curve2coeff(xf, y_old, new_grid, k)
        self.grid.copy_(new_grid)
        self.spline_weight.copy_(coef)

    def regularization_loss(self, regularize_activation: float = 1.0,
                            regularize_entropy: float = 1.0, *, x: Optional[torch.Tensor] = None,
                            mode: str = "activation") -> torch.Tensor:
        """Activation-based (KAN paper) or legacy coefficient-based penalty
        (spline_kan/reference_backend.py:499-617)."""
        if mode not in ("activation", "coefficient"):
            raise ValueError(f"mode must be 'activation' or 'coefficient', got {mode!r}")
        if mode == "activation":
            if x is None:
                raise ValueError(
                    "regularization_loss with mode='activation' requires x. Pass the layer's "
                    "input samples as x=<tensor>, or use mode='coefficient' for the legacy "
                    "coefficient-based loss.")
            xf = x.reshape(-1, self.in_features)
            H = compute_basis(xf, self.grid, self.spline_order)
            a = edge_abs_mean_dense(self.base_activation(xf), H, self.base_weight,
                                    self.effective_spline_weight())
            return regularization_from_edge_means(a, regularize_activation, regularize_entropy)
        mag = self.effective_spline_weight().abs() if self.enable_standalone_scale_spline \
            else self.spline_weight.abs()
        per_edge = mag.mean(dim=-1)                                          # [O, I]
        p = (per_edge / per_edge.sum(dim=-1, keepdim=True).clamp(min=1e-8)).clamp(min=1e-8)
        return regularize_activation * per_edge.sum() + regularize_entropy * (-(p * p.log()).sum())
