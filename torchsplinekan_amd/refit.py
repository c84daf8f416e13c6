"""Least-squares refit of a layer's spline curves onto new knots, on the
device: the work behind KANLinear.update_grid (fixed G, knots moved) and
KANLinear.extend_grid (new G).

The reference forms the old curves y_old[o, b, i] = sum_s coef[o, i, s] bo_s(x[b, i])
as a dense [O, B, I] tensor and solves, per feature, a least-squares problem
with the new basis A_i [B, Rn] (spline_kan/reference_backend.py:173-265,
483-489; spline_kan/kan_linear.py:579-582).  Both reduce to two small
per-feature matrices

    G_i = A_i^T A_i                    [Rn, Rn]
    C_i = A_i^T Bold_i                 [Rn, Ro]    (A_i^T y_old = C_i coef[:, i, :]^T)

which libkan_hip.so accumulates in float64 in one pass over the samples
(kan_hip_refit_gram), so y_old is never formed.  The [Rn, Rn] solves then run
in float64 on the same device:

  * solve_min_norm  -- the minimum-norm least-squares solution that
    curve2coeff's torch.linalg.lstsq returns, through the eigen-decomposition
    of G_i: eigenvalues at or below `rtol * max eigenvalue` count as zero.  The
    default rtol = 1e-12 sits above the rounding of the accumulated G_i, so it
    drops the directions of A_i with singular-value ratio below 1e-6 (lstsq's
    rank test drops those below eps * max(B, Rn)).  The two therefore differ
    only for fits with cond(A_i) > 1e6; measured cond(A_i) for quantile knots
    on mixture data is 12-60.
  * solve_ridge     -- fit_spline_coeffs: Cholesky of G_i + lam * tr(G_i)/Rn * I
    with lam = ridge, raised 1e3-fold up to three times while the
    factorisation fails, then a general solve (reference_backend.py:197-215).
"""

import torch

from . import _lib
from .reference_backend import ridge_solve


def refit_gram(x_flat: torch.Tensor, grid_old: torch.Tensor, grid_new: torch.Tensor, k: int):
    """(G [I, Rn, Rn], C [I, Rn, Ro]) in float64 on x's device."""
    if not (x_flat.is_cuda and grid_old.is_cuda and grid_new.is_cuda):
        raise RuntimeError("refit_gram: x and both grids must be device tensors")
    if x_flat.dim() != 2 or grid_old.dim() != 2 or grid_new.dim() != 2:
        raise RuntimeError("refit_gram: x must be [B, I] and the grids [I, G+2k+1]")
    B, I = x_flat.shape
    if grid_old.shape[0] != I or grid_new.shape[0] != I:
        raise RuntimeError("refit_gram: grid rows must match in_features")
    dt = x_flat.dtype
    Go = grid_old.shape[1] - 2 * k - 1
    Gn = grid_new.shape[1] - 2 * k - 1
    Ro, Rn = Go + k, Gn + k
    dev = x_flat.device
    xt = x_flat.t().contiguous()                                   # feature-major [I, B]
    go = grid_old.to(dt).contiguous()
    gn = grid_new.to(dt).contiguous()
    gram = torch.empty(I, Rn, Rn, dtype=torch.float64, device=dev)
    cross = torch.empty(I, Rn, Ro, dtype=torch.float64, device=dev)
    with torch.cuda.device(dev):
        _lib.check(_lib.LIB.kan_hip_refit_gram(
            _lib.dtype_code(dt), _lib.ptr(xt), _lib.ptr(go), _lib.ptr(gn), gram.data_ptr(),
            cross.data_ptr(), B, I, Go, Gn, k, _lib.stream_of(dev)))
    return gram, cross


def solve_min_norm(gram: torch.Tensor, cross: torch.Tensor, coef: torch.Tensor,
                   rtol: float = 1e-12) -> torch.Tensor:
    """Minimum-norm least-squares coefficients [O, I, Rn] (float64) of the
    curves coef [O, I, Ro] on the new basis (curve2coeff semantics)."""
    lam, V = torch.linalg.eigh(gram)                                # ascending, [I, Rn]
    top = lam[:, -1:].clamp_min(0.0)
    keep = lam > rtol * top
    inv = torch.where(keep, 1.0 / torch.where(keep, lam, torch.ones_like(lam)),
                      torch.zeros_like(lam))
    X = V @ (inv.unsqueeze(-1) * (V.transpose(-1, -2) @ cross))    # [I, Rn, Ro]
    return torch.einsum("irs,ois->oir", X, coef.to(torch.float64))


def solve_ridge(gram: torch.Tensor, cross: torch.Tensor, coef: torch.Tensor,
                ridge: float = 1e-12) -> torch.Tensor:
    """Ridge-regularised normal-equation coefficients [O, I, Rn] (float64) of
    fit_spline_coeffs (spline_kan/reference_backend.py:173-215): the right-hand
    side A_i^T y_old is C_i coef[:, i, :]^T, solved by the same shift ladder."""
    rhs = cross @ coef.to(torch.float64).permute(1, 2, 0)            # [I, Rn, O]
    return ridge_solve(gram, rhs, ridge).permute(2, 0, 1)            # [O, I, Rn]
