"""ATen formulations of the KANLinear forward/backward.

Two uses, both mirroring the reference's native extension:
  * the CPU dispatch of the raw ops (``kan_forward``/``kan_backward`` on CPU
    tensors; csrc/kan_cpu.cpp:136-290): forward plus the analytic backward;
  * the differentiable backward used when autograd records the backward
    itself (``create_graph=True``; kan_backward_composite,
    csrc/kan_cpu.cpp:301-345), which recomputes the basis and its derivative
    with differentiable ops so that higher-order derivatives are exact.  It
    runs on the tensors' own device (no host round trip).
"""

from typing import Optional, Tuple

import torch

from .reference_backend import compute_basis, compute_basis_derivative


def has_base(base_weight: Optional[torch.Tensor]) -> bool:
    """A layer has a fused SiLU base branch iff base_weight is non-empty
    (kan_has_base, csrc/kan_ops.h:22-24)."""
    return base_weight is not None and base_weight.numel() > 0


def _eff_weight(spline_weight, spline_scaler, has_scaler):
    return spline_weight * spline_scaler.unsqueeze(2) if has_scaler else spline_weight


def _silu_grad(x: torch.Tensor) -> torch.Tensor:
    sg = torch.sigmoid(x)
    return sg * (1.0 + x * (1.0 - sg))


def kan_forward_cpu(x, grid, base_weight, spline_weight, spline_scaler, spline_order: int,
                    has_scaler: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """(y [B, O], H [B, I, R]) with y = silu(x) bw^T + H (sw*scaler)^T."""
    B, I = x.shape
    O, _, R = spline_weight.shape
    H = compute_basis(x, grid, spline_order)
    y = H.reshape(B, I * R) @ _eff_weight(spline_weight, spline_scaler, has_scaler).reshape(O, I * R).t()
    if has_base(base_weight):
        y = torch.nn.functional.silu(x) @ base_weight.t() + y
    return y, H


def kan_backward_cpu(D, x, grid, base_weight, spline_weight, spline_scaler, basis,
                     spline_order: int, has_scaler: bool, need_x: bool = True):
    """Analytic first-order backward from the saved basis:
    gbw = D^T silu(x); DtH = D^T H; gsw = scaler*DtH; gscaler = sum_r sw*DtH;
    gx = sum_r (D W)[.,.,r] dB_r/dx + (D bw) silu'(x) (None when not need_x)."""
    B, I = x.shape
    O, _, R = spline_weight.shape
    hb = has_base(base_weight)
    gbw = D.t() @ torch.nn.functional.silu(x) if hb else None
    DtH = (D.t() @ basis.reshape(B, I * R)).reshape(O, I, R)
    if has_scaler:
        gsw = spline_scaler.unsqueeze(2) * DtH
        gsc = (spline_weight * DtH).sum(2)
    else:
        gsw, gsc = DtH, None
    if not need_x:
        return None, gbw, gsw, gsc
    W = _eff_weight(spline_weight, spline_scaler, has_scaler)
    DW = (D @ W.reshape(O, I * R)).reshape(B, I, R)
    gx = (DW * compute_basis_derivative(x, grid, spline_order)).sum(2)
    if hb:
        gx = gx + (D @ base_weight) * _silu_grad(x)
    return gx, gbw, gsw, gsc


def kan_backward_composite(D, x, grid, base_weight, spline_weight, spline_scaler,
                           spline_order: int, has_scaler: bool):
    """Same maths as kan_backward_cpu, but the basis is recomputed from x with
    differentiable ops, so the returned gradients carry the exact curvature
    when autograd records them (create_graph=True)."""
    B, I = x.shape
    H = compute_basis(x, grid, spline_order)
    return kan_backward_cpu(D, x, grid, base_weight, spline_weight, spline_scaler, H,
                            spline_order, has_scaler)
