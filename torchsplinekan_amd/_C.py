"""Drop-in replacement for the ``spline_kan._C`` extension module.

Same surface as the reference's pybind module (csrc/kan_ext.cpp:161-222):
attributes CUDA_MAX_DEG0_BASIS, CUDA_MAX_IN_FEATURES, HAS_FUSED_KERNELS and
functions kan_forward, kan_backward, kan_apply, set_basis_impl,
get_basis_impl, basis, basis_grad, edge_abs_mean, edge_abs_mean_backward,
with the same argument names, return conventions (empty tensor = absent
optional, None for gradients not computed) and error texts
(RuntimeError from the validation, as TORCH_CHECK raises).

Device tensors (ROCm tensors report ``is_cuda``) run on the gfx950 kernels
of libkan_hip.so, called through its C-ABI on the current torch stream of
the tensors' device.  CPU tensors dispatch to the ATen formulation, as the
reference dispatches to csrc/kan_cpu.cpp.  Importing this module raises
ImportError when libkan_hip.so has not been built.
"""

from typing import Optional, Tuple

import torch

from . import _lib
from . import composite as _cmp
from ._lib import LIB, check, dtype_code, ptr, stream_of

CUDA_MAX_DEG0_BASIS, CUDA_MAX_IN_FEATURES = _lib.limits()
HAS_FUSED_KERNELS = True

_F = (torch.float32, torch.float64)


def _req(cond: bool, *msg) -> None:
    if not cond:
        raise RuntimeError("".join(str(m) for m in msg))


def _check_inputs(x, grid, base_weight, spline_weight, spline_scaler, spline_order, has_scaler):
    """Validation of kan_check_inputs (csrc/kan_ops.h:27-78) with the same
    messages.  The reference's 32-bit index guard (B*I*(G+2k) <= INT_MAX) is
    not applied: every native kernel here uses 64-bit offsets."""
    _req(x.dim() == 2, "x must be 2-D [B, I], got ", x.dim(), "-D")
    _req(grid.dim() == 2, "grid must be 2-D [I, G+2k+1]")
    _req(spline_weight.dim() == 3, "spline_weight must be 3-D [O, I, R]")
    _req(1 <= spline_order <= 3, "spline_order must be 1, 2 or 3; got ", spline_order)
    I, O, nk = x.shape[1], spline_weight.shape[0], grid.shape[1]
    G = nk - 2 * spline_order - 1
    _req(G >= 1, "grid has ", nk, " knots, too few for spline_order ", spline_order)
    _req(grid.shape[0] == I, "grid.size(0)=", grid.shape[0], " must equal in_features=", I)
    _req(spline_weight.shape[1] == I, "spline_weight.size(1) must equal in_features=", I)
    _req(spline_weight.shape[2] == G + spline_order, "spline_weight.size(2)=",
         spline_weight.shape[2], " but grid implies R=G+k=", G + spline_order)
    _req(x.dtype in _F, "only FP32 and FP64 inputs are supported, got ", x.dtype)
    _req(grid.dtype == x.dtype and spline_weight.dtype == x.dtype,
         "x, grid and spline_weight must share a dtype")
    _req(grid.device == x.device and spline_weight.device == x.device,
         "x, grid and spline_weight must be on the same device")
    if _cmp.has_base(base_weight):
        _req(base_weight.dim() == 2 and tuple(base_weight.shape) == (O, I),
             "base_weight must have shape [O, I] = [", O, ", ", I, "]")
        _req(base_weight.dtype == x.dtype and base_weight.device == x.device,
             "base_weight must match x in dtype and device")
    if has_scaler:
        _req(spline_scaler is not None and spline_scaler.dim() == 2
             and tuple(spline_scaler.shape) == (O, I),
             "spline_scaler must have shape [O, I] = [", O, ", ", I, "]")
        _req(spline_scaler.dtype == x.dtype and spline_scaler.device == x.device,
             "spline_scaler must match x in dtype and device")
    if x.is_cuda:
        _req(G + 2 * spline_order <= CUDA_MAX_DEG0_BASIS, "CUDA kernel supports G + 2k <= ",
             CUDA_MAX_DEG0_BASIS, " (got G=", G, ", k=", spline_order,
             "); use backend='reference' for larger grids")
        _req(I <= CUDA_MAX_IN_FEATURES, "CUDA kernel supports in_features <= ",
             CUDA_MAX_IN_FEATURES, ", got ", I)
    return G


def _contig(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.contiguous()


# ---------------------------------------------------------------------------
# device implementations
# ---------------------------------------------------------------------------

def _forward_device(x, grid, base_weight, spline_weight, spline_scaler, k, has_scaler):
    """(y [B, O], basis_aug [B, W]) from the gfx950 forward."""
    G = grid.shape[1] - 2 * k - 1
    hb = _cmp.has_base(base_weight)
    x, grid, sw = x.contiguous(), grid.contiguous(), spline_weight.contiguous()
    bw = base_weight.contiguous() if hb else None
    sc = spline_scaler.contiguous() if has_scaler else None
    B, I = x.shape
    O = sw.shape[0]
    ld = int(LIB.kan_hip_aug_width(I, G, k, int(hb)))
    code = dtype_code(x.dtype)
    y = torch.empty(B, O, dtype=x.dtype, device=x.device)
    aug = torch.empty(B, ld, dtype=x.dtype, device=x.device)
    nbytes = _lib.ctypes.c_size_t(0)
    check(LIB.kan_hip_forward_workspace(code, B, I, O, G, k, int(hb), _lib.ctypes.byref(nbytes)))
    ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_forward(code, ptr(x), ptr(grid), ptr(bw), ptr(sw), ptr(sc), ptr(y),
                                  ptr(aug), ptr(ws), int(nbytes.value), B, I, O, G, k,
                                  stream_of(x.device)))
    return y, aug


def pack_weight(base_weight, spline_weight, spline_scaler, spline_order: int,
                has_scaler: bool) -> torch.Tensor:
    """Packed inference weight [O, ld] = [spline_weight * scaler | base_weight]
    (device); the operand kan_infer reads."""
    hb = _cmp.has_base(base_weight)
    sw = spline_weight.contiguous()
    O, I, R = sw.shape
    G = R - spline_order
    bw = base_weight.contiguous().to(sw.dtype) if hb else None
    sc = spline_scaler.contiguous().to(sw.dtype) if has_scaler else None
    ld = int(LIB.kan_hip_aug_width(I, G, spline_order, int(hb)))
    waug = torch.empty(O, ld, dtype=sw.dtype, device=sw.device)
    with torch.cuda.device(sw.device):
        check(LIB.kan_hip_pack_weight(dtype_code(sw.dtype), ptr(bw), ptr(sw), ptr(sc), ptr(waug),
                                      I, O, G, spline_order, stream_of(sw.device)))
    return waug


def kan_infer(x, grid, waug, spline_order: int, has_base: bool) -> torch.Tensor:
    """Inference forward y [B, O] from a packed weight (pack_weight): no
    autograd, no saved basis; small batches split the product over K."""
    _req(x.is_cuda and grid.is_cuda and waug.is_cuda, "kan_infer: tensors must be on the device")
    _req(x.dim() == 2 and waug.dim() == 2 and grid.dim() == 2, "kan_infer: x [B, I], waug [O, ld]")
    _req(x.dtype == grid.dtype == waug.dtype and x.dtype in _F, "kan_infer: dtype mismatch")
    B, I = x.shape
    G = grid.shape[1] - 2 * spline_order - 1
    O = waug.shape[0]
    ld = int(LIB.kan_hip_aug_width(I, G, spline_order, int(has_base)))
    _req(tuple(waug.shape) == (O, ld) and grid.shape[0] == I, "kan_infer: packed weight shape")
    x, grid, waug = x.contiguous(), grid.contiguous(), waug.contiguous()
    y = torch.empty(B, O, dtype=x.dtype, device=x.device)
    if B * O == 0:
        return y
    code = dtype_code(x.dtype)
    nbytes = _lib.ctypes.c_size_t(0)
    check(LIB.kan_hip_infer_workspace(code, B, I, O, G, spline_order, int(has_base),
                                      _lib.ctypes.byref(nbytes)))
    ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=x.device)
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_infer(code, ptr(x), ptr(grid), ptr(waug), ptr(y), ptr(ws),
                                int(nbytes.value), B, I, O, G, spline_order, int(has_base),
                                stream_of(x.device)))
    return y


def kan_infer_noalloc(x, grid, waug, spline_order: int, has_base: bool) -> torch.Tensor:
    """kan_infer without a workspace: kan_hip_infer_noalloc runs the same
    kernels on the library's fixed per-device scratch (at most
    KAN_NOALLOC_SCRATCH_BYTES of workspace; larger calls raise).  Calls that
    overlap on one GPU race on that scratch."""
    _req(x.is_cuda and grid.is_cuda and waug.is_cuda, "kan_infer_noalloc: tensors must be on the device")
    _req(x.dim() == 2 and waug.dim() == 2 and grid.dim() == 2,
         "kan_infer_noalloc: x [B, I], waug [O, ld]")
    _req(x.dtype == grid.dtype == waug.dtype and x.dtype in _F, "kan_infer_noalloc: dtype mismatch")
    B, I = x.shape
    G = grid.shape[1] - 2 * spline_order - 1
    O = waug.shape[0]
    ld = int(LIB.kan_hip_aug_width(I, G, spline_order, int(has_base)))
    _req(tuple(waug.shape) == (O, ld) and grid.shape[0] == I, "kan_infer_noalloc: packed weight shape")
    x, grid, waug = x.contiguous(), grid.contiguous(), waug.contiguous()
    y = torch.empty(B, O, dtype=x.dtype, device=x.device)
    if B * O == 0:
        return y
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_infer_noalloc(dtype_code(x.dtype), ptr(x), ptr(grid), ptr(waug), ptr(y),
                                        B, I, O, G, spline_order, int(has_base),
                                        stream_of(x.device)))
    return y


def _basis_of(aug: torch.Tensor, I: int, R: int) -> torch.Tensor:
    """basis [B, I, R] copied out of the augmented rows into its own
    contiguous tensor, the layout kan_forward_cuda returns
    (csrc/kan_cuda.cu:501), so callers may view or flatten it freely."""
    return aug[:, :I * R].reshape(aug.shape[0], I, R).contiguous()


def _backward_device(D, x, grid, base_weight, spline_weight, spline_scaler, aug, k, has_scaler,
                     need_x, need_base, need_spline):
    G = grid.shape[1] - 2 * k - 1
    hb = _cmp.has_base(base_weight)
    need_base = need_base and hb
    D, x, grid, sw = D.contiguous(), x.contiguous(), grid.contiguous(), spline_weight.contiguous()
    bw = base_weight.contiguous() if hb else None
    sc = spline_scaler.contiguous() if has_scaler else None
    B, I = x.shape
    O, _, R = sw.shape
    opts = dict(dtype=x.dtype, device=x.device)
    gx = torch.empty(B, I, **opts) if need_x else None
    gbw = torch.empty(O, I, **opts) if need_base else None
    gsw = torch.empty(O, I, R, **opts) if need_spline else None
    gsc = torch.empty(O, I, **opts) if (need_spline and has_scaler) else None
    if not (need_x or need_base or need_spline):
        return gx, gbw, gsw, gsc
    code = dtype_code(x.dtype)
    nbytes = _lib.ctypes.c_size_t()
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_backward_workspace(code, B, I, O, G, k, int(hb), int(need_x),
                                             int(need_base or need_spline),
                                             _lib.ctypes.byref(nbytes)))
        ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=x.device)
        check(LIB.kan_hip_backward(code, ptr(D), ptr(x), ptr(grid), ptr(bw), ptr(sw), ptr(sc),
                                   ptr(aug), ptr(gx), ptr(gbw), ptr(gsw), ptr(gsc), ptr(ws),
                                   int(nbytes.value), B, I, O, G, k, stream_of(x.device)))
    return gx, gbw, gsw, gsc


def _pack_basis_device(basis, x, grid, k, hb):
    G = grid.shape[1] - 2 * k - 1
    B, I = x.shape
    ld = int(LIB.kan_hip_aug_width(I, G, k, int(hb)))
    basis = basis.contiguous().to(x.dtype)
    xc = x.contiguous()
    aug = torch.empty(B, ld, dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_pack_basis(dtype_code(x.dtype), ptr(basis), ptr(xc), ptr(aug), B, I, G,
                                     k, int(hb), stream_of(x.device)))
    return aug


# ---------------------------------------------------------------------------
# raw ops (csrc/kan_ext.cpp:10-56)
# ---------------------------------------------------------------------------

def kan_forward(x, grid, base_weight, spline_weight, spline_scaler, spline_order: int,
                has_scaler: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """B-spline KAN forward (CPU/device dispatch) -> (output [B, O], basis [B, I, R])."""
    _check_inputs(x, grid, base_weight, spline_weight, spline_scaler, spline_order, has_scaler)
    if x.is_cuda:
        y, aug = _forward_device(x, grid, base_weight, spline_weight, spline_scaler,
                                 spline_order, has_scaler)
        return y, _basis_of(aug, x.shape[1], spline_weight.shape[2])
    return _cmp.kan_forward_cpu(x.contiguous(), grid.contiguous(), base_weight,
                                spline_weight.contiguous(), spline_scaler, spline_order,
                                has_scaler)


def kan_backward(grad_output, x, grid, base_weight, spline_weight, spline_scaler, basis,
                 spline_order: int, has_scaler: bool):
    """B-spline KAN backward (CPU/device dispatch) ->
    (grad_x, grad_base_weight | None, grad_spline_weight, grad_spline_scaler | None)."""
    if x.is_cuda:
        _check_inputs(x, grid, base_weight, spline_weight, spline_scaler, spline_order, has_scaler)
        hb = _cmp.has_base(base_weight)
        B, I = x.shape
        R = spline_weight.shape[2]
        _req(basis.numel() == B * I * R, "kan_backward_cuda: saved basis missing or wrong size")
        aug = _pack_basis_device(basis.reshape(B, I, R), x, grid, spline_order, hb)
        return _backward_device(grad_output, x, grid, base_weight, spline_weight, spline_scaler,
                                aug, spline_order, has_scaler, True, True, True)
    return _cmp.kan_backward_cpu(grad_output.contiguous(), x.contiguous(), grid.contiguous(),
                                 base_weight, spline_weight.contiguous(), spline_scaler,
                                 basis.contiguous(), spline_order, has_scaler)


class KANFunction(torch.autograd.Function):
    """Autograd function of kan_apply (csrc/kan_autograd.cpp:13-111).

    Forward saves the augmented basis produced by the kernels.  Backward
    computes only what autograd asks for (needs_input_grad); when the
    backward itself is being recorded (create_graph=True) it switches to a
    differentiable formulation so that higher-order derivatives are exact:
    on the device, kan_backward_composite_device (native basis derivatives
    of any order); on the CPU, the ATen composite.
    """

    @staticmethod
    def forward(ctx, x, grid, base_weight, spline_weight, spline_scaler, spline_order,
                has_scaler):
        if x.is_cuda:
            y, saved = _forward_device(x, grid, base_weight, spline_weight, spline_scaler,
                                       spline_order, has_scaler)
        else:
            y, saved = _cmp.kan_forward_cpu(x.contiguous(), grid.contiguous(), base_weight,
                                            spline_weight.contiguous(), spline_scaler,
                                            spline_order, has_scaler)
        ctx.spline_order = spline_order
        ctx.has_scaler = has_scaler
        ctx.save_for_backward(x, grid, base_weight, spline_weight,
                              spline_scaler if has_scaler else None, saved)
        return y

    @staticmethod
    def backward(ctx, D):
        x, grid, bw, sw, sc, saved = ctx.saved_tensors
        k, has_scaler = ctx.spline_order, ctx.has_scaler
        if torch.is_grad_enabled():
            if x.is_cuda:
                gx, gbw, gsw, gsc = kan_backward_composite_device(D, x, grid, bw, sw, sc, k,
                                                                  has_scaler)
            else:
                gx, gbw, gsw, gsc = _cmp.kan_backward_composite(D, x, grid, bw, sw, sc, k,
                                                                has_scaler)
        elif x.is_cuda:
            nig = ctx.needs_input_grad
            need_spline = bool(nig[3] or (has_scaler and nig[4]))
            gx, gbw, gsw, gsc = _backward_device(D, x, grid, bw, sw, sc, saved, k, has_scaler,
                                                 bool(nig[0]), bool(nig[2]), need_spline)
        else:
            gx, gbw, gsw, gsc = _cmp.kan_backward_cpu(D.contiguous(), x.contiguous(),
                                                      grid.contiguous(), bw, sw.contiguous(), sc,
                                                      saved, k, has_scaler)
        return (gx, None, gbw if _cmp.has_base(bw) else None, gsw,
                gsc if has_scaler else None, None, None)


def kan_apply(x, grid, base_weight, spline_weight, spline_scaler, spline_order: int,
              has_scaler: bool) -> torch.Tensor:
    """B-spline KAN forward with autograd (KANFunction)."""
    _check_inputs(x, grid, base_weight, spline_weight, spline_scaler, spline_order, has_scaler)
    return KANFunction.apply(x, grid, base_weight, spline_weight, spline_scaler, spline_order,
                             has_scaler)


def stream_probe(mode: int, a: torch.Tensor, b: torch.Tensor) -> None:
    """Streaming probe over a's bytes (measurement support): mode 0 writes a,
    1 reads a, 2 copies a into b (b at least as large as a for mode 2), 3
    writes a in the basis kernel's row-segment pattern (rows of 14336 floats);
    4-10 are candidate patterns on that layout (4, 6, 7, 8 and 9 write a, 5
    and 10 read a and write [rows, 1024] floats of b)."""
    _req(a.is_cuda and b.is_cuda and a.is_contiguous() and b.is_contiguous(),
         "stream_probe: contiguous device tensors")
    nbytes = a.numel() * a.element_size() // 16 * 16
    _req(mode != 2 or b.numel() * b.element_size() >= nbytes, "stream_probe: b too small")
    _req(mode not in (5, 10) or b.numel() * b.element_size() >= nbytes // 14,
         "stream_probe: b too small")
    with torch.cuda.device(a.device):
        check(LIB.kan_hip_stream_probe(int(mode), ptr(a), ptr(b), nbytes, stream_of(a.device)))


# ---------------------------------------------------------------------------
# basis implementation switch (csrc/kan_cuda.cu:274-279)
# ---------------------------------------------------------------------------

def set_basis_impl(impl: int) -> None:
    """Selects the native basis kernel: 0 = full Cox-de Boor recurrence, 1 = local (default)."""
    if int(impl) != impl:
        raise RuntimeError("basis impl must be 0 (recurrence) or 1 (local)")
    check(LIB.kan_hip_set_basis_impl(int(impl)))


def get_basis_impl() -> int:
    return int(LIB.kan_hip_get_basis_impl())


# ---------------------------------------------------------------------------
# building blocks of the fused regularisation path
# ---------------------------------------------------------------------------

def _check_basis_args(x, grid, k):
    """check_basis_args, csrc/kan_cuda.cu:649-664 (no 32-bit index guard)."""
    _req(x.is_cuda and grid.is_cuda, "kan_basis: x and grid must be CUDA tensors")
    _req(x.dim() == 2 and grid.dim() == 2 and grid.shape[0] == x.shape[1],
         "kan_basis: x must be [B, I] and grid [I, G+2k+1]")
    _req(1 <= k <= 3, "kan_basis: spline_order must be 1, 2 or 3")
    _req(x.dtype == grid.dtype, "kan_basis: dtype mismatch")
    _req(x.dtype in _F, "kan_basis: only FP32/FP64 supported")
    G = grid.shape[1] - 2 * k - 1
    _req(G >= 1, "kan_basis: grid too short")
    _req(G + 2 * k <= CUDA_MAX_DEG0_BASIS, "CUDA kernel supports G + 2k <= ",
         CUDA_MAX_DEG0_BASIS, " (got G=", G, ", k=", k, ")")
    _req(x.shape[1] <= CUDA_MAX_IN_FEATURES, "kan_basis: too many input features")
    return G


def basis(x, grid, spline_order: int) -> torch.Tensor:
    """B-spline basis H [B, I, R] (device)."""
    G = _check_basis_args(x, grid, spline_order)
    x, grid = x.contiguous(), grid.contiguous()
    B, I = x.shape
    H = torch.empty(B, I, G + spline_order, dtype=x.dtype, device=x.device)
    if B == 0:
        return H
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_basis(dtype_code(x.dtype), ptr(x), ptr(grid), ptr(H), B, I, G,
                                spline_order, stream_of(x.device)))
    return H


def basis_grad(x, grid, spline_order: int, grad_basis) -> torch.Tensor:
    """gx[b, i] = sum_r grad_basis[b, i, r] dB_r/dx (device; dH/dx is never stored)."""
    G = _check_basis_args(x, grid, spline_order)
    B, I = x.shape
    R = G + spline_order
    _req(grad_basis.dim() == 3 and tuple(grad_basis.shape) == (B, I, R),
         "kan_basis_grad: gH must be [B, I, G+k]")
    x, grid = x.contiguous(), grid.contiguous()
    gH = grad_basis.contiguous().to(x.dtype)
    gx = torch.empty(B, I, dtype=x.dtype, device=x.device)
    if B == 0:
        return gx
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_basis_grad(dtype_code(x.dtype), ptr(x), ptr(grid), ptr(gH), ptr(gx),
                                     B, I, G, spline_order, stream_of(x.device)))
    return gx


def basis_silu(x, grid, spline_order: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(silu(x) [B, I], basis H [B, I, R]) from one pass over x (device)."""
    G = _check_basis_args(x, grid, spline_order)
    x, grid = x.contiguous(), grid.contiguous()
    B, I = x.shape
    H = torch.empty(B, I, G + spline_order, dtype=x.dtype, device=x.device)
    s = torch.empty(B, I, dtype=x.dtype, device=x.device)
    if B == 0:
        return s, H
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_basis_silu(dtype_code(x.dtype), ptr(x), ptr(grid), ptr(H), ptr(s), B, I,
                                     G, spline_order, stream_of(x.device)))
    return s, H


def basis_silu_grad(x, grid, spline_order: int, grad_basis, grad_silu) -> torch.Tensor:
    """gx = sum_r grad_basis dB_r/dx + grad_silu silu'(x) in one pass (device)."""
    G = _check_basis_args(x, grid, spline_order)
    B, I = x.shape
    R = G + spline_order
    _req(grad_basis.dim() == 3 and tuple(grad_basis.shape) == (B, I, R),
         "kan_basis_silu_grad: gH must be [B, I, G+k]")
    _req(tuple(grad_silu.shape) == (B, I), "kan_basis_silu_grad: gs must be [B, I]")
    x, grid = x.contiguous(), grid.contiguous()
    gH = grad_basis.contiguous().to(x.dtype)
    gs = grad_silu.contiguous().to(x.dtype)
    gx = torch.empty(B, I, dtype=x.dtype, device=x.device)
    if B == 0:
        return gx
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_basis_silu_grad(dtype_code(x.dtype), ptr(x), ptr(grid), ptr(gH),
                                          ptr(gs), ptr(gx), B, I, G, spline_order,
                                          stream_of(x.device)))
    return gx


def _optional_operand(t, like, name):
    """A [B, I] factor of the derivative kernels (or None), contiguous in x's dtype."""
    if t is None:
        return None
    _req(tuple(t.shape) == tuple(like.shape), f"{name} must be [B, I]")
    return t.contiguous().to(like.dtype)


def basis_deriv(x, grid, spline_order: int, order: int, scale=None) -> torch.Tensor:
    """scale[b, i] * d^order B / dx^order [B, I, R] (device; order 0 = basis,
    order > k = 0; scale None = 1)."""
    G = _check_basis_args(x, grid, spline_order)
    _req(order >= 0, "kan_basis_deriv: order must be >= 0")
    x, grid = x.contiguous(), grid.contiguous()
    B, I = x.shape
    w = _optional_operand(scale, x, "kan_basis_deriv: scale")
    out = torch.empty(B, I, G + spline_order, dtype=x.dtype, device=x.device)
    if B == 0:
        return out
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_basis_deriv(dtype_code(x.dtype), ptr(x), ptr(grid), ptr(w), ptr(out), B,
                                      I, G, spline_order, int(order), stream_of(x.device)))
    return out


def basis_deriv_contract(x, grid, spline_order: int, grad_basis, order: int, grad_base=None,
                         scale=None) -> torch.Tensor:
    """gx[b, i] = scale * (sum_r grad_basis[b, i, r] d^order B_r/dx^order
    + grad_base[b, i] silu^(order)(x)) (device; grad_base and scale optional)."""
    G = _check_basis_args(x, grid, spline_order)
    _req(order >= 0, "kan_basis_deriv_contract: order must be >= 0")
    B, I = x.shape
    R = G + spline_order
    _req(grad_basis.dim() == 3 and tuple(grad_basis.shape) == (B, I, R),
         "kan_basis_deriv_contract: gH must be [B, I, G+k]")
    x, grid = x.contiguous(), grid.contiguous()
    gH = grad_basis.contiguous().to(x.dtype)
    gb = _optional_operand(grad_base, x, "kan_basis_deriv_contract: grad_base")
    w = _optional_operand(scale, x, "kan_basis_deriv_contract: scale")
    gx = torch.empty(B, I, dtype=x.dtype, device=x.device)
    if B == 0:
        return gx
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_basis_deriv_contract(dtype_code(x.dtype), ptr(x), ptr(grid), ptr(gH),
                                               ptr(gb), ptr(w), ptr(gx), B, I, G, spline_order,
                                               int(order), stream_of(x.device)))
    return gx


SILU_MAX_ORDER = 4   # native orders of silu_deriv (the base term of the kernels above)


def silu_deriv(x, order: int, scale=None) -> torch.Tensor:
    """scale * silu^(order)(x), elementwise on the device (order 0..4)."""
    _req(x.is_cuda and x.dtype in _F, "kan_silu_deriv: x must be a float32/float64 CUDA tensor")
    _req(0 <= order <= SILU_MAX_ORDER, "kan_silu_deriv: order must lie in 0..", SILU_MAX_ORDER)
    xc = x.contiguous()
    w = _optional_operand(scale, xc, "kan_silu_deriv: scale")
    out = torch.empty_like(xc)
    if xc.numel() == 0:
        return out
    with torch.cuda.device(x.device):
        check(LIB.kan_hip_silu_deriv(dtype_code(x.dtype), ptr(xc), ptr(w), ptr(out), xc.numel(),
                                     int(order), stream_of(x.device)))
    return out


def _mm_operand(t: torch.Tensor):
    """(tensor, trans, ld) presenting a 2-D tensor [rows, cols] to kan_hip_matmul
    without a copy when it is row-major or the transpose of a row-major
    buffer; anything else is made contiguous."""
    rows, cols = t.shape
    if rows > 1 and cols > 1:
        if t.stride(1) == 1 and t.stride(0) >= cols:
            return t, 0, t.stride(0)
        if t.stride(0) == 1 and t.stride(1) >= rows:
            return t, 1, t.stride(1)
    t = t.contiguous()
    return t, 0, max(cols, 1)


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a [M, K] @ b [K, N] on the MFMA contraction engine (device, fp32/fp64),
    transposed views taken as they lie; long-K products are split over K and
    summed in a fixed order."""
    _req(a.is_cuda and b.is_cuda, "kan_matmul: operands must be CUDA tensors")
    _req(a.dim() == 2 and b.dim() == 2 and a.shape[1] == b.shape[0],
         "kan_matmul: shapes ", tuple(a.shape), " and ", tuple(b.shape), " do not chain")
    _req(a.dtype == b.dtype and a.dtype in _F, "kan_matmul: operands must share an FP32/FP64 dtype")
    M, K = a.shape
    N = b.shape[1]
    a, ta, lda = _mm_operand(a)
    b, tb, ldb = _mm_operand(b)
    c = torch.empty(M, N, dtype=a.dtype, device=a.device)
    if M * N == 0:
        return c
    code = dtype_code(a.dtype)
    nbytes = _lib.ctypes.c_size_t(0)
    check(LIB.kan_hip_matmul_workspace(code, ta, tb, M, N, K, _lib.ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=a.device) if nbytes.value else None
    with torch.cuda.device(a.device):
        check(LIB.kan_hip_matmul(code, ta, tb, M, N, K, ptr(a), lda, ptr(b), ldb, ptr(c), N,
                                 ptr(ws) if ws is not None else None, nbytes.value,
                                 stream_of(a.device)))
    return c


class NativeMatmul(torch.autograd.Function):
    """a @ b through kan_hip_matmul, differentiable to any order (its
    gradients g b^T and a^T g are NativeMatmul products again)."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return matmul(a, b)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        ga = NativeMatmul.apply(g, b.t()) if ctx.needs_input_grad[0] else None
        gb = NativeMatmul.apply(a.t(), g) if ctx.needs_input_grad[1] else None
        return ga, gb


class BasisDeriv(torch.autograd.Function):
    """Y = w[:, :, None] * D^q B(x) [B, I, R] on the device kernels (w None
    for 1), differentiable to any order: dx = DerivContract(x, gY; q + 1, w),
    dw = DerivContract(x, gY; q).  Together with DerivContract and SiluDeriv
    it replaces the differentiable ATen recurrences the reference records
    under create_graph=True (compute_basis and compute_basis_derivative,
    spline_kan/reference_backend.py:69-125); w folds the elementwise factor
    a recorded backward puts on them, so no [B, I, R] product is launched."""

    @staticmethod
    def forward(ctx, x, grid, k: int, order: int, w):
        ctx.k, ctx.order = k, order
        ctx.save_for_backward(x, grid, w)
        return basis_deriv(x, grid, k, order, w)

    @staticmethod
    def backward(ctx, gY):
        x, grid, w = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[4]
        gx = deriv_contract(x, grid, gY, ctx.k, ctx.order + 1, None, w) if need_x else None
        gw = (deriv_contract(x, grid, gY, ctx.k, ctx.order, None, None)
              if need_w and w is not None else None)
        return gx, None, None, None, gw


def _silu_sigmoid_poly(q: int):
    """Coefficients c with d^q sigmoid / dx^q = sum_j c[j] s^j (s = sigmoid):
    d/dx s^j = j s^j (1 - s)."""
    c = [0.0, 1.0]                     # s
    for _ in range(q):
        nxt = [0.0] * (len(c) + 1)
        for j, a in enumerate(c):
            nxt[j] += j * a
            nxt[j + 1] -= j * a
        c = nxt
    return c


def _silu_deriv_torch(x, q: int):
    """silu^(q)(x) = x s^(q) + q s^(q-1) from differentiable ATen operations,
    for the orders past the native kernels."""
    s = torch.sigmoid(x)
    poly = lambda c: sum(a * s ** j for j, a in enumerate(c) if a != 0.0)
    return x * poly(_silu_sigmoid_poly(q)) + q * poly(_silu_sigmoid_poly(q - 1))


def silu_deriv_any(x, q: int, w=None):
    """w * silu^(q)(x), differentiable: native for q <= 4, ATen beyond."""
    if q <= SILU_MAX_ORDER:
        return SiluDeriv.apply(x, q, w)
    out = _silu_deriv_torch(x, q)
    return out if w is None else out * w


class SiluDeriv(torch.autograd.Function):
    """Y = w * silu^(q)(x) on the device (w None for 1): dx = w g silu^(q+1)(x),
    dw = g silu^(q)(x), each one launch (silu_deriv)."""

    @staticmethod
    def forward(ctx, x, q: int, w):
        ctx.q = q
        ctx.save_for_backward(x, w)
        return silu_deriv(x, q, w)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[2]
        gx = silu_deriv_any(x, ctx.q + 1, g if w is None else g * w) if need_x else None
        gw = silu_deriv_any(x, ctx.q, g) if need_w and w is not None else None
        return gx, None, gw


def deriv_contract(x, grid, G, k: int, order: int, Gb=None, w=None):
    """w * (sum_r G D^order B_r(x) + Gb silu^(order)(x)), differentiable;
    Gb and w optional."""
    if Gb is not None and order > SILU_MAX_ORDER:
        spline = DerivContract.apply(x, grid, G, k, order, None, None)
        out = spline + silu_deriv_any(x, order, Gb)
        return out if w is None else out * w
    return DerivContract.apply(x, grid, G, k, order, Gb, w)


class DerivContract(torch.autograd.Function):
    """gx[b, i] = w * (sum_r G[b, i, r] D^q B_r(x[b, i]) + Gb[b, i] silu^(q)(x))
    on the device kernels (Gb, w optional); the derivative tensor is never
    formed.  With v = g w: dx = DerivContract(x, G, Gb; q + 1, v),
    dG = BasisDeriv(x; q, v), dGb = SiluDeriv(x; q, v), dw = DerivContract(x,
    G, Gb; q, g).  Past q = k the spline part is zero between knots."""

    @staticmethod
    def forward(ctx, x, grid, G, k: int, order: int, Gb, w):
        ctx.k, ctx.order = k, order
        ctx.save_for_backward(x, grid, G, Gb, w)
        return basis_deriv_contract(x, grid, k, G, order, Gb, w)

    @staticmethod
    def backward(ctx, g):
        x, grid, G, Gb, w = ctx.saved_tensors
        need_x, _, need_G, _, _, need_Gb, need_w = ctx.needs_input_grad
        v = g if w is None else g * w
        gx = deriv_contract(x, grid, G, ctx.k, ctx.order + 1, Gb, v) if need_x else None
        gG = BasisDeriv.apply(x, grid, ctx.k, ctx.order, v) if need_G else None
        gGb = silu_deriv_any(x, ctx.order, v) if need_Gb and Gb is not None else None
        gw = (deriv_contract(x, grid, G, ctx.k, ctx.order, Gb, g)
              if need_w and w is not None else None)
        return gx, None, gG, None, None, gGb, gw


def kan_backward_composite_device(D, x, grid, base_weight, spline_weight, spline_scaler,
                                  spline_order: int, has_scaler: bool):
    """Differentiable first-order backward on the device (create_graph=True).

    Same maths as kan_backward_composite (csrc/kan_cpu.cpp:301-345): the
    basis is a function of x again, so the recorded graph carries the exact
    spline curvature.  Here the basis and its derivative come from the native
    kernels through BasisDeriv / DerivContract (dB/dx is contracted in
    registers, never stored; the SiLU branch's (D bw) silu'(x) is added in the
    same launch), silu(x) from SiluDeriv, and the products run on the MFMA
    contraction engine through NativeMatmul (split over the sample axis where
    the output is small), differentiable in turn.
    """
    B, I = x.shape
    O, _, R = spline_weight.shape
    hb = _cmp.has_base(base_weight)
    mm = NativeMatmul.apply
    H = BasisDeriv.apply(x, grid, spline_order, 0, None)
    DtH = mm(D.t(), H.reshape(B, I * R)).reshape(O, I, R)
    if has_scaler:
        gsw = spline_scaler.unsqueeze(2) * DtH
        gsc = (spline_weight * DtH).sum(2)
    else:
        gsw, gsc = DtH, None
    W = _cmp._eff_weight(spline_weight, spline_scaler, has_scaler)
    DW = mm(D, W.reshape(O, I * R)).reshape(B, I, R)
    gbw = None
    if hb:
        gbw = mm(D.t(), SiluDeriv.apply(x, 0, None))
        gx = deriv_contract(x, grid, DW, spline_order, 1, mm(D, base_weight), None)
    else:
        gx = deriv_contract(x, grid, DW, spline_order, 1, None, None)
    return gx, gbw, gsw, gsc


def _check_edge_inputs(s, H, bw, W, hb):
    """check_edge_inputs, csrc/kan_reg_cuda.cu:240-257."""
    _req(H.is_cuda and W.is_cuda, "edge_abs_mean: H and W must be CUDA tensors")
    _req(H.dim() == 3 and W.dim() == 3, "edge_abs_mean: H must be [N,I,R], W [O,I,R]")
    _req(H.shape[1] == W.shape[1] and H.shape[2] == W.shape[2], "edge_abs_mean: H/W shape mismatch")
    _req(H.shape[2] <= 72, "edge_abs_mean: R must be <= 72, got ", H.shape[2])
    _req(H.shape[1] <= CUDA_MAX_IN_FEATURES, "edge_abs_mean: too many input features")
    _req(H.shape[0] >= 1, "edge_abs_mean: need at least one sample")
    _req(H.dtype == W.dtype, "edge_abs_mean: dtype mismatch")
    _req(H.dtype in _F, "edge_abs_mean: only FP32/FP64 supported")
    if hb:
        _req(tuple(s.shape) == tuple(H.shape[:2]), "edge_abs_mean: s must be [N, I]")
        _req(tuple(bw.shape) == tuple(W.shape[:2]), "edge_abs_mean: base_weight must be [O, I]")
        _req(s.dtype == H.dtype and bw.dtype == H.dtype, "edge_abs_mean: dtype mismatch")


def edge_abs_mean(s, H, base_weight, W) -> torch.Tensor:
    """a[o,i] = mean_n |s*bw + sum_r H*W| without materialising [N, O, I] (device)."""
    hb = _cmp.has_base(base_weight)
    _check_edge_inputs(s, H, base_weight, W, hb)
    H, W = H.contiguous(), W.contiguous()
    sc = s.contiguous() if hb else None
    bw = base_weight.contiguous() if hb else None
    N, I, R = H.shape
    O = W.shape[0]
    a = torch.empty(O, I, dtype=W.dtype, device=W.device)
    if O * I == 0:
        return a
    code = dtype_code(H.dtype)
    nbytes = _lib.ctypes.c_size_t()
    with torch.cuda.device(H.device):
        check(LIB.kan_hip_edge_workspace(code, N, I, O, R, 0, _lib.ctypes.byref(nbytes)))
        ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=H.device)
        check(LIB.kan_hip_edge_abs_mean(code, ptr(sc), ptr(H), ptr(bw), ptr(W), ptr(a), ptr(ws),
                                        int(nbytes.value), N, I, O, R, stream_of(H.device)))
    return a


def edge_abs_mean_backward(grad_a, s, H, base_weight, W, need_s: bool, need_H: bool,
                           need_bw: bool, need_W: bool):
    """Backward of edge_abs_mean, recomputing phi ->
    (ds | None, dH | None, dbw | None, dW | None)."""
    hb = _cmp.has_base(base_weight)
    _check_edge_inputs(s, H, base_weight, W, hb)
    _req(tuple(grad_a.shape) == tuple(W.shape[:2]), "edge_abs_mean_backward: grad shape")
    H, W = H.contiguous(), W.contiguous()
    ga = grad_a.contiguous().to(W.dtype)
    sc = s.contiguous() if hb else None
    bw = base_weight.contiguous() if hb else None
    N, I, R = H.shape
    O = W.shape[0]
    opts = dict(dtype=H.dtype, device=H.device)
    ds = torch.empty(N, I, **opts) if (need_s and hb) else None
    dH = torch.empty(N, I, R, **opts) if need_H else None
    dbw = torch.empty(O, I, **opts) if (need_bw and hb) else None
    dW = torch.empty(O, I, R, **opts) if need_W else None
    if ds is None and dH is None and dbw is None and dW is None:
        return ds, dH, dbw, dW
    code = dtype_code(H.dtype)
    nbytes = _lib.ctypes.c_size_t(0)
    with torch.cuda.device(H.device):
        if dbw is not None or dW is not None:
            check(LIB.kan_hip_edge_workspace(code, N, I, O, R, 1, _lib.ctypes.byref(nbytes)))
        ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=H.device)
        check(LIB.kan_hip_edge_abs_mean_backward(
            code, ptr(ga), ptr(sc), ptr(H), ptr(bw), ptr(W), ptr(ds), ptr(dH), ptr(dbw), ptr(dW),
            ptr(ws), int(nbytes.value), N, I, O, R, stream_of(H.device)))
    return ds, dH, dbw, dW


def edge_linear_supported(H: torch.Tensor, W: torch.Tensor) -> bool:
    """True where edge_linear_backward applies to these operands (float32,
    0 < out_features <= 512, num_basis + 1 <= 16, at least one sample)."""
    if not (H.is_cuda and H.dim() == 3 and W.dim() == 3):
        return False
    N, I, R = H.shape
    return bool(LIB.kan_hip_edge_linear_supported(dtype_code(H.dtype) if H.dtype in _F else -1,
                                                  N, I, W.shape[0], R))


def edge_linear_forward_supported(H: torch.Tensor, W: torch.Tensor) -> bool:
    """True where edge_linear_forward applies to these operands (float32,
    num_basis + 1 <= 16, at least one sample, input and output)."""
    if not (H.is_cuda and H.dim() == 3 and W.dim() == 3):
        return False
    N, I, R = H.shape
    return bool(LIB.kan_hip_edge_linear_forward_supported(
        dtype_code(H.dtype) if H.dtype in _F else -1, N, I, W.shape[0], R))


def edge_linear_forward(s, H, base_weight, W):
    """(y, a) of one regularised layer in one pass over phi (device, float32;
    see edge_linear_forward_supported): y = s bw^T + H W^T [N, O] (flattened
    over I and R) and a = mean_n |phi| [O, I], phi[n,o,i] = s bw + <H, W>.
    The reference forms y with two F.linear calls and a with EdgeAbsMean
    (spline_kan/kan_linear.py:384-387, spline_kan/fused.py:64-73)."""
    hb = _cmp.has_base(base_weight)
    _check_edge_inputs(s, H, base_weight, W, hb)
    _req(edge_linear_forward_supported(H, W), "edge_linear_forward: configuration not supported")
    N, I, R = H.shape
    O = W.shape[0]
    H, W = H.contiguous(), W.contiguous()
    sc = s.contiguous() if hb else None
    bw = base_weight.contiguous() if hb else None
    y = torch.empty(N, O, dtype=H.dtype, device=H.device)
    a = torch.empty(O, I, dtype=H.dtype, device=H.device)
    code = dtype_code(H.dtype)
    nbytes = _lib.ctypes.c_size_t(0)
    with torch.cuda.device(H.device):
        check(LIB.kan_hip_edge_linear_forward_workspace(code, N, I, O, R,
                                                        _lib.ctypes.byref(nbytes)))
        ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=H.device)
        check(LIB.kan_hip_edge_linear_forward(
            code, ptr(sc), ptr(H), ptr(bw), ptr(W), ptr(y), ptr(a), ptr(ws), int(nbytes.value),
            N, I, O, R, stream_of(H.device)))
    return y, a


def edge_linear_backward(grad_a, grad_y, s, H, base_weight, W, need_s: bool, need_H: bool,
                         need_bw: bool, need_W: bool):
    """Gradients of one regularised layer's output y = s bw^T + H W^T and its
    edge statistic a together: with g' = grad_a sign(phi) / n + grad_y,
    (ds, dH, dbw, dW) = (sum_o g' bw, sum_o g' W, sum_n g' s, sum_n g' H), each
    None where not requested (device, float32; see edge_linear_supported)."""
    hb = _cmp.has_base(base_weight)
    _check_edge_inputs(s, H, base_weight, W, hb)
    _req(edge_linear_supported(H, W), "edge_linear_backward: configuration not supported")
    N, I, R = H.shape
    O = W.shape[0]
    _req(tuple(grad_a.shape) == (O, I), "edge_linear_backward: grad_a shape")
    _req(tuple(grad_y.shape) == (N, O), "edge_linear_backward: grad_y shape")
    H, W = H.contiguous(), W.contiguous()
    ga = grad_a.contiguous().to(W.dtype)
    gy = grad_y.contiguous().to(W.dtype)
    sc = s.contiguous() if hb else None
    bw = base_weight.contiguous() if hb else None
    opts = dict(dtype=H.dtype, device=H.device)
    ds = torch.empty(N, I, **opts) if (need_s and hb) else None
    dH = torch.empty(N, I, R, **opts) if need_H else None
    dbw = torch.empty(O, I, **opts) if (need_bw and hb) else None
    dW = torch.empty(O, I, R, **opts) if need_W else None
    if ds is None and dH is None and dbw is None and dW is None:
        return ds, dH, dbw, dW
    code = dtype_code(H.dtype)
    nbytes = _lib.ctypes.c_size_t(0)
    with torch.cuda.device(H.device):
        check(LIB.kan_hip_edge_workspace(code, N, I, O, R, 1, _lib.ctypes.byref(nbytes)))
        ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=H.device)
        check(LIB.kan_hip_edge_linear_backward(
            code, ptr(ga), ptr(gy), ptr(sc), ptr(H), ptr(bw), ptr(W), ptr(ds), ptr(dH), ptr(dbw),
            ptr(dW), ptr(ws), int(nbytes.value), N, I, O, R, stream_of(H.device)))
    return ds, dH, dbw, dW


def edge_regularization(a: torch.Tensor, mu1: float, mu2: float):
    """(reg, ws): reg = mu1 * sum(a) + mu2 * entropy(a / sum(a)) as a 0-d
    device tensor, and the workspace holding the statistics its backward
    reads (kan_hip_edge_reg; spline_kan/reference_backend.py:149-170)."""
    _req(a.is_cuda and a.dtype in _F, "edge_regularization: a must be a float32/float64 CUDA tensor")
    a = a.contiguous()
    code = dtype_code(a.dtype)
    nb = _lib.ctypes.c_size_t(0)
    check(LIB.kan_hip_edge_reg_workspace(code, a.numel(), _lib.ctypes.byref(nb)))
    ws = torch.empty(int(nb.value), dtype=torch.uint8, device=a.device)
    reg = torch.empty((), dtype=a.dtype, device=a.device)
    with torch.cuda.device(a.device):
        check(LIB.kan_hip_edge_reg(code, ptr(a), a.numel(), float(mu1), float(mu2), ptr(reg),
                                   ptr(ws), int(nb.value), stream_of(a.device)))
    return reg, ws


def edge_regularization_backward(grad_reg: torch.Tensor, a: torch.Tensor, mu1: float, mu2: float,
                                 ws: torch.Tensor) -> torch.Tensor:
    """d reg / d a times grad_reg (0-d), from the workspace of the forward
    over the same a (kan_hip_edge_reg_backward)."""
    a = a.contiguous()
    g = grad_reg.reshape(()).to(a.dtype).contiguous()
    ga = torch.empty_like(a)
    with torch.cuda.device(a.device):
        check(LIB.kan_hip_edge_reg_backward(dtype_code(a.dtype), ptr(g), ptr(a), a.numel(),
                                            float(mu1), float(mu2), ptr(ws), ws.numel(), ptr(ga),
                                            stream_of(a.device)))
    return ga


def edge_abs_mean_double_backward(grad_a, s, H, base_weight, W, u_ds, u_dH, u_dbw, u_dW,
                                  need_ga: bool, need_s: bool, need_H: bool, need_bw: bool,
                                  need_W: bool):
    """Double backward of edge_abs_mean at a fixed sign pattern (device):
    gradients of <u_ds, ds> + <u_dH, dH> + <u_dbw, dbw> + <u_dW, dW> with
    respect to (ga, s, H, bw, W); any u may be None (zero).  Returns
    (g_ga, g_s, g_H, g_bw, g_W), None where not requested."""
    hb = _cmp.has_base(base_weight)
    _check_edge_inputs(s, H, base_weight, W, hb)
    N, I, R = H.shape
    O = W.shape[0]
    _req(tuple(grad_a.shape) == (O, I), "edge_abs_mean_double_backward: grad shape")
    cont = lambda t: None if t is None else t.contiguous().to(H.dtype)
    if not hb:
        u_ds = u_dbw = None
    H, W, ga = H.contiguous(), W.contiguous(), cont(grad_a)
    sc, bw = (cont(s), cont(base_weight)) if hb else (None, None)
    u_ds, u_dH, u_dbw, u_dW = cont(u_ds), cont(u_dH), cont(u_dbw), cont(u_dW)
    for u, shape in ((u_ds, (N, I)), (u_dH, (N, I, R)), (u_dbw, (O, I)), (u_dW, (O, I, R))):
        _req(u is None or tuple(u.shape) == shape, "edge_abs_mean_double_backward: gradient shape")
    opts = dict(dtype=H.dtype, device=H.device)
    outs = (torch.empty(O, I, **opts) if need_ga else None,
            torch.empty(N, I, **opts) if (need_s and hb) else None,
            torch.empty(N, I, R, **opts) if need_H else None,
            torch.empty(O, I, **opts) if (need_bw and hb) else None,
            torch.empty(O, I, R, **opts) if need_W else None)
    if any(t is not None for t in outs):
        g_ga, g_s, g_H, g_bw, g_W = outs
        code = dtype_code(H.dtype)
        nbytes = _lib.ctypes.c_size_t(0)
        with torch.cuda.device(H.device):
            check(LIB.kan_hip_edge_abs_mean_double_backward_workspace(
                code, N, I, O, R, _lib.ctypes.byref(nbytes)))
            ws = torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=H.device)
            check(LIB.kan_hip_edge_abs_mean_double_backward(
                code, ptr(ga), ptr(sc), ptr(H), ptr(bw), ptr(W), ptr(u_ds), ptr(u_dH),
                ptr(u_dbw), ptr(u_dW), ptr(g_ga), ptr(g_s), ptr(g_H), ptr(g_bw), ptr(g_W),
                ptr(ws), int(nbytes.value), N, I, O, R, stream_of(H.device)))
    return outs


def _edge_double_backward_dense(ga, s, H, bw, W, u_ds, u_dH, u_dbw, u_dW, needs):
    """The same double backward as differentiable PyTorch formulas (used when
    it is itself recorded, i.e. third order).  Builds the [n, O, I] signs."""
    n = H.shape[0]
    phi = torch.einsum("oir,nir->noi", W, H)
    if bw is not None:
        phi = s.unsqueeze(1) * bw.unsqueeze(0) + phi
    S = phi.sign().detach()
    g = S * ga.unsqueeze(0) / n
    need_ga, need_s, need_H, need_bw, need_W = needs
    g_ga = g_s = g_H = g_bw = g_W = None
    if need_ga:
        t = torch.zeros_like(phi)
        if u_dH is not None:
            t = t + torch.einsum("nir,oir->noi", u_dH, W)
        if u_dW is not None:
            t = t + torch.einsum("nir,oir->noi", H, u_dW)
        if bw is not None and u_ds is not None:
            t = t + u_ds.unsqueeze(1) * bw.unsqueeze(0)
        if bw is not None and u_dbw is not None:
            t = t + s.unsqueeze(1) * u_dbw.unsqueeze(0)
        g_ga = (S * t).sum(0) / n
    if need_bw and bw is not None and u_ds is not None:
        g_bw = (g * u_ds.unsqueeze(1)).sum(0)
    if need_W and u_dH is not None:
        g_W = torch.einsum("noi,nir->oir", g, u_dH)
    if need_s and bw is not None and u_dbw is not None:
        g_s = (g * u_dbw.unsqueeze(0)).sum(1)
    if need_H and u_dW is not None:
        g_H = torch.einsum("noi,oir->nir", g, u_dW)
    return g_ga, g_s, g_H, g_bw, g_W


class EdgeAbsMeanBackward(torch.autograd.Function):
    """(ds, dH, dbw, dW) of edge_abs_mean as a differentiable function of
    (ga, s, H, bw, W): the recorded backward of EdgeAbsMean.  Forward is the
    native first-order backward; backward is the native double backward
    (kan_hip_edge_abs_mean_double_backward, sign pattern fixed), so second
    derivatives of the regulariser, mixed input x weight terms included,
    never form the [n, O, I] edge tensor.  A third order (this backward
    recorded again) uses the dense formulas.  ds and dbw are empty tensors
    for a layer without a base branch."""

    @staticmethod
    def forward(ctx, ga, s, H, bw, W):
        hb = bw is not None
        ctx.hb = hb
        ctx.set_materialize_grads(False)
        empty = H.new_empty(0)
        ctx.save_for_backward(ga, s if hb else empty, H, bw if hb else empty, W)
        ds, dH, dbw, dW = edge_abs_mean_backward(ga, s, H, bw, W, hb, True, hb, True)
        if not hb:
            ds, dbw = empty.clone(), empty.clone()
            ctx.mark_non_differentiable(ds, dbw)
        return ds, dH, dbw, dW

    @staticmethod
    def backward(ctx, u_ds, u_dH, u_dbw, u_dW):
        ga, s, H, bw, W = ctx.saved_tensors
        if not ctx.hb:
            s = bw = None
            u_ds = u_dbw = None
        needs = tuple(bool(v) for v in ctx.needs_input_grad)
        if torch.is_grad_enabled():
            return _edge_double_backward_dense(ga, s, H, bw, W, u_ds, u_dH, u_dbw, u_dW, needs)
        return edge_abs_mean_double_backward(ga, s, H, bw, W, u_ds, u_dH, u_dbw, u_dW, *needs)


# ---------------------------------------------------------------------------
# op registry: torch.ops.spline_kan.kan_forward / kan_backward
# (TORCH_LIBRARY(spline_kan) with CPU, CUDA and Meta kernels,
# csrc/kan_ext.cpp:62-155)
# ---------------------------------------------------------------------------

_KAN_FORWARD_SCHEMA = (
    "kan_forward(Tensor x, Tensor grid, Tensor base_weight, Tensor spline_weight, "
    "Tensor spline_scaler, int spline_order, bool has_scaler) -> (Tensor output, Tensor basis)")
_KAN_BACKWARD_SCHEMA = (
    "kan_backward(Tensor grad_output, Tensor x, Tensor grid, Tensor base_weight, "
    "Tensor spline_weight, Tensor spline_scaler, Tensor basis, int spline_order, "
    "bool has_scaler) -> (Tensor grad_x, Tensor grad_base_weight, Tensor grad_spline_weight, "
    "Tensor grad_spline_scaler)")


def _kan_forward_meta(x, grid, base_weight, spline_weight, spline_scaler, spline_order,
                      has_scaler):
    """Shapes only: output [B, O], basis [B, I, R] with R = knots - k - 1."""
    B, I = x.shape[0], x.shape[1]
    O = spline_weight.shape[0]
    R = grid.shape[1] - spline_order - 1
    return x.new_empty((B, O)), x.new_empty((B, I, R))


def _kan_backward_meta(grad_output, x, grid, base_weight, spline_weight, spline_scaler, basis,
                       spline_order, has_scaler):
    """Shapes only; an absent base branch or scaler gives an undefined
    gradient (None in Python), as the CPU and device kernels return."""
    gbw = base_weight.new_empty(base_weight.shape) if _cmp.has_base(base_weight) else None
    gsc = spline_scaler.new_empty(spline_scaler.shape) if has_scaler else None
    return (x.new_empty(x.shape), gbw, spline_weight.new_empty(spline_weight.shape), gsc)


def _register_ops():
    """Defines the spline_kan ops once per process.  The CPU and CUDA kernels
    are kan_forward / kan_backward above (CPU: the ATen formulation; CUDA,
    i.e. ROCm device tensors: libkan_hip.so); Meta gives shapes for tracing
    and FakeTensor.  A second import of this module (a rebuilt package in
    the same process) finds the ops defined and keeps them."""
    try:
        torch._C._dispatch_find_schema_or_throw("spline_kan::kan_forward", "")
        return None
    except RuntimeError:
        pass
    lib = torch.library.Library("spline_kan", "DEF")
    lib.define(_KAN_FORWARD_SCHEMA)
    lib.define(_KAN_BACKWARD_SCHEMA)
    for key in ("CPU", "CUDA"):
        lib.impl("kan_forward", kan_forward, key)
        lib.impl("kan_backward", kan_backward, key)
    lib.impl("kan_forward", _kan_forward_meta, "Meta")
    lib.impl("kan_backward", _kan_backward_meta, "Meta")
    return lib


_OPS_LIBRARY = _register_ops()
