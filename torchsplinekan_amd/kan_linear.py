"""KANLinear: one B-spline KAN layer with a native gfx950 backend
(mirrors spline_kan/kan_linear.py: same constructor, backend selection,
attributes, forward, regularisation API and state_dict keys).

Backend selection (kan_linear.py:127-150, 193-213 of the reference):
  "auto"      native kernels for device inputs when the configuration is
              supported (grid_size + 2*spline_order <= 71, in_features <= 65535);
              the reference backend for CPU inputs and unsupported shapes.
  "cuda"      native kernels; raises if the library is missing, the shape is
              unsupported or the input is on the CPU.
  "reference" the pure-PyTorch backend.
With "auto" and libkan_hip.so not built, device inputs run on the reference
backend as in the reference; the first such forward emits a RuntimeWarning
naming the missing library, so the fallback is never silent.
"""

import copy
import warnings
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import fused as _fused
from .reference_backend import (
    ReferenceKANLayer,
    compute_basis,
    edge_abs_mean_dense,
    fit_spline_coeffs,
    regularization_from_edge_means,
)

_C = _fused._C
_CUDA_EXT_LOADED: bool = _C is not None

REG_IMPLS = ("auto", "dense", "fused", "checkpoint")

CUDA_MAX_DEG0_BASIS = int(getattr(_C, "CUDA_MAX_DEG0_BASIS", 71)) if _C is not None else 71
CUDA_MAX_IN_FEATURES = int(getattr(_C, "CUDA_MAX_IN_FEATURES", 65535)) if _C is not None else 65535


_MISSING_WARNED = False


def _warn_missing_library() -> None:
    """One RuntimeWarning per process when backend="auto" falls back to the
    reference backend on a device tensor because libkan_hip.so is missing
    (the reference falls back silently, spline_kan/kan_linear.py:147-148)."""
    global _MISSING_WARNED
    if not _MISSING_WARNED:
        _MISSING_WARNED = True
        warnings.warn("KANLinear(backend='auto'): libkan_hip.so is not built, so device inputs "
                      "run on the pure-PyTorch reference backend; build it with "
                      "`python -m torchsplinekan_amd.build_lib`", RuntimeWarning, stacklevel=3)


def native_config_supported(in_features: int, grid_size: int, spline_order: int) -> Tuple[bool, str]:
    """(ok, reason): whether the native kernels accept a layer shape."""
    if grid_size + 2 * spline_order > CUDA_MAX_DEG0_BASIS:
        return False, (f"grid_size + 2*spline_order = {grid_size + 2 * spline_order} exceeds the "
                       f"CUDA kernel limit of {CUDA_MAX_DEG0_BASIS}")
    if in_features > CUDA_MAX_IN_FEATURES:
        return False, (f"in_features = {in_features} exceeds the CUDA kernel limit of "
                       f"{CUDA_MAX_IN_FEATURES}")
    return True, ""


def _uniform_knot_rows(span: torch.Tensor, G: int, k: int) -> torch.Tensor:
    """[I, G+2k+1] knot rows with G equal intervals between span[:, 0] and
    span[:, 1] and k more of the same width beyond each end."""
    lo, hi = span.unbind(1)
    offsets = torch.arange(-k, G + k + 1, device=span.device, dtype=span.dtype)
    return lo[:, None] + offsets[None] * ((hi - lo) / G)[:, None]


def _interior_points(grid: torch.Tensor, G: int, k: int, count: int) -> torch.Tensor:
    """[count, I] evenly spaced points from t_k to t_{k+G} of every knot row."""
    a, b = grid[:, k], grid[:, k + G]
    frac = torch.linspace(0, 1, count, device=grid.device, dtype=grid.dtype)
    return a[None] + frac[:, None] * (b - a)[None]


def _index_list(index, size: int, name: str, device) -> torch.Tensor:
    """Long index tensor for KANLinear.select: None keeps all `size` entries;
    a boolean mask of length `size` keeps its True positions; integer indices
    must lie in [0, size)."""
    if index is None:
        return torch.arange(size, device=device)
    t = torch.as_tensor(index, device=device)
    if t.dtype == torch.bool:
        if t.dim() != 1 or t.numel() != size:
            raise ValueError(f"{name}: a boolean mask must have shape [{size}], "
                             f"got {list(t.shape)}")
        return t.nonzero().flatten()
    if t.is_floating_point() or t.is_complex():
        raise TypeError(f"{name}: expected integer indices or a boolean mask, got {t.dtype}")
    t = t.to(torch.long).flatten()
    if t.numel() and (int(t.min()) < 0 or int(t.max()) >= size):
        raise IndexError(f"{name}: indices must lie in [0, {size}), got "
                         f"[{int(t.min())}, {int(t.max())}]")
    return t


class KANLinear(nn.Module):
    """B-spline KAN layer.

    Attributes: base_weight [O, I], spline_weight [O, I, G+k],
    spline_scaler [O, I] (if enabled), grid buffer [I, G+2k+1].  The
    parameters are owned by an inner ReferenceKANLayer (``_ref``) and
    re-exposed here, so state_dicts carry both key sets, as the reference's.
    """

    def __init__(self, in_features: int, out_features: int, grid_size: int = 5,
                 spline_order: int = 3, scale_noise: float = 0.1, scale_base: float = 1.0,
                 scale_spline: float = 1.0, enable_standalone_scale_spline: bool = True,
                 base_activation=nn.SiLU, grid_eps: float = 0.02,
                 grid_range: Tuple[float, float] = (-1.0, 1.0), backend: str = "auto") -> None:
        super().__init__()
        if grid_size < 1:
            raise ValueError(f"grid_size must be >= 1, got {grid_size}")
        if spline_order not in (1, 2, 3):
            raise ValueError(f"spline_order must be 1, 2, or 3, got {spline_order}")
        if backend not in ("auto", "cuda", "reference"):
            raise ValueError(f"backend must be 'auto', 'cuda', or 'reference', got {backend!r}")
        native_ok, reason = native_config_supported(in_features, grid_size, spline_order)
        if backend == "cuda":
            if not _CUDA_EXT_LOADED:
                raise RuntimeError(
                    "backend='cuda' requested but the native extension (libkan_hip.so) could not "
                    "be loaded.  Build it first (python -m torchsplinekan_amd.build_lib) or use "
                    "backend='reference'.")
            if not native_ok:
                raise ValueError(
                    f"backend='cuda' does not support this configuration: {reason}. "
                    "Use backend='reference' (or 'auto', which falls back automatically).")
            self._use_cuda = True
        elif backend == "reference":
            self._use_cuda = False
        else:
            self._use_cuda = _CUDA_EXT_LOADED and native_ok
        self._native_ok = native_ok
        self.backend = backend
        self.last_backend: Optional[str] = None
        self._waug_cache = None  # (key, packed inference weight) of a frozen eval-mode layer

        self._ref = ReferenceKANLayer(
            in_features=in_features, out_features=out_features, grid_size=grid_size,
            spline_order=spline_order, scale_noise=scale_noise, scale_base=scale_base,
            scale_spline=scale_spline,
            enable_standalone_scale_spline=enable_standalone_scale_spline,
            base_activation=base_activation, grid_eps=grid_eps, grid_range=grid_range)
        self.base_weight = self._ref.base_weight
        self.spline_weight = self._ref.spline_weight
        if enable_standalone_scale_spline:
            self.spline_scaler = self._ref.spline_scaler
        self.register_buffer("grid", self._ref.grid)

        self.in_features = in_features
        self.out_features = out_features
        self.grid_size = grid_size
        self.spline_order = spline_order
        self.enable_standalone_scale_spline = enable_standalone_scale_spline

    # ------------------------------------------------------------------ backends

    @property
    def selected_backend(self) -> str:
        """Backend used for device inputs: "cuda" (native) or "reference"."""
        return "cuda" if self._use_cuda else "reference"

    def backend_for(self, x: torch.Tensor) -> str:
        """Backend that :meth:`forward` uses for input ``x``."""
        if not self._use_cuda:
            if (x.is_cuda and self.backend == "auto" and self._native_ok
                    and not _CUDA_EXT_LOADED):
                _warn_missing_library()
            return "reference"
        if self.backend == "cuda" or x.is_cuda:
            return "cuda"
        return "reference"

    @property
    def _native_fuses_base(self) -> bool:
        # The kernels fuse SiLU; other activations run in PyTorch.
        return type(self._ref.base_activation) is nn.SiLU

    # ------------------------------------------------------------------ forward

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        backend = self.backend_for(x)
        self.last_backend = backend
        if backend == "cuda":
            return self._cuda_forward(x)
        return self._ref(x)

    def _cuda_forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError(
                "KANLinear with backend='cuda' received a CPU tensor. Move the input and model "
                "to a CUDA device, or use backend='reference'.")
        lead = x.shape[:-1]
        xf = x.reshape(-1, self.in_features)
        has_scaler = self.enable_standalone_scale_spline
        empty = xf.new_empty(0)
        fuse_base = self._native_fuses_base
        if self._needs_autograd(xf):
            out = _C.kan_apply(xf, self.grid, self.base_weight if fuse_base else empty,
                               self.spline_weight, self.spline_scaler if has_scaler else empty,
                               self.spline_order, has_scaler)
        else:
            # inference: packed weight (cached in eval mode), no saved basis
            _C._check_inputs(xf, self.grid, self.base_weight if fuse_base else empty,
                             self.spline_weight, self.spline_scaler if has_scaler else empty,
                             self.spline_order, has_scaler)
            out = _C.kan_infer(xf, self.grid, self._packed_weight(fuse_base, has_scaler),
                               self.spline_order, fuse_base)
        if not fuse_base:
            out = out + F.linear(self._ref.base_activation(xf), self.base_weight)
        return out.reshape(lead + (self.out_features,))

    def _needs_autograd(self, xf: torch.Tensor) -> bool:
        if not torch.is_grad_enabled():
            return False
        return xf.requires_grad or any(p.requires_grad for p in self.parameters())

    def _packed_weight(self, fuse_base: bool, has_scaler: bool) -> torch.Tensor:
        """[spline_weight * scaler | base_weight] for kan_infer.

        A frozen layer in eval mode (what export_inference returns) keeps it
        between calls, keyed on each parameter's storage and version counter,
        so repeated inference skips the packing.  Writes through ``.data``
        bypass the version counter: call release_packed_weight() after them.
        Any other layer packs per call and keeps nothing."""
        params = [self.spline_weight] + ([self.spline_scaler] if has_scaler else []) + \
                 ([self.base_weight] if fuse_base else [])
        key = (fuse_base, has_scaler) + tuple((p.data_ptr(), p._version, p.dtype) for p in params)
        cache = getattr(self, "_waug_cache", None)
        if cache is not None and cache[0] == key:
            return cache[1]
        waug = _C.pack_weight(self.base_weight if fuse_base else None, self.spline_weight,
                              self.spline_scaler if has_scaler else None, self.spline_order,
                              has_scaler)
        frozen = not self.training and not any(p.requires_grad for p in self.parameters())
        self._waug_cache = (key, waug) if frozen else None
        return waug

    def release_packed_weight(self) -> None:
        """Drops the kept inference weight (rebuilt on the next inference call)."""
        self._waug_cache = None

    # ------------------------------------------------------------------ grid update

    @torch.no_grad()
    def update_grid(self, x: torch.Tensor, margin: float = 0.01) -> None:
        """Moves the knots to the data and refits spline_weight to the old
        (unscaled) curves by least squares, keeping both grid buffers in sync
        (spline_kan/kan_linear.py:260-269, reference_backend.py:443-493).

        On the native backend the refit runs on the device: the per-feature
        Gram matrices come from libkan_hip.so in one pass over the samples
        and the minimum-norm solve runs in float64 (refit.solve_min_norm);
        the [O, B, I] curve tensor is never formed.  Otherwise the reference
        path (CPU least squares) runs."""
        if self.backend_for(x) != "cuda":
            self._ref.update_grid(x, margin=margin)
            self.grid.copy_(self._ref.grid)
            return
        from . import refit as _refit
        xf = self._ref.check_update_grid_args(x, margin).to(self.grid)
        new_grid = self._ref.grid_from_samples(xf, self.grid_size, margin)
        gram, cross = _refit.refit_gram(xf, self.grid, new_grid, self.spline_order)
        coef = _refit.solve_min_norm(gram, cross, self.spline_weight)
        self._copy_grid_(new_grid)
        self.spline_weight.copy_(coef.to(self.spline_weight.dtype))

    @torch.no_grad()
    def extend_grid(self, new_grid_size: int, x: torch.Tensor, *, margin: float = 0.01,
                    adapt_knots: bool = False, ridge: float = 1e-12,
                    n_dense: int = 0) -> "KANLinear":
        """New layer with `new_grid_size` intervals whose spline coefficients
        are the ridge-regularised least-squares fit of this layer's current
        (unscaled) spline curves; base_weight, spline_scaler and the base
        activation are copied (spline_kan/kan_linear.py:503-587).

        Knots: uniform over the current interior [t_k, t_{k+G}] widened to the
        samples (+margin) where they fall outside it, clipped to the old knot
        span; or, with adapt_knots, from the sample quantile/uniform mix as in
        update_grid.  n_dense adds that many uniformly spaced fit points per
        feature over the new interior.  On the native backend, the fit's
        normal equations come from libkan_hip.so (refit.refit_gram on float64
        samples, as fit_spline_coeffs evaluates its basis in float64) and are
        solved on the device (refit.solve_ridge)."""
        if new_grid_size < 1:
            raise ValueError(f"new_grid_size must be >= 1, got {new_grid_size}")
        x_flat = x.reshape(-1, self.in_features).to(self.grid)
        if x_flat.shape[0] < 2:
            raise ValueError("extend_grid needs at least 2 samples")
        k = self.spline_order
        new = self.make_like(grid_size=new_grid_size)
        if adapt_knots:
            new_grid = new._ref.grid_from_samples(x_flat, new_grid_size, margin)
        else:
            new_grid = _uniform_knot_rows(self._extension_span(x_flat, margin), new_grid_size, k)
        fit_x = x_flat
        if n_dense > 0:
            fit_x = torch.cat([x_flat, _interior_points(new_grid, new_grid_size, k, n_dense)], 0)
        if (self.backend_for(x) == "cuda"
                and native_config_supported(self.in_features, new_grid_size, k)[0]):
            from . import refit as _refit
            gram, cross = _refit.refit_gram(fit_x.double(), self.grid.double(),
                                            new_grid.double(), k)
            coeffs = _refit.solve_ridge(gram, cross, self.spline_weight, ridge)
        else:
            curves = torch.einsum("bir,oir->obi", compute_basis(fit_x, self.grid, k),
                                  self.spline_weight)          # unscaled curves [O, B, I]
            coeffs = fit_spline_coeffs(fit_x, curves, new_grid, k, ridge=ridge)
        new.base_weight.copy_(self.base_weight)
        new.spline_weight.copy_(coeffs.to(new.spline_weight.dtype))
        if self.enable_standalone_scale_spline:
            new.spline_scaler.copy_(self.spline_scaler)
        new._copy_grid_(new_grid)
        return new.train(self.training)

    def _extension_span(self, x_flat: torch.Tensor, margin: float) -> torch.Tensor:
        """[I, 2] end points of extend_grid's uniform knots: the current
        interior [t_k, t_{k+G}], moved out to min(x) - margin (max(x) + margin)
        on a side where samples lie beyond it, and clipped to the outermost
        current knots, past which the current spline is identically zero
        (spline_kan/kan_linear.py:567-572)."""
        k, g = self.spline_order, self.grid
        interior = g[:, [k, k + self.grid_size]]
        xmin, xmax = torch.aminmax(x_flat, dim=0)
        outside = torch.stack((xmin < interior[:, 0], xmax > interior[:, 1]), 1)
        widened = torch.stack((xmin - margin, xmax + margin), 1)
        span = torch.where(outside, widened, interior)
        return torch.clamp(span, min=g[:, :1], max=g[:, -1:])

    # ------------------------------------------------------------------ regularisation

    def regularization_loss(self, reg_act: float = 1.0, reg_entropy: float = 1.0, *,
                            x: Optional[torch.Tensor] = None, mode: str = "activation",
                            reg_impl: str = "auto", chunk_size: int = 1024) -> torch.Tensor:
        """Scalar regulariser: activation-based (KAN paper; needs x) or the legacy
        coefficient-based penalty (spline_kan/kan_linear.py:275-334)."""
        if mode not in ("activation", "coefficient"):
            raise ValueError(f"mode must be 'activation' or 'coefficient', got {mode!r}")
        if mode == "coefficient":
            return self._ref.regularization_loss(regularize_activation=reg_act,
                                                 regularize_entropy=reg_entropy,
                                                 mode="coefficient")
        if x is None:
            return self._ref.regularization_loss(reg_act, reg_entropy, x=None)
        xf = x.reshape(-1, self.in_features)
        s = self._ref.base_activation(xf)
        impl = self._resolve_reg_impl(reg_impl, xf)
        H = self._basis(xf, impl)
        a = self._edge_abs_mean(xf, s, H, self._ref.effective_spline_weight(), impl, chunk_size)
        return self._regularization(a, reg_act, reg_entropy, impl)

    def forward_with_regularization(self, x: torch.Tensor, reg_act: float = 1.0,
                                    reg_entropy: float = 1.0, *, mode: str = "activation",
                                    reg_impl: str = "auto", chunk_size: int = 1024
                                    ) -> Tuple[torch.Tensor, torch.Tensor]:
        """(self(x), self.regularization_loss(reg_act, reg_entropy, x=x)) with the
        base activation and the basis evaluated once.  reg_impl: "auto" (fused
        when the native kernels run this layer on this input, else dense),
        "dense", "fused" (phi never stored) or "checkpoint" (chunked recompute)
        (spline_kan/kan_linear.py:340-389)."""
        if mode == "coefficient":
            return self(x), self.regularization_loss(reg_act, reg_entropy, mode="coefficient")
        if mode != "activation":
            raise ValueError(f"mode must be 'activation' or 'coefficient', got {mode!r}")
        lead = x.shape[:-1]
        xf = x.reshape(-1, self.in_features)
        impl = self._resolve_reg_impl(reg_impl, xf)
        if impl == "fused" and self._native_fuses_base and xf.shape[0] > 0:
            # SiLU and the basis from one pass over x (gradients likewise)
            s, H = _fused.native_basis_silu(xf, self.grid, self.spline_order)
        else:
            s = self._ref.base_activation(xf)
            H = self._basis(xf, impl)
        W = self._ref.effective_spline_weight()
        B, R = xf.shape[0], self.grid_size + self.spline_order
        a = None
        if impl == "fused" and B > 0 and _fused.edge_linear_applies(s, H, self.base_weight, W):
            # output and edge statistic as one function: its backward folds
            # dL/dy into the edge kernel (one launch for all four gradients)
            y, a = _fused.edge_linear(s, H, self.base_weight, W)
        elif impl == "fused" and B > 0:
            y = _fused.native_linear(s, self.base_weight, H.reshape(B, self.in_features * R),
                                     W.reshape(self.out_features, -1))
        else:
            y = F.linear(s, self.base_weight) + F.linear(H.reshape(B, self.in_features * R),
                                                         W.reshape(self.out_features, -1))
        self.last_backend = "cuda" if impl == "fused" else "reference"
        if a is None:
            a = self._edge_abs_mean(xf, s, H, W, impl, chunk_size)
        reg = self._regularization(a, reg_act, reg_entropy, impl)
        return y.reshape(lead + (self.out_features,)), reg

    @staticmethod
    def _regularization(a: torch.Tensor, reg_act: float, reg_entropy: float,
                        impl: str) -> torch.Tensor:
        """The scalar from the edge means: native on the fused path, the
        tensor expression otherwise."""
        if impl == "fused":
            return _fused.edge_regularization(a, reg_act, reg_entropy)
        return regularization_from_edge_means(a, reg_act, reg_entropy)

    def _resolve_reg_impl(self, reg_impl: str, x_flat: torch.Tensor) -> str:
        if reg_impl not in REG_IMPLS:
            raise ValueError(f"reg_impl must be one of {REG_IMPLS}, got {reg_impl!r}")
        native_ok = (_fused.HAS_FUSED_KERNELS and x_flat.is_cuda
                     and self.backend_for(x_flat) == "cuda")
        if reg_impl == "auto":
            return "fused" if native_ok else "dense"
        if reg_impl == "fused" and not native_ok:
            raise RuntimeError(
                "reg_impl='fused' needs the native CUDA kernels, a CUDA input and a layer "
                "configuration supported by backend='cuda'.  Use reg_impl='dense' or "
                "'checkpoint' instead.")
        return reg_impl

    def _basis(self, x_flat: torch.Tensor, impl: str) -> torch.Tensor:
        if impl == "fused":
            return _fused.native_basis(x_flat, self.grid, self.spline_order)
        return compute_basis(x_flat, self.grid, self.spline_order)

    def _edge_abs_mean(self, x_flat, s, H, W, impl, chunk_size):
        if impl == "fused":
            return _fused.edge_abs_mean(s, H, self.base_weight, W)
        if impl == "checkpoint":
            if chunk_size < 1:
                raise ValueError(f"chunk_size must be >= 1, got {chunk_size}")
            return _fused.edge_abs_mean_chunked(s, x_flat, self.grid, self.spline_order,
                                                self.base_weight, W, chunk_size)
        return edge_abs_mean_dense(s, H, self.base_weight, W)

    @torch.no_grad()
    def edge_l1(self, x: torch.Tensor) -> torch.Tensor:
        """Per-edge L1 norm mean_n |phi_{o,i}(x_n)| -> [O, I] (no grad)."""
        xf = x.reshape(-1, self.in_features)
        impl = self._resolve_reg_impl("auto", xf)
        s = self._ref.base_activation(xf)
        H = self._basis(xf, impl)
        return self._edge_abs_mean(xf, s, H, self._ref.effective_spline_weight(), impl, 1024)

    # ------------------------------------------------------------------ copies

    def make_like(self, in_features: Optional[int] = None, out_features: Optional[int] = None,
                  grid_size: Optional[int] = None,
                  enable_standalone_scale_spline: Optional[bool] = None) -> "KANLinear":
        """Freshly initialised layer with this layer's hyper-parameters, dtype and device."""
        ref = self._ref
        return KANLinear(
            self.in_features if in_features is None else in_features,
            self.out_features if out_features is None else out_features,
            grid_size=self.grid_size if grid_size is None else grid_size,
            spline_order=self.spline_order, scale_noise=ref.scale_noise,
            scale_base=ref.scale_base, scale_spline=ref.scale_spline,
            enable_standalone_scale_spline=(self.enable_standalone_scale_spline
                                            if enable_standalone_scale_spline is None
                                            else enable_standalone_scale_spline),
            base_activation=copy.deepcopy(ref.base_activation), grid_eps=ref.grid_eps,
            grid_range=ref.grid_range, backend=self.backend,
        ).to(device=self.grid.device, dtype=self.grid.dtype)

    @torch.no_grad()
    def _copy_grid_(self, grid: torch.Tensor) -> None:
        # .to()/.double() re-create buffers per module: keep both grids in sync.
        self.grid.copy_(grid)
        self._ref.grid.copy_(grid)

    @torch.no_grad()
    def select(self, out_index: Optional[torch.Tensor] = None,
               in_index: Optional[torch.Tensor] = None) -> "KANLinear":
        """Independent layer restricted to the given outputs and inputs (index
        tensors; None keeps all): the edges between them keep their weights,
        scaler and knot rows, so on those inputs each kept output equals the
        original's minus the removed inputs' edges.  Hyper-parameters,
        dtype, device, training mode and requires_grad follow this layer."""
        dev = self.grid.device
        oi = _index_list(out_index, self.out_features, "out_index", dev)
        ii = _index_list(in_index, self.in_features, "in_index", dev)
        new = self.make_like(in_features=int(ii.numel()), out_features=int(oi.numel()))
        edges = lambda t: t.index_select(0, oi).index_select(1, ii)
        new.base_weight.copy_(edges(self.base_weight))
        new.spline_weight.copy_(edges(self.spline_weight))
        if self.enable_standalone_scale_spline:
            new.spline_scaler.copy_(edges(self.spline_scaler))
        new._copy_grid_(self.grid.index_select(0, ii))
        new.requires_grad_(any(p.requires_grad for p in self.parameters()))
        return new.train(self.training)

    def export_inference(self, requires_grad: bool = False) -> "KANLinear":
        """Independent layer computing the same function with spline_scaler
        folded into spline_weight (enable_standalone_scale_spline=False)."""
        new = self.make_like(enable_standalone_scale_spline=False)
        with torch.no_grad():
            new.base_weight.copy_(self.base_weight)
            new.spline_weight.copy_(self._ref.effective_spline_weight())
            new._copy_grid_(self.grid)
        new.requires_grad_(requires_grad)
        return new.train(self.training and requires_grad)
