"""Writes tests/golden/reference_vectors.npz from the reference implementation.

Run once in the build container (the reference tree is not present on the GPU
box):  python tests/golden/make_golden.py /root/reference

What it records (inputs and outputs only):
  * compute_basis (spline_kan/reference_backend.py:32-96) in float32 and
    float64 for k = 1, 2, 3 on uniform, nonuniform and repeated-knot grids,
    with points beyond both ends and on every knot -- this pins the exact
    float32 rounding sequence of the reference backend, which no closed form
    fixes;
  * compute_basis_derivative (reference_backend.py:99-125) on the same points;
  * config 1: ReferenceKANLayer(16 -> 8, G=5, k=3)
    fp32 forward + backward of sum(y * D) on the reference backend, with the
    layer's parameters set from seeded draws (so the RNG order of the
    reference's reset_parameters does not matter), in float32 and float64;
  * ReferenceKANLayer.update_grid (reference_backend.py:443-493) on a
    two-component mixture, in float32 and float64 -- the knots pin the exact
    rounding of grid_from_samples and the coefficients curve2coeff's
    least-squares solution -- and on a rank-deficient input (two distinct
    values per feature), where lstsq's minimum-norm choice matters;
  * fit_spline_coeffs (reference_backend.py:173-215) refitting the old curves
    onto a uniformly refined grid (the fit behind KANLinear.extend_grid).
"""

import importlib.util
import os
import sys

import numpy as np
import torch


def load_reference_backend(root):
    path = os.path.join(root, "spline_kan", "reference_backend.py")
    spec = importlib.util.spec_from_file_location("ref_reference_backend", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def grids(I, G, k, kind, seed):
    g = torch.Generator().manual_seed(seed)
    n = G + 2 * k + 1
    if kind == "uniform":
        r = torch.arange(n, dtype=torch.float32)
        return (-1.0 + (r - k) * 2.0 / G)[None].expand(I, -1).contiguous()
    gaps = torch.rand(I, n - 1, generator=g, dtype=torch.float64) * 0.9 + 0.1
    if kind == "repeated":
        gaps[:, k + G // 2] = 0.0
    t = torch.cat([torch.zeros(I, 1, dtype=torch.float64), gaps.cumsum(1)], 1)
    return (t - t[:, k:k + 1] - 1.0).float()


def points(grid, n, seed):
    g = torch.Generator().manual_seed(seed)
    lo, hi = grid[:, 0].min().item(), grid[:, -1].max().item()
    span = hi - lo
    x = torch.rand(n, grid.shape[0], generator=g) * 1.4 * span + lo - 0.2 * span
    return torch.cat([x, grid.t()], 0)


def main(root):
    rb = load_reference_backend(root)
    out = {}
    for k in (1, 2, 3):
        for kind in ("uniform", "nonuniform", "repeated"):
            grid = grids(3, 6, k, kind, seed=10 * k + len(kind))
            x = points(grid, 200, seed=k)
            tag = f"basis_k{k}_{kind}"
            out[tag + "_grid"] = grid.numpy()
            out[tag + "_x"] = x.numpy()
            out[tag + "_H32"] = rb.compute_basis(x, grid, k).numpy()
            out[tag + "_H64"] = rb.compute_basis(x.double(), grid.double(), k).numpy()
            out[tag + "_dH64"] = rb.compute_basis_derivative(x.double(), grid.double(), k).numpy()

    # config 1
    g = torch.Generator().manual_seed(0)
    N, I, O, G, k = 32, 16, 8, 5, 3
    x = torch.rand(N, I, generator=g) * 2 - 1
    coef = torch.randn(O, I, G + k, generator=g) * 0.1
    bw = (torch.rand(O, I, generator=g) * 2 - 1) / (I ** 0.5)
    D = torch.randn(N, O, generator=g)
    out.update(c1_x=x.numpy(), c1_coef=coef.numpy(), c1_bw=bw.numpy(), c1_D=D.numpy())
    for dt, tag in ((torch.float32, "32"), (torch.float64, "64")):
        layer = rb.ReferenceKANLayer(I, O, grid_size=G, spline_order=k).to(dt)
        with torch.no_grad():
            layer.spline_weight.copy_(coef)
            layer.base_weight.copy_(bw)
            layer.spline_scaler.fill_(1.0)
        xx = x.to(dt).clone().requires_grad_()
        y = layer(xx)
        (y * D.to(dt)).sum().backward()
        out["c1_grid" + tag] = layer.grid.detach().numpy()
        out["c1_y" + tag] = y.detach().numpy()
        out["c1_gx" + tag] = xx.grad.numpy()
        out["c1_gbw" + tag] = layer.base_weight.grad.numpy()
        out["c1_gsw" + tag] = layer.spline_weight.grad.numpy()
        out["c1_gsc" + tag] = layer.spline_scaler.grad.numpy()

    # update_grid: knots from a two-component mixture, curves refitted
    g = torch.Generator().manual_seed(5)
    B, I, O, G, k = 200, 3, 2, 5, 3
    comp = torch.randint(0, 2, (B, I), generator=g)
    xu = torch.where(comp == 0, -0.5, 0.6) + 0.15 * torch.randn(B, I, generator=g)
    coef_u = torch.randn(O, I, G + k, generator=g) * 0.1
    out.update(ug_x=xu.numpy(), ug_coef=coef_u.numpy())
    for dt, tag in ((torch.float32, "32"), (torch.float64, "64")):
        layer = rb.ReferenceKANLayer(I, O, grid_size=G, spline_order=k).to(dt)
        with torch.no_grad():
            layer.spline_weight.copy_(coef_u.to(dt))
        out["ug_grid_old" + tag] = layer.grid.numpy().copy()
        out["ug_grid_eps"] = np.array(layer.grid_eps)
        layer.update_grid(xu.to(dt), margin=0.01)
        out["ug_grid" + tag] = layer.grid.numpy().copy()
        out["ug_sw" + tag] = layer.spline_weight.detach().numpy().copy()

    # rank-deficient update: every feature takes only the values -1 and +1
    xr = torch.where(torch.arange(60)[:, None] < 30, -1.0, 1.0).double().expand(60, 4).contiguous()
    coef_r = torch.randn(2, 4, 4 + 2, generator=g, dtype=torch.float64) * 0.1
    layer = rb.ReferenceKANLayer(4, 2, grid_size=4, spline_order=2).double()
    with torch.no_grad():
        layer.spline_weight.copy_(coef_r)
    out["rd_grid_old"] = layer.grid.numpy().copy()
    layer.update_grid(xr, margin=0.05)
    out.update(rd_x=xr.numpy(), rd_coef=coef_r.numpy(), rd_grid=layer.grid.numpy().copy(),
               rd_sw=layer.spline_weight.detach().numpy().copy())

    # fit_spline_coeffs onto a uniform refinement (G = 5 -> 10) of config 1's grid
    x64 = torch.rand(300, 3, generator=g, dtype=torch.float64) * 2 - 1
    grid_old = torch.linspace(-1 - 3 * 0.4, 1 + 3 * 0.4, 12, dtype=torch.float64)[None].repeat(3, 1)
    coef_f = torch.randn(2, 3, 8, generator=g, dtype=torch.float64) * 0.1
    grid_new = torch.linspace(-1 - 3 * 0.2, 1 + 3 * 0.2, 17, dtype=torch.float64)[None].repeat(3, 1)
    y_old = torch.einsum("oir,bir->obi", coef_f, rb.compute_basis(x64, grid_old, 3))
    out.update(fs_x=x64.numpy(), fs_grid_old=grid_old.numpy(), fs_coef=coef_f.numpy(),
               fs_grid_new=grid_new.numpy(),
               fs_sw=rb.fit_spline_coeffs(x64, y_old, grid_new, 3, ridge=1e-12).numpy())

    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
