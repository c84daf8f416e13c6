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
    reference's reset_parameters does not matter), in float32 and float64.
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
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
