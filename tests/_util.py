"""Shared helpers of the test suite: seeded knot rows and sample points in
the style of the reference's own tests (tests/test_local_basis.py:19-37,
tests/test_math_correctness.py:23-44), and the normwise error metric of
tests/test_fused_regularization.py:36-39."""

import numpy as np
import torch


def make_grid(I, G, k, kind, seed=0, dtype=torch.float64):
    """Knot rows [I, G+2k+1]: "uniform" on [-1, 1] extended by k knots per
    side, "nonuniform" (random positive gaps in [0.1, 1)), or "repeated"
    (nonuniform with one zero-length interior span)."""
    g = torch.Generator().manual_seed(seed)
    n = G + 2 * k + 1
    if kind == "uniform":
        t = -1 + (torch.arange(n, dtype=torch.float64) - k) * 2 / G
        return t[None].expand(I, -1).contiguous().to(dtype)
    gaps = torch.rand(I, n - 1, generator=g, dtype=torch.float64) * 0.9 + 0.1
    if kind == "repeated":
        gaps[:, k + G // 2] = 0.0
    t = torch.cat([torch.zeros(I, 1, dtype=torch.float64), gaps.cumsum(1)], 1)
    return (t - t[:, k:k + 1] - 1.0).to(dtype)


def make_points(grid, n=3000, seed=0):
    """n random points 20 % beyond the knot span on each side, followed by
    every knot exactly (both ends included) -> [n + nk, I]."""
    g = torch.Generator().manual_seed(seed)
    lo, hi = grid[:, 0].min().item(), grid[:, -1].max().item()
    span = hi - lo
    x = torch.rand(n, grid.shape[0], generator=g, dtype=torch.float64) * 1.4 * span + lo - 0.2 * span
    return torch.cat([x, grid.t().to(torch.float64)], 0).to(grid.dtype)


def normwise(u, v):
    """max|u - v| / max|v| (0 when both vanish)."""
    u = np.asarray(u, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    den = np.abs(v).max() if v.size else 0.0
    num = np.abs(u - v).max() if v.size else 0.0
    if den == 0.0:
        return num
    return num / den


def np64(t):
    return t.detach().cpu().double().numpy()
