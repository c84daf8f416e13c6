"""GPU parity of the native refit behind update_grid and extend_grid:
kan_hip_refit_gram (per-feature Gram and cross matrices, one pass over the
samples) and the float64 device solves, against the oracle
(oracle/kan_oracle.py: refit_gram, update_grid, curve2coeff,
fit_spline_coeffs) and the reference's golden vectors.

Tolerances (normwise, max|u - v| / max|v|):
  * Gram/cross matrices: fp64 inputs 1e-13; fp32 inputs 1e-6 (the device
    evaluates the fp32 basis with the local recurrence, the oracle with the
    dense one: both round differently at the last bit);
  * refitted coefficients: fp64 1e-10 (normal equations carry cond(A)^2 * eps,
    cond(A) <= 60 here, against lstsq's cond(A) * eps); fp32 1e-5.
"""

import os

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests._util import make_grid, normwise, np64

pytestmark = pytest.mark.gpu

GOLD = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                            "reference_vectors.npz"))


def _mixture(n, I, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    means = torch.tensor([-0.8, -0.5, 0.5, 0.8], dtype=torch.float64)
    comp = torch.randint(0, 4, (n, I), generator=g)
    return (means[comp] + 0.1 * torch.randn(n, I, generator=g, dtype=torch.float64)).to(dtype)


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-13), (torch.float32, 1e-6)])
@pytest.mark.parametrize("k,Go,Gn,kind", [(3, 5, 8, "uniform"), (2, 7, 4, "nonuniform"),
                                          (1, 6, 12, "repeated"), (3, 65, 20, "uniform")])
def test_refit_gram_matches_oracle(dtype, tol, k, Go, Gn, kind):
    from torchsplinekan_amd import refit
    print(f"refit_gram k={k} Go={Go} Gn={Gn} {kind} {dtype}", flush=True)
    I = 6
    g_old = make_grid(I, Go, k, kind, seed=Go).to(dtype)
    g_new = make_grid(I, Gn, k, "uniform").to(dtype) * 1.05
    x = (torch.rand(700, I, generator=torch.Generator().manual_seed(k), dtype=torch.float64)
         * 2.6 - 1.3).to(dtype)
    G, C = refit.refit_gram(x.cuda(), g_old.cuda(), g_new.cuda(), k)
    rG, rC = ko.refit_gram(np64(x), np64(g_old), np64(g_new), k)
    assert normwise(np64(G), rG) < tol and normwise(np64(C), rC) < tol
    # empty sample set: zero matrices
    G0, C0 = refit.refit_gram(x[:0].cuda(), g_old.cuda(), g_new.cuda(), k)
    assert G0.abs().max().item() == 0.0 and C0.abs().max().item() == 0.0


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-5)])
def test_update_grid_on_device_matches_oracle(dtype, tol):
    from torchsplinekan_amd import KANLinear, _lib
    I, O, G, k = 48, 24, 8, 3
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda").to(dtype)
    with torch.no_grad():
        L.spline_weight.copy_(torch.randn(O, I, G + k, generator=torch.Generator().manual_seed(1),
                                          dtype=dtype) * 0.1)
    x = _mixture(4096, I, seed=2, dtype=dtype)
    a = lambda t: t.detach().cpu().numpy()
    grid_ref, sw_ref = ko.update_grid(a(x), a(L.grid), a(L.spline_weight), G, k,
                                      L._ref.grid_eps, 0.01)
    L = L.cuda()
    _lib.timing_enable(True)
    L.update_grid(x.cuda(), margin=0.01)
    torch.cuda.synchronize()
    _, launches, _ = _lib.timing_read("other")
    _lib.timing_enable(False)
    assert launches >= 1                                   # the native Gram kernel ran
    assert torch.equal(L.grid, L._ref.grid)
    assert normwise(np64(L.grid), grid_ref) < (1e-15 if dtype == torch.float64 else 1e-6)
    assert normwise(np64(L.spline_weight), sw_ref) < tol


@pytest.mark.timeout(900)
def test_update_grid_refit_workload_matches_oracle():
    """bench.py's refit workload itself (KANLinear 512 -> 512 G8 k3 fp32,
    update_grid on N = 16384 samples of the Gaussian mixture, the same
    draws): every knot and every refitted coefficient against the oracle's
    update_grid, run one feature at a time (the refit is separable over
    features) in threads; knots at 1e-6, coefficients block by block (64
    outputs x 16 features) at 1e-5."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits
    from torchsplinekan_amd import KANLinear
    from tests._fullcheck import block_error
    from tests._netcheck import WORKERS
    N, I, O, G, k = 16384, 512, 512, 8, 3
    g = torch.Generator().manual_seed(0)
    means = torch.tensor([-0.8, -0.5, 0.5, 0.8])
    x = means[torch.randint(0, 4, (N, I), generator=g)] + 0.1 * torch.randn(N, I, generator=g)
    coef = torch.randn(O, I, G + k, generator=g) * 0.1
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda")
    with torch.no_grad():
        L.spline_weight.copy_(coef)
    grid0, eps = L.grid.detach().numpy().copy(), L._ref.grid_eps
    L = L.cuda()
    L.update_grid(x.cuda())
    torch.cuda.synchronize()
    xs, cs = x.numpy(), coef.numpy()

    def one(i):
        return ko.update_grid(xs[:, i:i + 1], grid0[i:i + 1], cs[:, i:i + 1], G, k, eps, 0.01)

    with threadpool_limits(limits=1, user_api="blas"):
        with ThreadPoolExecutor(WORKERS) as ex:
            parts = list(ex.map(one, range(I)))
    grid_ref = np.concatenate([p[0] for p in parts], axis=0)
    sw_ref = np.concatenate([p[1] for p in parts], axis=1)
    e = normwise(np64(L.grid), grid_ref)
    worst, block, whole = block_error(np64(L.spline_weight).reshape(O, -1),
                                      sw_ref.reshape(O, -1), 64, 16 * (G + k))
    print(f"refit workload: knots {e:.2e}; coefficients whole {whole:.2e}, worst block "
          f"{worst:.2e} at {block}", flush=True)
    assert e < 1e-6
    assert worst < 1e-5


@pytest.mark.parametrize("tag,dtype,tol", [("32", torch.float32, 1e-5), ("64", torch.float64, 1e-10)])
def test_update_grid_golden_on_device(tag, dtype, tol):
    from torchsplinekan_amd import KANLinear
    L = KANLinear(3, 2, grid_size=5, spline_order=3, backend="cuda").to(dtype)
    with torch.no_grad():
        L.spline_weight.copy_(torch.from_numpy(GOLD["ug_coef"]).to(dtype))
    assert np.array_equal(np64(L.grid), GOLD["ug_grid_old" + tag].astype(np.float64))
    L = L.cuda()
    L.update_grid(torch.from_numpy(GOLD["ug_x"]).to(dtype).cuda(), margin=0.01)
    assert normwise(np64(L.grid), GOLD["ug_grid" + tag]) < (1e-6 if tag == "32" else 1e-15)
    assert normwise(np64(L.spline_weight), GOLD["ug_sw" + tag]) < tol


def test_update_grid_rank_deficient_is_minimum_norm():
    """x takes two values per feature: the device result is the minimum-norm
    least-squares solution (the oracle's), not the reference's gelsy output."""
    from torchsplinekan_amd import KANLinear
    L = KANLinear(4, 2, grid_size=4, spline_order=2, backend="cuda").double()
    with torch.no_grad():
        L.spline_weight.copy_(torch.from_numpy(GOLD["rd_coef"]))
    L = L.cuda()
    x = GOLD["rd_x"]
    L.update_grid(torch.from_numpy(x).cuda(), margin=0.05)
    grid_ref, sw_ref = ko.update_grid(x, GOLD["rd_grid_old"], GOLD["rd_coef"], 4, 2,
                                      L._ref.grid_eps, 0.05)
    assert normwise(np64(L.grid), grid_ref) < 1e-15
    assert np.abs(np64(L.spline_weight) - sw_ref).max() < 1e-8


@pytest.mark.parametrize("adapt", [False, True])
def test_extend_grid_on_device_matches_oracle(adapt):
    from torchsplinekan_amd import KAN, KANLinear
    I, O, G, k = 16, 8, 5, 3
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda").double()
    with torch.no_grad():
        L.spline_weight.copy_(torch.randn(O, I, G + k, generator=torch.Generator().manual_seed(3),
                                          dtype=torch.float64) * 0.1)
    L = L.cuda()
    if adapt:
        x = _mixture(2000, I, seed=4).cuda()
    else:   # inside the interior: G 5 -> 10 keeps the old knots, so the fit is exact
        x = (torch.rand(2000, I, generator=torch.Generator().manual_seed(4),
                        dtype=torch.float64) * 1.9 - 0.95).cuda()
    new = L.extend_grid(10, x, adapt_knots=adapt, n_dense=50 if adapt else 0)
    assert new.grid_size == 10 and new.spline_weight.shape == (O, I, 10 + k)
    xs = x
    if adapt:
        lo, hi = new.grid[:, k], new.grid[:, k + 10]
        t = torch.linspace(0, 1, 50, device=x.device, dtype=x.dtype)
        xs = torch.cat([x, lo[None] + t[:, None] * (hi - lo)[None]], 0)
    y_old = np.einsum("oir,bir->obi", np64(L.spline_weight), ko.basis_dense(np64(xs), np64(L.grid), k))
    ref = ko.fit_spline_coeffs(np64(xs), y_old, np64(new.grid), k, 1e-12)
    assert normwise(np64(new.spline_weight), ref) < 1e-10
    if not adapt:
        xt = (torch.rand(128, I, dtype=torch.float64) * 1.8 - 0.9).cuda()
        assert torch.allclose(new(xt), L(xt), atol=1e-9)
    net = KAN([I, 6, 3], grid_size=G, backend="cuda").double().cuda()
    fine = net.extend_grid(10, x)
    assert all(l.grid_size == 10 for l in fine.layers)
