"""GPU parity of the native higher-order path: kan_hip_basis_deriv /
kan_hip_basis_deriv_contract and the recorded (create_graph=True) backward
built on them (BasisDeriv, DerivContract, kan_backward_composite_device),
against the oracle's basis_derivative_n / kan_edge_derivative
(oracle/kan_oracle.py), which tests/test_oracle_derivs.py pins.

Tolerances (normwise, max|u - v| / max|v|): fp64 1e-12 for derivative
values and contractions, 1e-10 for PINN quantities built on two or three
chained derivatives; fp32 2e-5 for derivative values of order <= 1 and 1e-4
for orders 2 and 3 (each derivative step divides by knot spacings, which
amplifies the float32 rounding of the lower-order values), against the fp64
oracle evaluated on the same fp32 operands.
"""

import numpy as np
import pytest
import torch

from oracle import kan_oracle as ko
from tests._util import make_grid, normwise, np64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C():
    from torchsplinekan_amd import _C
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return _C


def _tol(dtype, q):
    if dtype == torch.float64:
        return 1e-12
    return 2e-5 if q <= 1 else 1e-4


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("k,G,kind", [(1, 6, "uniform"), (2, 7, "nonuniform"),
                                      (3, 10, "uniform"), (3, 5, "repeated")])
def test_basis_derivatives_match_oracle(C, dtype, k, G, kind):
    print(f"basis_deriv k={k} G={G} {kind} {dtype}", flush=True)
    I, N = 37, 301
    grid = make_grid(I, G, k, kind, seed=G).to(dtype)
    g = torch.Generator().manual_seed(k)
    x = (torch.rand(N, I, generator=g, dtype=torch.float64) * 2.4 - 1.2).to(dtype)
    x[0, :5] = grid[:5, 0]                   # on the first knot
    x[1, :5] = grid[:5, -1]                  # on the last knot
    x[2, :5] = grid[:5, k + 2]               # on an interior knot
    gH = torch.randn(N, I, G + k, generator=g, dtype=torch.float64).to(dtype)
    xd, gd = x.cuda(), grid.cuda()
    for q in range(0, k + 2):
        ref = ko.basis_derivative_n(np64(x), np64(grid), k, q)
        got = np64(C.basis_deriv(xd, gd, k, q))
        if q > k:
            assert not got.any()
            continue
        assert normwise(got, ref) < _tol(dtype, q), q
        gx = np64(C.basis_deriv_contract(xd, gd, k, gH.cuda(), q))
        rgx = np.einsum("nir,nir->ni", np64(gH), ref)
        assert normwise(gx, rgx) < _tol(dtype, q), q
    # order 1 of the contraction is the first-order basis_grad, bit for bit
    assert torch.equal(C.basis_deriv_contract(xd, gd, k, gH.cuda(), 1),
                       C.basis_grad(xd, gd, k, gH.cuda()))
    assert torch.equal(C.basis_deriv(xd, gd, k, 0), C.basis(xd, gd, k))


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("k,G,kind", [(2, 7, "nonuniform"), (3, 10, "uniform")])
def test_scaled_and_base_derivative_terms_match_oracle(C, dtype, k, G, kind):
    """basis_deriv with a per-item factor, basis_deriv_contract with the SiLU
    base term and a factor, and silu_deriv, for every order the recorded
    backward reaches, against the oracle; order 1 with the base term and no
    factor is the first-order kernel (kan_hip_basis_silu_grad) bit for bit."""
    print(f"scaled/base derivative terms k={k} G={G} {kind} {dtype}", flush=True)
    I, N = 45, 257
    grid = make_grid(I, G, k, kind, seed=G + 1).to(dtype)
    g = torch.Generator().manual_seed(11 * k)
    x = (torch.rand(N, I, generator=g, dtype=torch.float64) * 2.4 - 1.2).to(dtype)
    gH = torch.randn(N, I, G + k, generator=g, dtype=torch.float64).to(dtype)
    gb = torch.randn(N, I, generator=g, dtype=torch.float64).to(dtype)
    w = (torch.rand(N, I, generator=g, dtype=torch.float64) + 0.5).to(dtype)
    xd, gd = x.cuda(), grid.cuda()
    xs = np64(x)
    for q in range(0, 5):
        silu_q = ko.silu_derivative(xs, q)
        tol = 1e-12 if dtype == torch.float64 else 1e-5
        assert normwise(np64(C.silu_deriv(xd, q)), silu_q) < tol, q
        assert normwise(np64(C.silu_deriv(xd, q, w.cuda())), np64(w) * silu_q) < tol, q
        Dq = ko.basis_derivative_n(xs, np64(grid), k, q)
        got = np64(C.basis_deriv(xd, gd, k, q, w.cuda()))
        ref = np64(w)[:, :, None] * Dq
        if q > k:
            assert not got.any()
        else:
            assert normwise(got, ref) < _tol(dtype, q), q
        gx = np64(C.basis_deriv_contract(xd, gd, k, gH.cuda(), q, gb.cuda(), w.cuda()))
        rgx = np64(w) * (np.einsum("nir,nir->ni", np64(gH), Dq) + np64(gb) * silu_q)
        assert normwise(gx, rgx) < max(_tol(dtype, q), tol), q
    assert torch.equal(C.basis_deriv_contract(xd, gd, k, gH.cuda(), 1, gb.cuda()),
                       C.basis_silu_grad(xd, gd, k, gH.cuda(), gb.cuda()))
    with pytest.raises(RuntimeError):
        C.silu_deriv(xd, 5)


def test_deriv_contract_gradients(C):
    """deriv_contract with the base term and a factor: first and second
    derivatives in every operand (gradcheck, gradgradcheck, float64)."""
    torch.manual_seed(2)
    I, N, G, k = 3, 9, 5, 3
    grid = make_grid(I, G, k, "nonuniform", seed=4).double().cuda()
    x = (torch.rand(N, I, dtype=torch.float64) * 1.6 - 0.8).cuda().requires_grad_()
    Gs = torch.randn(N, I, G + k, dtype=torch.float64).cuda().requires_grad_()
    Gb = torch.randn(N, I, dtype=torch.float64).cuda().requires_grad_()
    w = (torch.rand(N, I, dtype=torch.float64) + 0.5).cuda().requires_grad_()
    for q in (0, 1, 2):
        f = lambda a, b, c, d: C.deriv_contract(a, grid, b, k, q, c, d)
        assert torch.autograd.gradcheck(f, (x, Gs, Gb, w), eps=1e-6, atol=1e-6)
        assert torch.autograd.gradgradcheck(f, (x, Gs, Gb, w), eps=1e-6, atol=1e-5)
    h = lambda a, d: C.BasisDeriv.apply(a, grid, k, 1, d)
    assert torch.autograd.gradgradcheck(h, (x, w), eps=1e-6, atol=1e-5)
    s = lambda a, d: C.SiluDeriv.apply(a, 2, d)
    assert torch.autograd.gradgradcheck(s, (x, w), eps=1e-6, atol=1e-5)


def test_deriv_entry_points_reject_bad_orders(C):
    x = torch.rand(4, 3, device="cuda")
    grid = make_grid(3, 5, 3, "uniform").float().cuda()
    with pytest.raises(RuntimeError):
        C.basis_deriv(x, grid, 3, -1)
    with pytest.raises(RuntimeError):
        C.basis_deriv_contract(x, grid, 3, torch.zeros(4, 3, 8, device="cuda"), -2)


def _layer(I, O, G, k, dtype, seed=0):
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(seed)
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda").to("cuda", dtype)
    with torch.no_grad():
        L.spline_weight.normal_(0, 0.2)
        L.spline_scaler.uniform_(0.5, 1.5)
    return L


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-4)])
def test_pinn_derivatives_of_one_layer_match_oracle(C, dtype, tol):
    """u_x, u_xx and the parameter/input gradients of a loss on u_xx, through
    the native recorded backward, against closed forms of the oracle."""
    I, O, G, k, N = 5, 4, 8, 3, 257
    L = _layer(I, O, G, k, dtype)
    x = (torch.rand(N, I, device="cuda", dtype=dtype) * 1.8 - 0.9).requires_grad_()
    u = L(x)
    ux = torch.autograd.grad(u.sum(), x, create_graph=True)[0]
    uxx = torch.autograd.grad(ux.sum(), x, create_graph=True)[0]
    tgt = torch.randn(N, I, device="cuda", dtype=dtype)
    loss = ((uxx - tgt) ** 2).mean()
    loss.backward()
    a = lambda t: np64(t.detach())
    args = (a(x), a(L.grid), a(L.base_weight), a(L.spline_weight), a(L.spline_scaler), k)
    assert normwise(a(ux), ko.kan_edge_derivative(*args, 1).sum(1)) < tol
    r_uxx = ko.kan_edge_derivative(*args, 2).sum(1)
    assert normwise(a(uxx), r_uxx) < tol
    # d loss / d(.) with g = 2 (u_xx - tgt) / (N I): u_xx[n, i] = sum_o phi''_oi(x[n, i])
    gl = 2.0 * (r_uxx - a(tgt)) / (N * I)
    B2 = ko.basis_derivative_n(args[0], args[1], k, 2)
    r_gx = gl * ko.kan_edge_derivative(*args, 3).sum(1)
    r_gbw = np.einsum("ni,ni->i", gl, ko.silu_derivative(args[0], 2))[None].repeat(O, 0)
    dWeff = np.einsum("ni,nir->ir", gl, B2)[None].repeat(O, 0)
    r_gsw = args[4][:, :, None] * dWeff
    r_gsc = (args[3] * dWeff).sum(2)
    for got, ref in [(x.grad, r_gx), (L.base_weight.grad, r_gbw),
                     (L.spline_weight.grad, r_gsw), (L.spline_scaler.grad, r_gsc)]:
        assert normwise(a(got), ref) < tol


def test_recorded_backward_runs_native_kernels(C, monkeypatch):
    """The device create_graph path never evaluates the dense ATen basis."""
    from torchsplinekan_amd import _lib, composite, reference_backend

    def boom(*args, **kwargs):
        raise AssertionError("dense basis evaluated on the device create_graph path")

    for mod in (composite, reference_backend):
        monkeypatch.setattr(mod, "compute_basis", boom)
        monkeypatch.setattr(mod, "compute_basis_derivative", boom)
    L = _layer(6, 3, 5, 3, torch.float64, seed=1)
    x = (torch.rand(64, 6, device="cuda", dtype=torch.float64) * 1.6 - 0.8).requires_grad_()
    _lib.timing_enable(True)
    try:
        ux = torch.autograd.grad(L(x).sum(), x, create_graph=True)[0]
        uxx = torch.autograd.grad(ux.sum(), x, create_graph=True)[0]
        uxx.square().sum().backward()
        torch.cuda.synchronize()
        _, n_basis, _ = _lib.timing_read("basis")
        _, n_contract, _ = _lib.timing_read("basis_grad")
    finally:
        _lib.timing_enable(False)
    assert n_basis >= 1 and n_contract >= 3
    assert torch.isfinite(x.grad).all()


def test_gradgradcheck_native_layer(C):
    """Second derivatives with respect to x and every parameter, through the
    device recorded backward (float64)."""
    L = _layer(3, 2, 6, 3, torch.float64, seed=2)
    x = (torch.rand(20, 3, device="cuda", dtype=torch.float64) * 1.6 - 0.8).requires_grad_()
    assert torch.autograd.gradcheck(lambda t: L(t), (x,), eps=1e-6, atol=1e-6)
    assert torch.autograd.gradgradcheck(lambda t: L(t), (x,), eps=1e-6, atol=1e-5)
    sw = L.spline_weight.detach().clone().requires_grad_()
    bw = L.base_weight.detach().clone().requires_grad_()
    sc = L.spline_scaler.detach().clone().requires_grad_()
    f = lambda t, w, b, s: C.kan_apply(t, L.grid, b, w, s, 3, True)
    assert torch.autograd.gradgradcheck(f, (x, sw, bw, sc), eps=1e-6, atol=1e-5)


def test_pinn_two_layer_matches_reference_backend(C):
    """README's PDE example shape (KAN [1, 16, 1]): u_xx and the loss
    gradients on the device against the reference backend on the CPU
    (autograd through the dense recurrences), float64."""
    from torchsplinekan_amd import KAN
    torch.manual_seed(3)
    net = KAN([1, 16, 1], grid_size=5, backend="cuda").double()
    ref = KAN([1, 16, 1], grid_size=5, backend="reference").double()
    ref.load_state_dict(net.state_dict())
    net = net.cuda()
    xs = torch.linspace(-1, 1, 50, dtype=torch.float64).unsqueeze(1)
    tgt = torch.sin(3 * xs)

    def pde(model, x, t):
        x = x.clone().requires_grad_()
        u = model(x)
        ux = torch.autograd.grad(u.sum(), x, create_graph=True)[0]
        uxx = torch.autograd.grad(ux.sum(), x, create_graph=True)[0]
        loss = ((uxx - t) ** 2).mean()
        loss.backward()
        return uxx.detach(), x.grad

    uxx_d, gx_d = pde(net, xs.cuda(), tgt.cuda())
    uxx_r, gx_r = pde(ref, xs, tgt)
    assert normwise(np64(uxx_d), np64(uxx_r)) < 1e-10
    assert normwise(np64(gx_d), np64(gx_r)) < 1e-10
    for (n, p), (_, q) in zip(net.named_parameters(), ref.named_parameters()):
        assert normwise(np64(p.grad), np64(q.grad)) < 1e-10, n


@pytest.mark.timeout(900)
def test_pinn_workload_matches_reference_backend(C):
    """bench.py's PINN workload itself (KAN([2, 128, 128, 1]) G8 k3 fp64,
    N = 16384, the same draws): one step, u -> grad u -> Laplacian through
    create_graph -> MSE -> backward, on the native path against the
    reference backend on the CPU (autograd through the dense recurrences):
    the Laplacian, the loss and every parameter gradient at the fp64 bar."""
    from torchsplinekan_amd import KAN
    N, widths, G, k = 16384, [2, 128, 128, 1], 8, 3
    g = torch.Generator().manual_seed(0)
    x = torch.rand(N, 2, generator=g, dtype=torch.float64) * 1.8 - 0.9
    f = torch.sin(3 * x[:, :1]) * torch.cos(2 * x[:, 1:])
    torch.manual_seed(0)
    net = KAN(widths, grid_size=G, spline_order=k, backend="cuda").double()
    with torch.no_grad():
        for layer in net.layers:
            layer.spline_weight.normal_(0.0, 0.1, generator=g)
    ref = KAN(widths, grid_size=G, spline_order=k, backend="reference").double()
    ref.load_state_dict(net.state_dict())
    net = net.cuda()

    def step(model, xx, ff):
        xg = xx.clone().requires_grad_()
        u = model(xg)
        gu = torch.autograd.grad(u.sum(), xg, create_graph=True)[0]
        lap = (torch.autograd.grad(gu[:, 0].sum(), xg, create_graph=True)[0][:, 0]
               + torch.autograd.grad(gu[:, 1].sum(), xg, create_graph=True)[0][:, 1])
        loss = ((lap.unsqueeze(1) - ff) ** 2).mean()
        loss.backward()
        return lap.detach(), loss.detach()

    lap_d, loss_d = step(net, x.cuda(), f.cuda())
    assert all(l.last_backend == "cuda" for l in net.layers)
    lap_r, loss_r = step(ref, x, f)
    e = normwise(np64(lap_d), np64(lap_r))
    el = abs(loss_d.item() - loss_r.item()) / abs(loss_r.item())
    print(f"pinn workload: Laplacian {e:.2e}, loss {el:.2e}", flush=True)
    assert e < 1e-10 and el < 1e-10
    for (n, p), (_, q) in zip(net.named_parameters(), ref.named_parameters()):
        e = normwise(np64(p.grad), np64(q.grad))
        print(f"pinn workload: {n} grad {e:.2e}", flush=True)
        assert e < 1e-10, n


def _view(t, trans):
    """t itself, or the same values as the transpose of a row-major buffer."""
    return t.t().contiguous().t() if trans else t


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 1e-5)])
@pytest.mark.parametrize("M,K,N", [(5, 3, 7), (128, 16384, 1408), (300, 37, 19), (1, 10, 64),
                                   (64, 10, 1), (7, 0, 5), (257, 4100, 33),
                                   # thin products (an output side or K of at most 16)
                                   (4096, 2304, 10), (10, 4096, 2304), (4096, 10, 2304),
                                   (16, 777, 1001), (1003, 300, 16), (17, 300, 17),
                                   (3, 5000, 1), (1, 4099, 5), (513, 16, 77), (2, 17, 3),
                                   (4097, 1, 6)])
def test_native_matmul_matches_torch(C, dtype, tol, M, K, N):
    """kan_hip_matmul on all four transposition pairs, long-K (split),
    degenerate and thin shapes (an output side or a contraction of at most 16,
    as in a classifier's output layer, with ragged edges and split slices),
    against the float64 product of the same operands; two calls agree bit for
    bit."""
    print(f"matmul M={M} K={K} N={N} {dtype}", flush=True)
    g = torch.Generator().manual_seed(M + K + N)
    a = torch.randn(M, K, generator=g, dtype=torch.float64).to(dtype)
    b = torch.randn(K, N, generator=g, dtype=torch.float64).to(dtype)
    ref = np64(a) @ np64(b)
    for ta in (False, True):
        for tb in (False, True):
            c = C.matmul(_view(a.cuda(), ta), _view(b.cuda(), tb))
            if K == 0:
                assert not np64(c).any()
                continue
            assert normwise(np64(c), ref) < tol, (ta, tb)
            assert torch.equal(c, C.matmul(_view(a.cuda(), ta), _view(b.cuda(), tb)))


@pytest.mark.parametrize("tile", ["256x64", "128", "256", "256w4"])
@pytest.mark.parametrize("M,K,N", [(600, 5632, 64), (513, 407, 61), (16384, 64, 64),
                                   (333, 16384, 19), (64, 100, 3)])
def test_matmul_tile_configs_match_torch(C, routes, tile, M, K, N):
    """The fp32 tile configurations forced through the gemm_tile route on
    narrow products (N <= 64, the narrow 256x64 tile's range): ragged rows,
    K tails past the 32-deep slab, unaligned leading dimensions and split-K,
    all four transposition pairs, against the float64 product."""
    print(f"matmul tile={tile} M={M} K={K} N={N}", flush=True)
    routes.set_route("gemm_tile", routes.GEMM_TILES[tile])
    g = torch.Generator().manual_seed(M + 3 * K + N)
    a = torch.randn(M, K, generator=g, dtype=torch.float64).float()
    b = torch.randn(K, N, generator=g, dtype=torch.float64).float()
    ref = np64(a) @ np64(b)
    for ta in (False, True):
        for tb in (False, True):
            c = C.matmul(_view(a.cuda(), ta), _view(b.cuda(), tb))
            assert normwise(np64(c), ref) < 1e-5, (ta, tb)


@pytest.mark.parametrize("tile", [0, 1, 2, 3], ids=["256x128", "128x128", "128x128x32-pipelined",
                                             "64x64x32-pipelined"])
@pytest.mark.parametrize("M,K,N", [(256, 512, 256), (128, 64, 128), (300, 37, 129),
                                   (1000, 777, 555), (513, 1000, 300), (257, 4100, 33),
                                   (65, 33000, 70)])
def test_matmul_fp64_tile_configs_match_torch(C, routes, tile, M, K, N):
    """The float64 tile configurations forced through the gemm_tile route
    (0: 256x128 tiles of 8 waves, 1: 128x128 of 4 waves, both with 16-deep
    slabs; 2: the software-pipelined 128x128 tile with 32-deep slabs; 3: the
    pipelined 64x64 tile, two blocks per CU): whole
    tiles, ragged rows and columns, K tails past both slab depths, split-K on
    long contractions, all four transposition pairs, against the float64
    product at 1e-12; two calls agree bit for bit."""
    print(f"matmul fp64 tile={tile} M={M} K={K} N={N}", flush=True)
    routes.set_route("gemm_tile", tile)
    g = torch.Generator().manual_seed(M + 5 * K + N)
    a = torch.randn(M, K, generator=g, dtype=torch.float64)
    b = torch.randn(K, N, generator=g, dtype=torch.float64)
    ref = np64(a) @ np64(b)
    for ta in (False, True):
        for tb in (False, True):
            c = C.matmul(_view(a.cuda(), ta), _view(b.cuda(), tb))
            assert normwise(np64(c), ref) < 1e-12, (ta, tb)
            assert torch.equal(c, C.matmul(_view(a.cuda(), ta), _view(b.cuda(), tb)))


def test_matmul_whole_tiles_with_wide_leading_dimension(C):
    """Whole tiles whose slab span exceeds 31-bit byte offsets (row stride
    2^21 + 64 floats: 256 rows span 2 GiB) take the guarded loads instead of
    the buffer-resource ones; both transposition routes of A, against the
    float64 product (2.1 GB operand buffer)."""
    ld = (1 << 21) + 64
    M, K, N = 256, 96, 64
    print(f"matmul wide ld={ld}", flush=True)
    buf = torch.empty(M, ld, device="cuda")
    a = buf[:, :K]
    g = torch.Generator().manual_seed(7)
    a.copy_(torch.randn(M, K, generator=g))
    b = torch.randn(K, N, generator=g).cuda()
    ref = np64(a.cpu()) @ np64(b.cpu())
    assert normwise(np64(C.matmul(a, b)), ref) < 1e-5
    bt = torch.empty(N, ld, device="cuda")[:, :K]
    bt.copy_(b.t())
    assert normwise(np64(C.matmul(a, bt.t())), ref) < 1e-5
    del buf, bt
    torch.cuda.empty_cache()


def test_native_matmul_gradients_and_workspace_check(C):
    from torchsplinekan_amd import _lib
    a = torch.randn(9, 6, device="cuda", dtype=torch.float64, requires_grad=True)
    b = torch.randn(6, 4, device="cuda", dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(C.NativeMatmul.apply, (a, b))
    assert torch.autograd.gradgradcheck(C.NativeMatmul.apply, (a, b))
    # a split product refuses a short workspace before launching anything
    M, N, K = 64, 64, 1 << 16
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.check(_lib.LIB.kan_hip_matmul_workspace(_lib.dtype_code(torch.float32), 0, 0, M, N, K,
                                                 _lib.ctypes.byref(nbytes)))
    assert nbytes.value > 0
    x = torch.zeros(M, K, device="cuda")
    y = torch.zeros(K, N, device="cuda")
    z = torch.empty(M, N, device="cuda")
    rc = _lib.LIB.kan_hip_matmul(_lib.dtype_code(torch.float32), 0, 0, M, N, K, _lib.ptr(x), K,
                                 _lib.ptr(y), N, _lib.ptr(z), N, None, 0, None)
    assert rc != 0
