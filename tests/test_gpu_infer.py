"""GPU parity of the inference path (kan_hip_pack_weight + kan_hip_infer and
KANLinear's no-autograd forward): the packed weight is built once for a
frozen eval-mode layer (export_inference), the basis is never kept, and
small batches split the product over K.

Checked against the oracle's kan_forward (oracle/kan_oracle.py, after
csrc/kan_cpu.cpp:136-173) at the forward tolerances: fp64 1e-12 and fp32
1e-5 normwise."""

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


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 1e-5)])
@pytest.mark.parametrize("N,I,O,G,k,base,scaler", [
    (1, 1024, 1024, 10, 3, True, True),      # single sample: the product splits over K
    (3, 200, 96, 7, 2, True, False),
    (64, 512, 512, 8, 3, False, True),
    (700, 33, 19, 5, 1, True, True),
])
def test_infer_matches_oracle(C, dtype, tol, N, I, O, G, k, base, scaler):
    print(f"infer N={N} I={I} O={O} G={G} k={k} base={base} scaler={scaler} {dtype}", flush=True)
    g = torch.Generator().manual_seed(N + I)
    grid = make_grid(I, G, k, "nonuniform", seed=G).to(dtype)
    x = ((torch.rand(N, I, generator=g, dtype=torch.float64) * 2.2 - 1.1)).to(dtype)
    sw = (torch.randn(O, I, G + k, generator=g, dtype=torch.float64) * 0.1).to(dtype)
    bw = ((torch.rand(O, I, generator=g, dtype=torch.float64) * 2 - 1) / np.sqrt(I)).to(dtype)
    sc = (torch.rand(O, I, generator=g, dtype=torch.float64) + 0.5).to(dtype)
    d = lambda t: t.cuda() if t is not None else None
    waug = C.pack_weight(d(bw) if base else None, d(sw), d(sc) if scaler else None, k, scaler)
    y = C.kan_infer(d(x), d(grid), waug, k, base)
    ry, _ = ko.kan_forward(np64(x), np64(grid), np64(bw) if base else None, np64(sw),
                           np64(sc) if scaler else None, k)
    assert normwise(np64(y), ry) < tol
    # same output as the training forward up to the summation order of split products
    yf, _ = C.kan_forward(d(x), d(grid), d(bw) if base else torch.empty(0, device="cuda"),
                          d(sw), d(sc) if scaler else torch.empty(0, device="cuda"), k, scaler)
    assert normwise(np64(y), np64(yf)) < tol


@pytest.mark.timeout(900)
def test_infer_c3_layer_every_output(C):
    """bench.py's inference workload itself: c3's layer (KANLinear 1024 ->
    1024 G10 k3 fp32, the same draws) exported, at N = 65536, through
    kan_hip_infer with the packed weight: every output against the oracle,
    in 256 x 256 blocks (tests/_fullcheck.py, block_error), at 1e-5."""
    from torchsplinekan_amd import KANLinear
    from tests._fullcheck import block_error
    from tests._netcheck import basis_threaded
    N, I, O, G, k = 65536, 1024, 1024, 10, 3
    g = torch.Generator().manual_seed(0)
    L = KANLinear(I, O, grid_size=G, spline_order=k, backend="cuda")
    with torch.no_grad():
        L.spline_weight.normal_(0.0, 0.1, generator=g)
        L.spline_scaler.uniform_(0.5, 1.5, generator=g)
    E = L.export_inference().cuda()
    x = torch.rand(N, I, generator=g) * 2.2 - 1.1
    with torch.no_grad():
        y = E(x.cuda())
    assert E.last_backend == "cuda"
    grid, bw, sw = np64(E.grid), np64(E.base_weight), np64(E.spline_weight)
    sc = np64(E.spline_scaler) if getattr(E, "spline_scaler", None) is not None else None
    xs = x.double().numpy()
    ref = np.empty((N, O))
    for n0 in range(0, N, 4096):
        xc = xs[n0:n0 + 4096]
        ref[n0:n0 + 4096] = ko.kan_forward(xc, grid, bw, sw, sc, k,
                                           basis=basis_threaded(xc, grid, k))[0]
    worst, block, whole = block_error(np64(y), ref, 256, 256)
    print(f"infer c3 layer: whole {whole:.2e}, worst block {worst:.2e} at {block}", flush=True)
    assert worst < 1e-5


def test_frozen_eval_layer_keeps_packed_weight(C):
    from torchsplinekan_amd import KANLinear
    torch.manual_seed(0)
    L = KANLinear(64, 32, grid_size=6, backend="cuda").cuda()
    with torch.no_grad():
        L.spline_weight.normal_(0, 0.1)
    x = torch.rand(50, 64, device="cuda") * 2 - 1
    y_train = L(x)                                   # autograd path (parameters require grad)
    E = L.export_inference()
    assert not E.training and not any(p.requires_grad for p in E.parameters())
    with torch.no_grad():
        y1 = E(x)
        kept = E._waug_cache[1]
        y2 = E(x)
        assert E._waug_cache[1] is kept              # reused, not rebuilt
    assert normwise(np64(y1), np64(y_train.detach())) < 1e-5
    assert torch.equal(y1, y2)
    # an in-place update (version counter) rebuilds it
    with torch.no_grad():
        E.spline_weight.mul_(2.0)
        y3 = E(x)
    assert E._waug_cache[1] is not kept
    a = lambda t: np64(t.detach())
    ry, _ = ko.kan_forward(a(x), a(E.grid), a(E.base_weight), a(E.spline_weight), None, 3)
    assert normwise(np64(y3), ry) < 1e-5
    E.release_packed_weight()
    assert E._waug_cache is None


def test_training_layer_under_no_grad_keeps_nothing(C):
    from torchsplinekan_amd import KAN
    torch.manual_seed(1)
    net = KAN([16, 12, 4], grid_size=5, backend="cuda").cuda()
    x = torch.rand(33, 16, device="cuda") * 2 - 1
    y_grad = net(x)
    with torch.no_grad():
        y_ng = net(x)
    assert all(getattr(l, "_waug_cache", None) is None for l in net.layers)
    assert normwise(np64(y_ng), np64(y_grad.detach())) < 1e-5
    net.eval()
    with torch.no_grad():
        net(x)
    assert all(getattr(l, "_waug_cache", None) is None for l in net.layers)  # not frozen


def test_infer_rejects_short_workspace(C):
    from torchsplinekan_amd import _lib
    x = torch.zeros(4, 8, device="cuda")
    grid = make_grid(8, 5, 3, "uniform").float().cuda()
    waug = C.pack_weight(torch.zeros(6, 8, device="cuda"), torch.zeros(6, 8, 8, device="cuda"),
                         None, 3, False)
    y = torch.empty(4, 6, device="cuda")
    rc = _lib.LIB.kan_hip_infer(_lib.dtype_code(torch.float32), _lib.ptr(x), _lib.ptr(grid),
                                _lib.ptr(waug), _lib.ptr(y), None, 0, 4, 8, 6, 5, 3, 1, None)
    assert rc != 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("I,O,G,k,base,scaler", [(70, 9, 5, 3, True, True),
                                                 (13, 5, 4, 1, False, True),
                                                 (33, 6, 7, 2, True, False)])
def test_pack_weight_layout_and_unaligned_output(C, dtype, I, O, G, k, base, scaler):
    """The packed weight row [sw * scaler | base_weight | 0-padding] element
    by element (one rounding per product, as the tensor expression), both
    into an aligned buffer (16-byte stores) and one float past an aligned
    address (scalar stores)."""
    from torchsplinekan_amd import _lib
    g = torch.Generator().manual_seed(I + O)
    R = G + k
    sw = torch.randn(O, I, R, generator=g, dtype=torch.float64).to(dtype).cuda()
    bw = torch.randn(O, I, generator=g, dtype=torch.float64).to(dtype).cuda() if base else None
    sc = (torch.rand(O, I, generator=g, dtype=torch.float64) + 0.5).to(dtype).cuda() \
        if scaler else None
    ld = int(_lib.LIB.kan_hip_aug_width(I, G, k, int(base)))
    ref = torch.zeros(O, ld, dtype=dtype, device="cuda")
    ref[:, :I * R] = (sw * sc[..., None] if scaler else sw).reshape(O, I * R)
    if base:
        ref[:, I * R:I * R + I] = bw
    aligned = C.pack_weight(bw, sw, sc, k, scaler)
    assert torch.equal(aligned, ref)
    buf = torch.full((O * ld + 1,), float("nan"), dtype=dtype, device="cuda")
    out = buf[1:]
    assert out.data_ptr() % 16 != 0
    _lib.check(_lib.LIB.kan_hip_pack_weight(
        _lib.KAN_DTYPE_F32 if dtype == torch.float32 else _lib.KAN_DTYPE_F64,
        _lib.ptr(bw), _lib.ptr(sw), _lib.ptr(sc), _lib.ptr(out), I, O, G, k,
        _lib.stream_of(sw.device)))
    torch.cuda.synchronize()
    assert torch.equal(out.view(O, ld), ref)
