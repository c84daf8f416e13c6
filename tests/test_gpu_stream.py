"""The streaming probe (kan_hip_stream_probe, measurement support): write
fills the buffer with the (1, 2, 3, 4) float4 pattern, copy reproduces the
source exactly, read leaves its operands untouched; sizes that are not whole
float4 are refused before any launch; the row-segment modes write exactly
the whole rows that fit, and the segment-read mode reads the segments it
names."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_stream_probe_modes():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from torchsplinekan_amd import _C, _lib
    n = (1 << 20) + 4 * 37          # not a whole number of 16 KiB chunks
    a = torch.zeros(n, device="cuda")
    b = torch.zeros(n, device="cuda")
    _C.stream_probe(0, a, b)
    pat = torch.tensor([1.0, 2.0, 3.0, 4.0], device="cuda").repeat(n // 4)
    assert torch.equal(a, pat) and bool((b == 0).all())
    src = torch.randn(n, generator=torch.Generator().manual_seed(1)).cuda()
    _C.stream_probe(2, src, b)
    assert torch.equal(b, src)
    before = src.clone()
    _C.stream_probe(1, src, b)
    torch.cuda.synchronize()
    assert torch.equal(src, before) and torch.equal(b, before)
    assert _lib.LIB.kan_hip_stream_probe(0, a.data_ptr(), b.data_ptr(), 20, None) == \
        _lib.KAN_ERR_INVALID
    assert _lib.LIB.kan_hip_stream_probe(11, a.data_ptr(), b.data_ptr(), 16, None) == \
        _lib.KAN_ERR_INVALID
    # mode 3: every float of the whole rows (13 * 1024 segment values of 4-float
    # pattern, then 1024 values of 5.0) is written, nothing past them
    ld, rows = 14336, 37
    c = torch.zeros(rows * ld + 100, device="cuda")
    _C.stream_probe(3, c, c)
    torch.cuda.synchronize()
    body = c[:rows * ld].view(rows, ld)
    assert torch.equal(body[:, :13312], torch.tensor([1.0, 2.0, 3.0, 4.0], device="cuda")
                       .repeat(rows, 3328))
    assert bool((body[:, 13312:] == 5.0).all()) and bool((c[rows * ld:] == 0).all())
    # mode 6 (one step per workgroup) writes what mode 3 writes; modes 4, 7,
    # 8 and 9 the 4-float pattern everywhere in the rows, nothing past them
    for mode, tail in ((6, 5.0), (4, None), (7, None), (8, None), (9, None)):
        c.zero_()
        _C.stream_probe(mode, c, c)
        torch.cuda.synchronize()
        want = torch.tensor([1.0, 2.0, 3.0, 4.0], device="cuda")
        if tail is None:
            assert torch.equal(body, want.repeat(rows, ld // 4)), mode
        else:
            assert torch.equal(body[:, :13312], want.repeat(rows, 3328)), mode
            assert bool((body[:, 13312:] == tail).all()), mode
        assert bool((c[rows * ld:] == 0).all()), mode
    # mode 5: b[r, 64 fb + t] = the sum of float4 t of row r's segment fb;
    # mode 10: b[r, 128 fb2 + t] = the sum of float4 t of the two segments
    # 2 fb2, 2 fb2 + 1
    src = torch.randn(rows * ld + 100, generator=torch.Generator().manual_seed(2)).cuda()
    for mode, per in ((5, 1), (10, 2)):
        out = torch.full((rows * 1024 + 8,), -7.0, device="cuda")
        _C.stream_probe(mode, src, out)
        torch.cuda.synchronize()
        seg = src[:rows * ld].view(rows, ld)[:, :13312].view(rows, 16 // per, 208 * per, 4)
        seg = seg[:, :, :64 * per, :]
        want = (seg[..., 0] + seg[..., 1]) + (seg[..., 2] + seg[..., 3])
        assert torch.equal(out[:rows * 1024], want.reshape(-1)), mode
        assert bool((out[rows * 1024:] == -7.0).all()), mode
