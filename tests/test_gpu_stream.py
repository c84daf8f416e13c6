"""The streaming probe (kan_hip_stream_probe, measurement support): write
fills the buffer with the (1, 2, 3, 4) float4 pattern, copy reproduces the
source exactly, read leaves its operands untouched; sizes that are not whole
float4 are refused before any launch; the row-segment mode writes exactly
the whole rows that fit."""

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
    assert _lib.LIB.kan_hip_stream_probe(4, a.data_ptr(), b.data_ptr(), 16, None) == \
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
