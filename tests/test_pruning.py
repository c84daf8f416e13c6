"""Node pruning (paper eq. 23; spline_kan/pruning.py) on the CPU and, for the
scores, on the GPU through the native edge kernel.  Cases follow the
reference's own tests (tests/test_pruning.py:24-106): nodes whose incoming or
outgoing edges are all zero are removed, removing nodes without outgoing
edges leaves the function unchanged, scores are the row/column maxima of the
per-edge mean |phi| (checked against the fp64 oracle), and min_keep /
explicit keep lists behave as documented."""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import kan_oracle as ko
from torchsplinekan_amd import KAN, prune_nodes
from tests._util import np64


def _zero_edges(model, hidden, nodes, side):
    """Zero every edge entering (side="in") or leaving (side="out") the given
    nodes of hidden layer `hidden` (1-based)."""
    with torch.no_grad():
        if side == "in":
            layer = model.layers[hidden - 1]
            layer.base_weight[nodes] = 0
            layer.spline_weight[nodes] = 0
        else:
            layer = model.layers[hidden]
            layer.base_weight[:, nodes] = 0
            layer.spline_weight[:, nodes] = 0


def _oracle_edge_means(layer, h):
    """mean_n |phi| [O, I] of one layer on inputs h, by the fp64 oracle."""
    a = lambda t: np64(t)
    x = a(h)
    H = ko.basis_dense(x, a(layer.grid), layer.spline_order)
    W = a(layer.spline_weight) * a(layer.spline_scaler)[..., None]
    s = a(F.silu(h.double()))
    return ko.edge_abs_mean(s, H, a(layer.base_weight), W)


def test_nodes_without_edges_are_removed():
    torch.manual_seed(0)
    m = KAN([3, 6, 5, 2], grid_size=4, backend="reference").double()
    with torch.no_grad():
        for layer in m.layers:
            layer.base_weight.mul_(10)
    _zero_edges(m, 1, [1, 4], "out")
    _zero_edges(m, 2, [0], "in")
    _zero_edges(m, 2, [3], "out")
    x = torch.rand(300, 3, dtype=torch.float64) * 2 - 1
    res = prune_nodes(m, x, threshold=1e-2)
    assert res.kept == [[0, 2, 3, 5], [1, 2, 4]]
    assert res.widths_before == [3, 6, 5, 2] and res.widths_after == [3, 4, 3, 2]
    p = res.model
    assert p.layers[0].base_weight.shape == (4, 3)
    assert p.layers[1].spline_weight.shape == (3, 4, 7)
    assert torch.equal(p.layers[1].grid, m.layers[1].grid[[0, 2, 3, 5]])
    assert torch.equal(p.layers[2].spline_weight, m.layers[2].spline_weight[:, [1, 2, 4]])
    assert res.old_to_new == [{0: 0, 2: 1, 3: 2, 5: 3}, {1: 0, 2: 1, 4: 2}]
    assert res.params_after < res.params_before
    # hidden-2 node 0 has no incoming edges: its value is the constant 0 and
    # removing it shifts the output by its outgoing edges' phi(0)
    l2 = m.layers[2]
    only0 = l2.make_like()
    only0.load_state_dict(l2.state_dict())
    with torch.no_grad():
        only0.base_weight[:, 1:] = 0
        only0.spline_weight[:, 1:] = 0
        shift = only0(torch.zeros(1, 5, dtype=torch.float64))
    xt = torch.rand(50, 3, dtype=torch.float64) * 2 - 1
    assert torch.allclose(p(xt) + shift, m(xt), atol=1e-10)


def test_removing_dead_outgoing_nodes_is_exact():
    torch.manual_seed(1)
    m = KAN([4, 7, 3], grid_size=5, base_activation=nn.Tanh, backend="reference").double()
    _zero_edges(m, 1, [0, 3, 6], "out")
    x = torch.rand(200, 4, dtype=torch.float64) * 2 - 1
    res = m.prune(x)
    assert res.kept == [[1, 2, 4, 5]]
    assert torch.allclose(res.model(x), m(x), atol=1e-12)
    removed = 3 * (4 * (1 + 8 + 1) + 3 * (1 + 8 + 1))   # per node: bw, coef row, scaler
    assert res.params_after == sum(p.numel() for p in m.parameters()) - removed


def test_scores_are_row_and_column_maxima_of_edge_means():
    torch.manual_seed(2)
    m = KAN([2, 3, 2], grid_size=3, backend="reference").double()
    x = torch.rand(64, 2, dtype=torch.float64) * 2 - 1
    res = prune_nodes(m, x, threshold=0.0)
    a0 = _oracle_edge_means(m.layers[0], x)
    a1 = _oracle_edge_means(m.layers[1], m.layers[0](x).detach())
    assert np.allclose(np64(res.scores_in[0]), a0.max(axis=1), rtol=1e-12, atol=0)
    assert np.allclose(np64(res.scores_out[0]), a1.max(axis=0), rtol=1e-12, atol=0)


def test_min_keep_and_explicit_keep():
    m = KAN([2, 4, 1], grid_size=3, backend="reference")
    with torch.no_grad():
        for p in m.parameters():
            p.zero_()
    x = torch.rand(20, 2)
    assert prune_nodes(m, x, min_keep=1).widths_after == [2, 1, 1]
    res = prune_nodes(m, keep=[[0, 3]])
    assert res.widths_after == [2, 2, 1] and res.old_to_new == [{0: 0, 3: 1}]
    with pytest.raises(ValueError):
        prune_nodes(m, keep=[[]])
    with pytest.raises(ValueError):
        prune_nodes(m, keep=[[0, 9]])
    with pytest.raises(ValueError):
        prune_nodes(m)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_gpu_scores_use_native_edge_kernel(dtype):
    """On a device tensor edge_l1 runs the fused native statistic; the node
    scores then match the oracle (fp64 1e-12, fp32 1e-5 relative)."""
    assert torch.cuda.is_available()
    torch.manual_seed(4)
    m = KAN([8, 16, 12, 3], grid_size=5, backend="cuda").to(dtype)
    _zero_edges(m, 1, [2, 9], "out")
    from torchsplinekan_amd import _lib
    md = m.cuda()
    x = (torch.rand(500, 8, dtype=dtype) * 2 - 1).cuda()
    _lib.timing_enable(True)
    res = prune_nodes(md, x, threshold=1e-3)
    torch.cuda.synchronize()
    _, edge_launches, _ = _lib.timing_read("edge")
    _lib.timing_enable(False)
    assert edge_launches == len(md.layers), edge_launches   # one fused statistic per layer
    assert 2 not in res.kept[0] and 9 not in res.kept[0]
    h = x
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    for l in range(1, len(md.layers)):
        a_in = _oracle_edge_means(md.layers[l - 1], h)
        h = md.layers[l - 1](h).detach()
        a_out = _oracle_edge_means(md.layers[l], h)
        for got, ref in ((res.scores_in[l - 1], a_in.max(axis=1)),
                         (res.scores_out[l - 1], a_out.max(axis=0))):
            err = np.abs(np64(got) - ref).max() / np.abs(ref).max()
            assert err < tol, err
    xt = (torch.rand(64, 8, dtype=dtype) * 2 - 1).cuda()
    assert torch.allclose(res.model(xt), md(xt), atol=1e-4 if dtype == torch.float32 else 1e-12)
