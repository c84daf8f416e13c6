"""A training step of the native path captured in a HIP graph (torch.cuda.graph)
and replayed: every launch of the step goes to the capturing stream, no
library call synchronises or allocates outside torch's allocator, so a
replay is the eager step.  Each replay is checked against an eager step on
the same inputs (loss and every parameter gradient, bit for bit), with eager
work and synchronisations between the replays (a graph node that only the
first replay gets right would show here).  The loss is F.mse_loss at c2's
size (the step bench.py replays) or the mean squared error formed as
d^T d / numel by the library's split-K product: torch's multi-block mean
over a larger output (16384 x 64) was wrong on every replay after the first
(the gradients were not), so the regularised test uses the native form."""

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _net_and_data(widths, N, seed):
    from torchsplinekan_amd import KAN
    torch.manual_seed(seed)
    net = KAN(widths, grid_size=5, backend="cuda").cuda()
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.rand(N, widths[0], device="cuda", generator=g) * 2.0 - 1.0
    t = torch.randn(N, widths[-1], device="cuda", generator=g)
    return net, x, t


def _mse(y, t):
    from torchsplinekan_amd import _C
    d = (y - t).reshape(1, -1)
    return _C.NativeMatmul.apply(d, d.t()).reshape(()) / d.shape[1]


def _step(net, x, t, loss_fn):
    for p in net.parameters():
        p.grad = None
    loss = loss_fn(net(x), t)
    loss.backward()
    return loss


@pytest.mark.parametrize("loss", ["native", "torch"])
@pytest.mark.parametrize("widths,N", [([784, 256, 10], 4096), ([784, 256, 10], 1024),
                                      ([64, 48, 8], 300)])
def test_captured_step_replays_the_eager_step(widths, N, loss):
    """loss "torch" (F.mse_loss) at c2's own size is what bench.py's c2 line
    replays."""
    loss_fn = _mse if loss == "native" else F.mse_loss
    net, x, t = _net_and_data(widths, N, seed=len(widths) + N)
    params = list(net.parameters())
    # eager reference
    loss_ref = _step(net, x, t, loss_fn).detach().clone()
    grads_ref = [p.grad.clone() for p in params]
    assert all(l.last_backend == "cuda" for l in net.layers)
    # warm up on a side stream (default priority), then capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(net, x, t, loss_fn)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss_g = _step(net, x, t, loss_fn)
    grads_g = [p.grad for p in params]
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(loss_g, loss_ref), rep
        for i, (g, r) in enumerate(zip(grads_g, grads_ref)):
            assert torch.equal(g, r), (rep, i)
        # eager work between replays: the same step on other inputs
        y = net(torch.rand_like(x))
        y.sum().item()
        torch.cuda.synchronize()
    # the replay follows changed inputs written in place
    x.mul_(0.5)
    t.add_(0.25)
    graph.replay()
    torch.cuda.synchronize()
    saved = [g.clone() for g in grads_g]
    loss_new = loss_g.clone()
    eager_loss = _step(net, x, t, loss_fn)
    assert torch.equal(loss_new, eager_loss.detach())
    for i, (g, p) in enumerate(zip(saved, params)):
        assert torch.equal(g, p.grad), i


def test_captured_regularised_step_replays_the_eager_step():
    """forward_with_regularization + MSE + backward (the fused edge kernels,
    the regulariser scalar's launches, the loss over 16384 x 64 outputs)
    captured and replayed: loss, regulariser and every gradient equal to the
    eager step's on each replay."""
    from torchsplinekan_amd import KAN
    torch.manual_seed(7)
    net = KAN([64, 128, 64], grid_size=8, backend="cuda").cuda()
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.rand(16384, 64, device="cuda", generator=g) * 2.0 - 1.0
    t = torch.randn(16384, 64, device="cuda", generator=g)
    params = list(net.parameters())

    def step():
        for p in params:
            p.grad = None
        y, reg = net.forward_with_regularization(x, 1e-2, 1e-2, reg_impl="auto")
        loss = _mse(y, t) + reg
        loss.backward()
        return loss, reg

    loss_ref, reg_ref = [v.detach().clone() for v in step()]
    grads_ref = [p.grad.clone() for p in params]
    assert all(l.last_backend == "cuda" for l in net.layers)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss_g, reg_g = step()
    grads_g = [p.grad for p in params]
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(loss_g, loss_ref) and torch.equal(reg_g, reg_ref), rep
        for i, (a, b) in enumerate(zip(grads_g, grads_ref)):
            assert torch.equal(a, b), (rep, i)
        net(torch.rand_like(x)).sum().item()
        torch.cuda.synchronize()

