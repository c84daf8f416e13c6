"""Physical node pruning of a KAN from per-edge L1 scores (the paper's
Appendix M.1, eq. 23), as spline_kan/pruning.py:1-160 defines it.

Hidden node i sits between layer l-1 (as its output i) and layer l (as its
input i).  Its scores are the largest mean |phi| over the edges that enter
and that leave it:

    incoming  I_i = max_o' a_{l-1}[i, o']   (row i of layer l-1's [O, I] means)
    outgoing  O_i = max_o  a_l[o, i]        (column i of layer l's means)

where a = mean_n |phi(x_n)| is taken on the inputs each layer actually sees
(base branch included).  On a device tensor of a supported shape,
KANLinear.edge_l1 evaluates a with the fused native edge kernel
(kan_hip_edge_abs_mean), so the [N, O, I] edge tensor is never formed.  A node
survives iff both scores exceed the threshold; removed nodes are sliced out of
layer l-1's rows and layer l's columns (weights, scaler and grid row), and a
smaller KAN is assembled.  Input and output widths never change.
"""

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import torch

from .kan import KAN
from .kan_linear import KANLinear


@dataclass
class PruneResult:
    """Outcome of prune_nodes (spline_kan/pruning.py:30-52)."""
    model: KAN
    kept: List[List[int]]                 # per hidden layer: surviving original indices
    old_to_new: List[Dict[int, int]]      # per hidden layer: original index -> new index
    widths_before: List[int]
    widths_after: List[int]
    params_before: int
    params_after: int
    scores_in: List[torch.Tensor] = field(repr=False, default_factory=list)
    scores_out: List[torch.Tensor] = field(repr=False, default_factory=list)
    threshold: float = 1e-2

    def summary(self) -> dict:
        return {"widths_before": self.widths_before, "widths_after": self.widths_after,
                "params_before": self.params_before, "params_after": self.params_after,
                "kept": self.kept, "threshold": self.threshold}


@torch.no_grad()
def node_scores(model: KAN, x: torch.Tensor):
    """Incoming and outgoing scores, one [width] tensor per hidden layer
    (spline_kan/pruning.py:55-68)."""
    means = []
    h = x
    for layer in model.layers:
        means.append(layer.edge_l1(h))      # [O, I] on this layer's own inputs
        h = layer(h)
    incoming = [means[l - 1].amax(dim=1) for l in range(1, len(model.layers))]
    outgoing = [means[l].amax(dim=0) for l in range(1, len(model.layers))]
    return incoming, outgoing


def _sliced(layer: KANLinear, rows: torch.Tensor, cols: torch.Tensor) -> KANLinear:
    """Layer restricted to output rows `rows` and input columns `cols`
    (spline_kan/pruning.py:71-81)."""
    new = layer.make_like(in_features=len(cols), out_features=len(rows))
    with torch.no_grad():
        new.base_weight.copy_(layer.base_weight[rows][:, cols])
        new.spline_weight.copy_(layer.spline_weight[rows][:, cols])
        if layer.enable_standalone_scale_spline:
            new.spline_scaler.copy_(layer.spline_scaler[rows][:, cols])
        new._copy_grid_(layer.grid[cols])
    new.requires_grad_(any(p.requires_grad for p in layer.parameters()))
    return new.train(layer.training)


def prune_nodes(model: KAN, x_calib: Optional[torch.Tensor] = None, threshold: float = 1e-2, *,
                keep: Optional[Sequence[Sequence[int]]] = None,
                min_keep: int = 1) -> PruneResult:
    """Smaller KAN without the hidden nodes whose incoming or outgoing score
    is at most `threshold` (spline_kan/pruning.py:84-160).

    `keep` (one index list per hidden layer) overrides the scores.  With
    scores, at least `min_keep` nodes per hidden layer survive (those with the
    largest min(incoming, outgoing)).  `model` is left unchanged; the result's
    parameters are independent copies, so an optimiser must be rebuilt."""
    n_hidden = len(model.layers) - 1
    s_in: List[torch.Tensor] = []
    s_out: List[torch.Tensor] = []
    if keep is None:
        if x_calib is None:
            raise ValueError("prune_nodes needs x_calib (or explicit keep indices)")
        s_in, s_out = node_scores(model, x_calib)
        keep = []
        for si, so in zip(s_in, s_out):
            idx = ((si > threshold) & (so > threshold)).nonzero().flatten()
            if len(idx) < min_keep:
                best = torch.minimum(si, so).topk(min(min_keep, len(si))).indices
                idx = best.sort().values
            keep.append(idx.tolist())
    if len(keep) != n_hidden:
        raise ValueError(f"keep must list {n_hidden} hidden layers, got {len(keep)}")

    dev = model.layers[0].grid.device
    widths = model.widths
    index = [torch.arange(widths[0], device=dev)]
    for l, k in enumerate(keep):
        k = sorted(set(int(i) for i in k))
        if not k:
            raise ValueError(f"hidden layer {l + 1} would have no nodes")
        if k[0] < 0 or k[-1] >= widths[l + 1]:
            raise ValueError(f"keep indices out of range for hidden layer {l + 1}")
        index.append(torch.tensor(k, device=dev))
    index.append(torch.arange(widths[-1], device=dev))

    layers = [_sliced(layer, index[l + 1], index[l]) for l, layer in enumerate(model.layers)]
    new = KAN.from_layers(layers).train(model.training)
    kept = [t.tolist() for t in index[1:-1]]
    return PruneResult(
        model=new, kept=kept, old_to_new=[{o: n for n, o in enumerate(k)} for k in kept],
        widths_before=widths, widths_after=new.widths,
        params_before=sum(p.numel() for p in model.parameters()),
        params_after=sum(p.numel() for p in new.parameters()),
        scores_in=s_in, scores_out=s_out, threshold=threshold)
