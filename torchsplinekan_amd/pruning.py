"""Physical node pruning of a KAN (the KAN paper's Appendix M.1, eq. 23);
the API of spline_kan/pruning.py (PruneResult, node_scores, prune_nodes).

A hidden node j sits between two layers: it is output j of the layer before
and input j of the layer after.  With a_l = mean_n |phi_l(x_n)| [O, I] the
per-edge L1 norms of layer l on the inputs it actually sees (base branch
included), its importance is read off two edges:

    incoming  = max over the row j of a_{l-1}     (edges entering j)
    outgoing  = max over the column j of a_l      (edges leaving j)

and the node stays iff min(incoming, outgoing) exceeds the threshold.  The
norms come from KANLinear.edge_l1, which on a device tensor runs the fused
native statistic (one launch per layer, no [N, O, I] tensor).  The decision
is a boolean mask per hidden layer; a mask becomes the index tensors that
KANLinear.select uses to cut the layers on either side of the boundary.
"""

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .kan import KAN


@dataclass
class PruneResult:
    """Pruned model plus the bookkeeping a caller needs to map old node ids
    to new ones (per hidden layer), the widths and parameter counts before
    and after, and the scores the decision was taken on."""
    model: KAN
    kept: List[List[int]]
    old_to_new: List[Dict[int, int]]
    widths_before: List[int]
    widths_after: List[int]
    params_before: int
    params_after: int
    scores_in: List[torch.Tensor] = field(repr=False, default_factory=list)
    scores_out: List[torch.Tensor] = field(repr=False, default_factory=list)
    threshold: float = 1e-2

    def summary(self) -> dict:
        keys = ("widths_before", "widths_after", "params_before", "params_after", "kept",
                "threshold")
        return {k: getattr(self, k) for k in keys}


@torch.no_grad()
def _edge_norms(model: KAN, x: torch.Tensor) -> List[torch.Tensor]:
    """a_l [O_l, I_l] for every layer, each on the activations it receives."""
    norms, h = [], x
    for layer in model.layers:
        norms.append(layer.edge_l1(h))
        h = layer(h)
    return norms


@torch.no_grad()
def node_scores(model: KAN, x: torch.Tensor) -> Tuple[List[torch.Tensor], List[torch.Tensor]]:
    """(incoming, outgoing): one [width] tensor per hidden boundary."""
    a = _edge_norms(model, x)
    incoming = [a_before.amax(dim=1) for a_before in a[:-1]]
    outgoing = [a_after.amax(dim=0) for a_after in a[1:]]
    return incoming, outgoing


def _score_masks(incoming, outgoing, threshold: float, min_keep: int) -> List[torch.Tensor]:
    """Keep masks from eq. 23; a boundary left with fewer than min_keep nodes
    keeps the min_keep nodes of largest min(incoming, outgoing)."""
    masks = []
    for s_in, s_out in zip(incoming, outgoing):
        score = torch.minimum(s_in, s_out)
        mask = score > threshold
        short = min(min_keep, score.numel())
        if int(mask.sum()) < short:
            mask = torch.zeros_like(mask)
            mask[score.topk(short).indices] = True
        masks.append(mask)
    return masks


def _explicit_masks(keep: Sequence[Sequence[int]], widths: List[int],
                    device: torch.device) -> List[torch.Tensor]:
    masks = []
    for b, ids in enumerate(keep, start=1):
        ids = [int(i) for i in ids]
        if not ids:
            raise ValueError(f"hidden layer {b} would have no nodes")
        if min(ids) < 0 or max(ids) >= widths[b]:
            raise ValueError(f"keep indices out of range for hidden layer {b}")
        mask = torch.zeros(widths[b], dtype=torch.bool, device=device)
        mask[torch.tensor(ids, device=device)] = True
        masks.append(mask)
    return masks


def prune_nodes(model: KAN, x_calib: Optional[torch.Tensor] = None, threshold: float = 1e-2, *,
                keep: Optional[Sequence[Sequence[int]]] = None,
                min_keep: int = 1) -> PruneResult:
    """Smaller KAN without the hidden nodes eq. 23 finds unimportant on
    x_calib (or with exactly the nodes listed in `keep`, one index list per
    hidden layer).  `model` is not modified; the new model has its own
    parameters (an optimiser of the old one does not fit it)."""
    widths = model.widths
    n_hidden = len(model.layers) - 1
    dev = model.layers[0].grid.device
    incoming: List[torch.Tensor] = []
    outgoing: List[torch.Tensor] = []
    if keep is None:
        if x_calib is None:
            raise ValueError("prune_nodes needs x_calib (or explicit keep indices)")
        incoming, outgoing = node_scores(model, x_calib)
        masks = _score_masks(incoming, outgoing, threshold, min_keep)
    else:
        if len(keep) != n_hidden:
            raise ValueError(f"keep must list {n_hidden} hidden layers, got {len(keep)}")
        masks = _explicit_masks(keep, widths, dev)
    # node indices kept at every boundary (network input and output: all)
    index = ([None] + [m.nonzero().flatten() for m in masks] + [None])
    layers = [layer.select(out_index=index[l + 1], in_index=index[l])
              for l, layer in enumerate(model.layers)]
    pruned = KAN.from_layers(layers).train(model.training)
    kept = [ix.tolist() for ix in index[1:-1]]
    count = lambda m: sum(p.numel() for p in m.parameters())
    return PruneResult(model=pruned, kept=kept,
                       old_to_new=[dict(zip(k, range(len(k)))) for k in kept],
                       widths_before=widths, widths_after=pruned.widths,
                       params_before=count(model), params_after=count(pruned),
                       scores_in=incoming, scores_out=outgoing, threshold=threshold)
