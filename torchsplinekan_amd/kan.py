"""KAN: stacked KANLinear layers (mirrors spline_kan/kan.py)."""

from typing import List, Tuple

import torch
import torch.nn as nn

from .kan_linear import KANLinear


class KAN(nn.Module):
    """Kolmogorov-Arnold Network: layers_hidden=[16, 32, 8] builds the layers
    16->32 and 32->8; every other argument is forwarded to each KANLinear."""

    def __init__(self, layers_hidden: List[int], grid_size: int = 5, spline_order: int = 3,
                 scale_noise: float = 0.1, scale_base: float = 1.0, scale_spline: float = 1.0,
                 enable_standalone_scale_spline: bool = True, base_activation=nn.SiLU,
                 grid_eps: float = 0.02, grid_range: tuple = (-1.0, 1.0),
                 backend: str = "auto") -> None:
        super().__init__()
        if len(layers_hidden) < 2:
            raise ValueError(
                "layers_hidden must have at least two entries (in_features and out_features of "
                f"the first layer), got {layers_hidden}")
        self.layers = nn.ModuleList([
            KANLinear(layers_hidden[i], layers_hidden[i + 1], grid_size=grid_size,
                      spline_order=spline_order, scale_noise=scale_noise, scale_base=scale_base,
                      scale_spline=scale_spline,
                      enable_standalone_scale_spline=enable_standalone_scale_spline,
                      base_activation=base_activation, grid_eps=grid_eps, grid_range=grid_range,
                      backend=backend)
            for i in range(len(layers_hidden) - 1)])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for layer in self.layers:
            x = layer(x)
        return x

    def update_grid(self, x: torch.Tensor, margin: float = 0.01) -> None:
        """Updates each layer's knots on the input that layer actually sees."""
        with torch.no_grad():
            for layer in self.layers:
                layer.update_grid(x, margin=margin)
                x = layer(x)

    def regularization_loss(self, reg_act: float = 1.0, reg_entropy: float = 1.0, *,
                            x: torch.Tensor, mode: str = "activation", reg_impl: str = "auto",
                            chunk_size: int = 1024) -> torch.Tensor:
        """Sum of the layers' penalties on their actual inputs (paper eq. 22);
        hidden activations stay in the graph."""
        if mode == "coefficient":
            total = x.new_zeros(())
            for layer in self.layers:
                total = total + layer.regularization_loss(reg_act, reg_entropy, mode="coefficient")
            return total
        _, reg = self.forward_with_regularization(x, reg_act, reg_entropy, mode=mode,
                                                  reg_impl=reg_impl, chunk_size=chunk_size)
        return reg

    def forward_with_regularization(self, x: torch.Tensor, reg_act: float = 1.0,
                                    reg_entropy: float = 1.0, *, mode: str = "activation",
                                    reg_impl: str = "auto", chunk_size: int = 1024
                                    ) -> Tuple[torch.Tensor, torch.Tensor]:
        """(self(x), regularization_loss) from a single pass over the layers."""
        if mode == "coefficient":
            return self(x), self.regularization_loss(reg_act, reg_entropy, x=x, mode="coefficient")
        total = x.new_zeros(())
        h = x
        for layer in self.layers:
            h, r = layer.forward_with_regularization(h, reg_act, reg_entropy, mode=mode,
                                                     reg_impl=reg_impl, chunk_size=chunk_size)
            total = total + r
        return h, total

    def export_inference(self, requires_grad: bool = False) -> "KAN":
        """Independent KAN whose layers fold spline_scaler into spline_weight."""
        new = KAN.from_layers([l.export_inference(requires_grad) for l in self.layers])
        return new.train(self.training and requires_grad)

    @torch.no_grad()
    def extend_grid(self, new_grid_size: int, x: torch.Tensor, **kw) -> "KAN":
        """New KAN with every layer refined to new_grid_size
        (KANLinear.extend_grid), each fitted on the input that layer sees in
        this network (spline_kan/kan.py:209-222)."""
        layers, h = [], x
        for layer in self.layers:
            layers.append(layer.extend_grid(new_grid_size, h, **kw))
            h = layer(h)
        return KAN.from_layers(layers).train(self.training)

    def prune(self, x_calib: torch.Tensor, threshold: float = 1e-2, **kw):
        """Physical node pruning (paper eq. 23); see pruning.prune_nodes
        (spline_kan/kan.py:204-207)."""
        from .pruning import prune_nodes
        return prune_nodes(self, x_calib, threshold, **kw)

    @classmethod
    def from_layers(cls, layers: List[KANLinear]) -> "KAN":
        """KAN around existing KANLinear layers (widths must chain)."""
        for a, b in zip(layers[:-1], layers[1:]):
            if a.out_features != b.in_features:
                raise ValueError(f"layer widths do not chain: {a.out_features} -> {b.in_features}")
        net = cls.__new__(cls)
        nn.Module.__init__(net)
        net.layers = nn.ModuleList(layers)
        return net

    @property
    def widths(self) -> List[int]:
        return [self.layers[0].in_features] + [l.out_features for l in self.layers]
