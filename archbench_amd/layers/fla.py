"""fla-style mixer construction (archbench/layers/fla.py:11-38) with the gated DeltaNet layer served natively.

``FLAMixer`` wraps a layer and returns ``out[0]`` when the layer returns a tuple (fla.py:11-18);
``build_fla(cls_name, ...)`` passes ``hidden_size``/``layer_idx``/``num_hidden_layers`` only when the layer's
constructor accepts them (fla.py:21-33).  ``"GatedDeltaNet"`` is this package's MI355X layer; any other fla
class needs the flash-linear-attention package, and raises ImportError when it is absent, as the reference does.
"""

from __future__ import annotations

import inspect

import torch.nn as nn

from . import register
from .gdn import GatedDeltaNet

NATIVE_LAYERS = {"GatedDeltaNet": GatedDeltaNet}


class FLAMixer(nn.Module):
    def __init__(self, layer: nn.Module):
        super().__init__()
        self.layer = layer

    def forward(self, x):
        out = self.layer(x)
        return out[0] if isinstance(out, tuple) else out


def build_fla(cls_name: str, d_model: int, layer_idx: int, n_layer: int, **kwargs) -> FLAMixer:
    cls = NATIVE_LAYERS.get(cls_name)
    if cls is None:
        try:
            import fla.layers as L
        except ImportError as e:
            raise ImportError(f"fla:{cls_name} needs flash-linear-attention (pip install flash-linear-attention); "
                              f"natively available: {sorted(NATIVE_LAYERS)}") from e
        cls = getattr(L, cls_name)
    accepted = inspect.signature(cls).parameters
    auto = {"hidden_size": d_model, "layer_idx": layer_idx, "num_hidden_layers": n_layer}
    kwargs = {**{k: v for k, v in auto.items() if k in accepted}, **kwargs}
    return FLAMixer(cls(**kwargs))


@register("gdn")
def build_gdn(d_model, layer_idx, n_layer, **kwargs):
    return build_fla("GatedDeltaNet", d_model, layer_idx, n_layer, **kwargs)
