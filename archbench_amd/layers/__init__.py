"""Mixer registry with the reference's plugin surface (archbench/layers/__init__.py:1-26).

``register(name)`` decorates a builder, ``available()`` lists names, ``build_mixer(name, d_model, layer_idx,
n_layer, **kwargs)`` builds one; an unknown name raises KeyError and ``"fla:<Class>"`` routes to
``build_fla`` exactly as in the reference.  The gated DeltaNet mixers are provided here, on the MI355X kernels:
``"gdn"`` (fla's GatedDeltaNet, archbench/layers/fla.py:36-38) and ``"nsgdn"`` (the n-step family,
archbench/layers/nsgdn.py:545-547); the reference's other mixers are outside this package.
"""

from __future__ import annotations

_REGISTRY: dict[str, callable] = {}


def register(name: str):
    def deco(fn):
        _REGISTRY[name] = fn
        return fn

    return deco


def available() -> list[str]:
    return sorted(_REGISTRY)


def build_mixer(name: str, d_model: int, layer_idx: int, n_layer: int, **kwargs):
    if name.startswith("fla:"):
        from .fla import build_fla

        return build_fla(name[4:], d_model, layer_idx, n_layer, **kwargs)
    if name not in _REGISTRY:
        raise KeyError(f"unknown arch {name!r}; available: {available()} or 'fla:<ClassName>'")
    return _REGISTRY[name](d_model=d_model, layer_idx=layer_idx, n_layer=n_layer, **kwargs)


from . import fla  # noqa: E402,F401  (registers "gdn")
from . import nsgdn  # noqa: E402,F401  (registers "nsgdn")
