"""Mixer registry with the reference's plugin surface (archbench/layers/__init__.py:1-26).

``register(name)`` decorates a builder, ``available()`` lists names, ``build_mixer(name, d_model, layer_idx,
n_layer, **kwargs)`` builds one; an unknown name raises KeyError and ``"fla:<Class>"`` routes to
``build_fla`` exactly as in the reference.  Only the gated DeltaNet mixer (``"gdn"``) is provided here, on the
MI355X kernels; the reference's other mixers are outside this package.
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
