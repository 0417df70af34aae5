"""Seeded synthetic inputs for the gated DeltaNet op (the benchmark and parity workloads).

Distributions follow the in-model conventions of archbench's GDN-family layer (archbench/layers/nsgdn.py:525-534):
q and k are L2-normalised per head vector (nsgdn.py:527-528), beta = sigmoid(.) (nsgdn.py:534) and the
log-decay g is a log-sigmoid (a negative natural-log retention, nsgdn.py:531 produces the same sign/range).

Draw order is fixed so every consumer sees identical tensors for a seed: a CPU ``torch.Generator`` seeded with
``seed`` draws fp32 q, k, v, b_raw, g_raw, then [h0], then [dO]; transforms are applied; then the cast; then the
move to ``device``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class GDNInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    g: torch.Tensor
    beta: torch.Tensor
    h0: torch.Tensor | None = None
    do: torch.Tensor | None = None

    def to(self, device=None, dtype=None):
        """q, k, v, do move to ``dtype``; g, beta and h0 stay fp32 (they are fp32 at the op boundary)."""
        c = lambda x, dt: None if x is None else x.to(device=device, dtype=dt)
        return GDNInputs(c(self.q, dtype), c(self.k, dtype), c(self.v, dtype), c(self.g, torch.float32),
                         c(self.beta, torch.float32), c(self.h0, torch.float32), c(self.do, dtype))


def make_inputs(B: int, T: int, H: int, K: int, V: int, seed: int = 0, g_shift: float = 4.0,
                h0_std: float | None = None, with_do: bool = False) -> GDNInputs:
    """fp32 CPU tensors: q,k [B,T,H,K] (unit rows), v [B,T,H,V] ~ N(0,1), beta = sigmoid(N(0,1)),
    g = logsigmoid(N(0,1) + g_shift), optional h0 ~ N(0, h0_std^2) [B,H,K,V], optional dO ~ N(0,1) [B,T,H,V]."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen)
    k = torch.randn(B, T, H, K, generator=gen)
    v = torch.randn(B, T, H, V, generator=gen)
    b_raw = torch.randn(B, T, H, generator=gen)
    g_raw = torch.randn(B, T, H, generator=gen)
    h0 = None if h0_std is None else torch.randn(B, H, K, V, generator=gen) * h0_std
    do = torch.randn(B, T, H, V, generator=gen) if with_do else None
    return GDNInputs(F.normalize(q, dim=-1), F.normalize(k, dim=-1), v, F.logsigmoid(g_raw + g_shift),
                     torch.sigmoid(b_raw), h0, do)


def make_step_inputs(B: int, H: int, K: int, V: int, seed: int = 0, g_shift: float = 4.0,
                     state_std: float = 0.1):
    """Decode-step inputs: q,k [B,H,K] (unit rows), v [B,H,V], g,beta [B,H], state [B,H,K,V] ~ N(0, state_std^2)."""
    x = make_inputs(B, 1, H, K, V, seed=seed, g_shift=g_shift, h0_std=state_std)
    return x.q[:, 0], x.k[:, 0], x.v[:, 0], x.g[:, 0], x.beta[:, 0], x.h0
