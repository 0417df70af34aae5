"""The n-step gated DeltaNet mixer (archbench's ``nsgdn`` arch) on the MI355X kernels.

Constructor and parameter names follow ``NStepGDN`` (archbench/layers/nsgdn.py:473-516): ``in_proj`` (q, k, v,
gate, and the a / b gate inputs in one projection), ``conv.weight`` [2*H*DK + H*DV, 1, conv_size], ``A_log``,
``dt_bias``, ``b_bias``, ``lam``, ``norm`` (RMSNorm over DV) and ``o_proj``, so the reference's checkpoints and
zero-init rule for ``o_proj`` (archbench/model.py:14, :80-82) apply.  The forward computes what
``NStepGDN.forward`` does (nsgdn.py:518-542):

    qkv = conv(in_proj(x)) with SiLU           -> ops.mixer_input_stage, three conv launches on the weight's rows, q and k
                                                  L2-normalised per head inside the conv (nsgdn.py:527-528)
    la, beta from ab                           -> ops.gdn_gates (nsgdn.py:531-534, optional la_min clamp)
    u = write_direction(k, p, beta, lam, n)    -> ops.write_direction, one HIP pass each way with p = the previous
                                                  token's k (nsgdn.py:61-75, :535-536)
    y = scan(q, k, u, v, la)                   -> ops.nsgdn_scan_chunk, the chunk kernels with write keys u; the
                                                  q scale DK^-1/2 is the op's scale instead of a separate pass
    y = norm(y) * silu(g); o_proj              -> ops.gated_rmsnorm

``scan_impl``: "chunk" and "dplr" run the HIP chunk kernels in bf16 with fp32 state and accumulation, which is
what the reference's "chunk" (its default) and "dplr" run (``nsgdn.py:404-405``).  "triton" and "ref" are the
reference's exact fp32 token scan (``nsgdn.py:52-58``, ``:80-216``, ``:408-417``), here ``ops.nsgdn_scan`` (the HIP
token scan with its checkpointed reverse-time backward): fp32 q, k, u, v, the write direction computed in fp32, and
y kept in fp32 through the output norm, as the reference's module keeps them.  That scan is compiled for head_dim
64 and 128; other head sizes fall back to the chunk kernels with a warning.
"""

from __future__ import annotations

import math
import warnings

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops
from . import register
from .gdn import _grouped_linear, _linear


class NStepGDN(nn.Module):
    def __init__(self, d_model: int, num_heads: int = 8, head_dim: int = 128, expand_v: float = 2.0,
                 n_steps: int = 2, lam: float = 1.0, use_gate: bool = True, use_short_conv: bool = True,
                 conv_size: int = 4, norm_eps: float = 1e-5, scan_impl: str = "chunk", la_min: float | None = None,
                 layer_idx: int | None = None):
        super().__init__()
        DK, DV = head_dim, int(head_dim * expand_v)
        if DK & (DK - 1) or DV & (DV - 1):
            raise ValueError("head_dim and head_dim * expand_v must be powers of 2")
        if n_steps < 1:
            raise ValueError("n_steps must be >= 1")
        if lam <= 0:
            raise ValueError("lam must be > 0")
        if scan_impl not in ("chunk", "dplr", "triton", "ref"):
            raise ValueError(f"unknown scan_impl {scan_impl!r}")
        if scan_impl in ("triton", "ref") and DK not in (64, 128):
            warnings.warn(f"NStepGDN(scan_impl={scan_impl!r}): the exact fp32 token scan is compiled for head_dim 64 "
                          f"and 128; head_dim {DK} runs the bf16 chunk kernels (fp32 state and accumulation, relative "
                          "L2 within 1e-2 of the fp32 recurrence)", UserWarning, stacklevel=2)
        self.H, self.DK, self.DV, self.n_steps = num_heads, DK, DV, n_steps
        self.qk_dim, self.v_dim = num_heads * DK, num_heads * DV
        self.use_gate = use_gate
        self.n_gate = self.v_dim if use_gate else 0
        width = 2 * self.qk_dim + self.v_dim + self.n_gate + 2 * num_heads
        self.in_proj = nn.Linear(d_model, (width + 7) // 8 * 8, bias=False)
        self.conv = _ConvWeight(2 * self.qk_dim + self.v_dim, conv_size) if use_short_conv else None
        self.A_log = nn.Parameter(torch.empty(num_heads).uniform_(1, 16).log())
        dt = torch.exp(torch.rand(num_heads) * (math.log(0.1) - math.log(0.001)) + math.log(0.001))
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.b_bias = nn.Parameter(torch.zeros(num_heads))
        self.lam = nn.Parameter(torch.full((num_heads,), math.log(math.expm1(lam))))
        self.norm = nn.RMSNorm(DV, eps=norm_eps)
        self.scan_impl, self.la_min, self.layer_idx = scan_impl, la_min, layer_idx
        self.o_proj = nn.Linear(self.v_dim, d_model, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, _ = x.shape
        H, DK, DV = self.H, self.DK, self.DV
        n_qkv = 2 * self.qk_dim + self.v_dim
        n_main = n_qkv + self.n_gate
        dev_type = x.device.type
        xp = x
        if torch.is_autocast_enabled(dev_type) and x.dtype == torch.float32:
            xp = x.to(torch.get_autocast_dtype(dev_type))  # autocast's cast, made once for both GEMMs below
        # in_proj's rows [q k v], [gate] and [a b] as one GEMM each (the first a multiple of 256 wide at the
        # reference shapes); the rows past them pad the projection and are not computed (their gradient is zero)
        bounds = [0, n_qkv] + ([n_main] if self.n_gate else []) + [n_main + 2 * H]
        y, *g, ab = _grouped_linear(xp, self.in_proj.weight, bounds)
        g = g[0] if g else None
        # the exact token scan takes fp32 q and k normalised after the conv, as the reference normalises the fp32
        # copies of the conv output (nsgdn.py:525-528); the chunk path gets them normalised inside the conv
        exact = self.scan_impl in ("triton", "ref") and DK in (64, 128)
        if self.conv is not None:
            # q, k, v convolved straight out of y (ops.mixer_input_stage; the taps used rounded to y's dtype, as
            # the reference's conv runs them)
            q, k, v = ops.mixer_input_stage(y, self.conv.weight.squeeze(1), self.qk_dim, self.v_dim,
                                            0 if exact else DK)
        else:
            q, k, v = torch.split(y, [self.qk_dim, self.qk_dim, self.v_dim], dim=-1)
        q, k, v = q.reshape(B, T, H, DK), k.reshape(B, T, H, DK), v.reshape(B, T, H, DV)
        if not exact and self.conv is None:
            q, k = ops.l2norm(q, 1e-12, 1.0), ops.l2norm(k, 1e-12, 1.0)
        la, beta = ops.gdn_gates_ab(ab, self.A_log, self.dt_bias, self.b_bias, 1.0,
                                 float("-inf") if self.la_min is None else float(self.la_min))
        gate = g.reshape(B, T, H, DV) if self.use_gate else None
        lam = F.softplus(self.lam.float())
        eps = self.norm.eps or 1e-5
        if exact:
            # the reference's exact fp32 token scan (nsgdn.py:525-536 with its "triton" / "ref" scan): q and k
            # normalised in fp32 (q with the DK^-1/2 scale), u from fp32 k, y fp32 through the norm, cast for
            # o_proj as autocast casts the projection's input
            qf = ops.l2norm(q.float(), 1e-12, DK ** -0.5)
            kf = ops.l2norm(k.float(), 1e-12, 1.0)
            u = ops.write_direction(kf, beta, lam, self.n_steps)
            y = ops.nsgdn_scan(qf, kf, u, v.float(), la)
            y = ops.gated_rmsnorm(y, None if gate is None else gate.float(), self.norm.weight, eps)
            return _linear(y.reshape(B, T, -1).to(xp.dtype), self.o_proj.weight)
        # u from k, the previous token's k and beta in one HIP pass (fp32 arithmetic, written in k's dtype, which
        # the scan takes u in)
        u = ops.write_direction(k, beta, lam, self.n_steps)
        y = ops.nsgdn_scan_chunk(q, k, u, v, la, scale=DK ** -0.5)
        y = ops.gated_rmsnorm(y.to(xp.dtype), gate, self.norm.weight, eps)
        return _linear(y.reshape(B, T, -1), self.o_proj.weight)


class _ConvWeight(nn.Module):
    """Holds the depthwise conv weight [D, 1, size] under the reference's name (ShortConv.weight, nsgdn.py:457-462)."""

    def __init__(self, dim: int, size: int):
        super().__init__()
        self.size = size
        self.weight = nn.Parameter(torch.empty(dim, 1, size).uniform_(-1 / math.sqrt(size), 1 / math.sqrt(size)))


@register("nsgdn")
def build_nsgdn(d_model: int, layer_idx: int, n_layer: int, **kwargs):
    return NStepGDN(d_model, layer_idx=layer_idx, **kwargs)
