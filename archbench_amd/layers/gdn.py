"""Gated DeltaNet mixer layer on the MI355X kernels, with the constructor and forward of the fla layer that
archbench's ``gdn`` arch builds (archbench/layers/fla.py:36-38 via build_fla, fla.py:21-33).

Constructor kwargs are those archbench passes from YAML (configs/arch/gdn.yaml:4-9: head_dim, expand_v,
use_gate, use_short_conv, conv_size; configs/*/gdn.yaml: num_heads) plus the auto-passed hidden_size and
layer_idx.  Input conventions follow the in-tree GDN-family layer (archbench/layers/nsgdn.py:525-534):
q, k L2-normalised per head (q scaled by head_dim^-1/2 through the op's default scale), beta = sigmoid(.),
g = -exp(A_log) softplus(a + dt_bias) (natural-log decay), fp32 state.  The output projection is named
``o_proj`` so the reference's zero-init rule for output projections (archbench/model.py:14, :80-82) applies.

The token mixing itself is always the HIP chunk op (training / prefill) or the HIP decode step (T = 1 with
a recurrent state, no grad).  The short causal convolutions (with the q / k normalisation fused in), the gate
functions and the output gated RMSNorm run on their own HIP kernels; the projections are PyTorch linears.  The
six input projections (q, k, v, a, b and the gate) keep fla's separate ``nn.Linear`` parameters (names, shapes
and initialisation, so checkpoints and the reference's init rules carry over) but run as three GEMMs against
their concatenated weights: q, k, v as one (2 key_dim + value_dim columns: a multiple of 256 at the reference
configs, which hipBLASLt's 256-wide tiles cover exactly; with the eight a and b columns added the forward GEMM ran
1.6x longer), the gate (its own contiguous output, which the output norm reads as it is), and a and b.  The
backward accumulates the groups' input gradients inside their GEMMs and splits each weight gradient over the
tokens (_GroupedLinear).
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops


def _weight_grad(dy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """dW = dy^T x (dy [M, N], x [M, K]) in fp32, split over the M tokens: a batch of chunk products summed in fp32.
    A weight gradient reduces over every token into a small N x K output; as one GEMM it has too few output tiles
    to fill the GPU (hipBLASLt at M = 65536: 131 us for N = 8, K = 512; 248 us for N = 512, K = 1024; 400 us for
    N = 3072, K = 512), split 8 or 16 ways 27, 77 and 211 us.  The smaller operand's chunks enter the batched
    product as the transposed left operand (a layout the GEMM reads directly; copying them transposed first cost
    140 us at these sizes); the right operand is always contiguous."""
    M, N = dy.shape
    K = x.shape[1]
    C = 16 if N * K <= 1 << 20 else 8
    if dy.dtype == torch.float32:
        return dy.t() @ x
    if M % C or M // C < 1024:
        return torch.mm(dy.t(), x, out_dtype=torch.float32)
    if N <= K:
        return torch.bmm(dy.view(C, M // C, N).transpose(1, 2), x.view(C, M // C, K), out_dtype=torch.float32).sum(0)
    return torch.bmm(x.view(C, M // C, K).transpose(1, 2), dy.view(C, M // C, N), out_dtype=torch.float32).sum(0).t()


class _GroupedLinear(torch.autograd.Function):
    """y_g = x W[r_g:r_{g+1}]^T for consecutive row groups of one weight: one GEMM per group, each output its own
    contiguous tensor, W cast to x's dtype once (as autocast casts it).  Backward: the groups' input gradients
    accumulated in place into the first (dx += dy_g W_g in the GEMM, no separate sum), and each group's weight
    gradient split over the tokens (_weight_grad) written into its rows of one fp32 gradient (rows outside every
    group: zero), returned in W's dtype."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor, bounds: tuple):
        wc = w.to(x.dtype)
        ctx.save_for_backward(x, wc)
        ctx.bounds, ctx.w_dtype = bounds, w.dtype
        return tuple(F.linear(x, wc[r0:r1]) for r0, r1 in zip(bounds[:-1], bounds[1:]))

    @staticmethod
    def backward(ctx, *dys):
        x, wc = ctx.saved_tensors
        groups = [(r0, r1, None if dy is None else dy.reshape(-1, dy.shape[-1]))
                  for r0, r1, dy in zip(ctx.bounds[:-1], ctx.bounds[1:], dys)]
        x2 = x.reshape(-1, x.shape[-1])
        dx = dw = None
        if ctx.needs_input_grad[0]:
            for r0, r1, dy in groups:
                if dy is not None:
                    dx = dy @ wc[r0:r1] if dx is None else dx.addmm_(dy, wc[r0:r1])
            dx = torch.zeros_like(x) if dx is None else dx.view(x.shape)
        if ctx.needs_input_grad[1]:
            whole = ctx.bounds[0] == 0 and ctx.bounds[-1] == wc.shape[0] and all(g[2] is not None for g in groups)
            dw = (torch.empty if whole else torch.zeros)(wc.shape, dtype=torch.float32, device=wc.device)
            for r0, r1, dy in groups:
                if dy is not None:
                    dw[r0:r1] = _weight_grad(dy, x2)
            dw = dw.to(ctx.w_dtype)
        return dx, dw, None


def _grouped_linear(x: torch.Tensor, w: torch.Tensor, bounds) -> tuple[torch.Tensor, ...]:
    """(x W[r_0:r_1]^T, x W[r_1:r_2]^T, ...) for row bounds r_0 < r_1 < ...; on GPUs one GEMM per group with the
    backward of _GroupedLinear."""
    bounds = tuple(int(r) for r in bounds)
    if x.is_cuda:
        return _GroupedLinear.apply(x, w, bounds)
    wc = w.to(x.dtype)
    return tuple(F.linear(x, wc[r0:r1]) for r0, r1 in zip(bounds[:-1], bounds[1:]))


def _linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """F.linear for a bf16 (or fp32) activation under the layer's own cast; the split-K weight gradient on GPUs."""
    return _grouped_linear(x, w, (0, w.shape[0]))[0]


class ShortConvolution(nn.Module):
    """Depthwise causal conv1d (kernel ``size``) + SiLU over [B, T, D] (the ShortConv of nsgdn.py:457-470), on
    the HIP kernel (``ops.short_conv``).  With ``state`` ([B, D, size-1], the previous inputs) it continues a
    sequence; it always returns the new state.  ``norm_group`` > 0 L2-normalises each group of that many
    channels after the SiLU (one head of q or k, nsgdn.py:527-528)."""

    def __init__(self, dim: int, size: int = 4, bias: bool = False, norm_group: int = 0):
        super().__init__()
        self.size, self.norm_group = size, norm_group
        self.weight = nn.Parameter(torch.empty(dim, 1, size).uniform_(-1 / math.sqrt(size), 1 / math.sqrt(size)))
        self.bias = nn.Parameter(torch.zeros(dim)) if bias else None

    def forward(self, x: torch.Tensor, state: torch.Tensor | None = None):
        # the kernel uses the taps rounded to the activation dtype, as the reference's conv runs its weight
        # (nsgdn.py:464); the bias is rounded here
        b = None if self.bias is None else self.bias.to(x.dtype).float()
        return ops.short_conv(x, self.weight.squeeze(1), b, state, self.norm_group)


class GatedRMSNorm(nn.Module):
    """RMSNorm over the head dimension times swish(gate) (fla's FusedRMSNormGated, nsgdn.py:539-541), one HIP
    pass (``ops.gated_rmsnorm``), fp32 arithmetic, output in x's dtype."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor, gate: torch.Tensor | None = None) -> torch.Tensor:
        return ops.gated_rmsnorm(x, gate, self.weight, self.eps)


class GatedDeltaNet(nn.Module):
    def __init__(self, hidden_size: int = 2048, expand_v: float = 2.0, head_dim: int = 256, num_heads: int = 6,
                 mode: str = "chunk", use_gate: bool = True, use_short_conv: bool = True,
                 allow_neg_eigval: bool = False, conv_size: int = 4, conv_bias: bool = False,
                 layer_idx: int | None = None, norm_eps: float = 1e-5, **kwargs):
        super().__init__()
        if mode not in ("chunk", "fused_recurrent"):
            raise ValueError(f"unknown mode {mode!r}; choose chunk or fused_recurrent")
        self.hidden_size, self.mode = hidden_size, mode
        self.num_heads, self.head_k_dim = num_heads, head_dim
        self.head_v_dim = int(head_dim * expand_v)
        self.key_dim, self.value_dim = num_heads * head_dim, num_heads * self.head_v_dim
        self.use_gate, self.use_short_conv, self.allow_neg_eigval = use_gate, use_short_conv, allow_neg_eigval
        self.layer_idx = layer_idx
        self.q_proj = nn.Linear(hidden_size, self.key_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.key_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.value_dim, bias=False)
        self.a_proj = nn.Linear(hidden_size, num_heads, bias=False)
        self.b_proj = nn.Linear(hidden_size, num_heads, bias=False)
        A = torch.empty(num_heads).uniform_(0, 16)
        self.A_log = nn.Parameter(torch.log(A))
        self.A_log._no_weight_decay = True
        dt_min, dt_max, dt_floor = 0.001, 0.1, 1e-4
        dt = torch.exp(torch.rand(num_heads) * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min))
        dt = dt.clamp(min=dt_floor)
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.dt_bias._no_weight_decay = True
        if use_short_conv:
            # q and k leave their convolution L2-normalised per head (the op's in-kernel normalisation then off)
            self.q_conv1d = ShortConvolution(self.key_dim, conv_size, conv_bias, norm_group=head_dim)
            self.k_conv1d = ShortConvolution(self.key_dim, conv_size, conv_bias, norm_group=head_dim)
            self.v_conv1d = ShortConvolution(self.value_dim, conv_size, conv_bias)
        if use_gate:
            self.g_proj = nn.Linear(hidden_size, self.value_dim, bias=False)
        self.o_norm = GatedRMSNorm(self.head_v_dim, norm_eps)
        self.o_proj = nn.Linear(self.value_dim, hidden_size, bias=False)

    def _grouped_projections(self, hidden_states: torch.Tensor):
        """([q | k | v], gate or None, [a | b]): the six input linears against their concatenated weights, one GEMM
        per group."""
        mods = [self.q_proj, self.k_proj, self.v_proj] + ([self.g_proj] if self.use_gate else [])
        mods += [self.a_proj, self.b_proj]
        n_qkv = 2 * self.key_dim + self.value_dim
        bounds = [0, n_qkv] + ([n_qkv + self.value_dim] if self.use_gate else [])
        bounds.append(bounds[-1] + self.a_proj.out_features + self.b_proj.out_features)
        outs = _grouped_linear(hidden_states, torch.cat([m.weight for m in mods], 0), bounds)
        return outs[0], (outs[1] if self.use_gate else None), outs[-1]

    def input_projections(self, hidden_states: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """(q, k, v, a, b[, gate]) = the six linears of ``hidden_states``, computed as three GEMMs: q, k, v against
        their concatenated weights, the gate, and a and b against theirs."""
        y, gate, ab = self._grouped_projections(hidden_states)
        q, k, v = torch.split(y, [self.key_dim, self.key_dim, self.value_dim], dim=-1)
        a, b = torch.split(ab, [self.a_proj.out_features, self.b_proj.out_features], dim=-1)
        return (q, k, v, a, b) + ((gate,) if self.use_gate else ())

    def forward(self, hidden_states: torch.Tensor, attention_mask: torch.Tensor | None = None,
                past_key_values: dict | None = None, use_cache: bool = False, output_attentions: bool = False,
                **kwargs):
        """hidden_states [B, T, hidden]; returns (o [B, T, hidden], None, past_key_values).

        ``past_key_values`` is a dict keyed by layer_idx holding {"recurrent_state", "conv_state"}; with
        ``use_cache`` the entry is created or advanced (decode continues from it)."""
        if attention_mask is not None:
            raise ValueError("padding masks are not supported by the gated DeltaNet layer")
        B, T, _ = hidden_states.shape
        H, DK, DV = self.num_heads, self.head_k_dim, self.head_v_dim
        dev_type = hidden_states.device.type
        if torch.is_autocast_enabled(dev_type) and hidden_states.dtype == torch.float32:
            # the cast autocast would make in front of each projection GEMM, made once for both (and one cast of
            # the input gradient back in the backward instead of two and their fp32 sum)
            hidden_states = hidden_states.to(torch.get_autocast_dtype(dev_type))
        entry = None if past_key_values is None else past_key_values.get(self.layer_idx)
        conv_in = entry["conv_state"] if entry is not None else (None, None, None)
        conv_out = (None, None, None)
        convs = (self.q_conv1d, self.k_conv1d, self.v_conv1d) if self.use_short_conv else ()
        if convs and entry is None and not use_cache and all(c.bias is None for c in convs):
            # training / prefill without a cache: the convolutions read q, k, v straight out of the projection's
            # output and their backward writes into one gradient of it (ops.mixer_input_stage)
            y, gate, ab = self._grouped_projections(hidden_states)
            w = torch.cat([c.weight.squeeze(1) for c in convs], 0)
            q, k, v = ops.mixer_input_stage(y, w, self.key_dim, self.value_dim, DK)
            gp = [gate] if self.use_gate else []
        else:
            ab = None
            q, k, v, a, b, *gp = self.input_projections(hidden_states)
            if convs:
                (q, cq), (k, ck), (v, cv) = (self.q_conv1d(q, conv_in[0]), self.k_conv1d(k, conv_in[1]),
                                             self.v_conv1d(v, conv_in[2]))
                conv_out = (cq, ck, cv)
            else:
                q, k, v = F.silu(q), F.silu(k), F.silu(v)
        q, k, v = q.reshape(B, T, H, DK), k.reshape(B, T, H, DK), v.reshape(B, T, H, DV)
        # g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) (x2 with negative eigenvalues), one HIP pass;
        # from the [a | b] projection output in place when there is one
        scale_b = 2.0 if self.allow_neg_eigval else 1.0
        if ab is not None:
            g, beta = ops.gdn_gates_ab(ab, self.A_log, self.dt_bias, None, scale_b, float("-inf"))
        else:
            g, beta = ops.gdn_gates(a, b, self.A_log, self.dt_bias, None, scale_b, float("-inf"))
        state = entry["recurrent_state"] if entry is not None else None
        # The op runs in the dtype the projections produced, as fla's layer passes them on: bf16 under the
        # trainer's bf16 autocast (archbench/trainer.py:66), even though the block hands the mixer fp32 hidden
        # states (archbench/model.py:44-45); fp32 only for a caller that runs the projections in fp32.
        if q.dtype not in (torch.bfloat16, torch.float32):
            q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
        l2 = not self.use_short_conv  # the convolutions already normalised q and k
        if self.mode == "fused_recurrent" or (T == 1 and not torch.is_grad_enabled() and state is not None):
            # decode: the cache owns its fp32 state, which the step kernel advances in place
            o, new_state = ops.fused_recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=state,
                                                                output_final_state=use_cache,
                                                                use_qk_l2norm_in_kernel=l2,
                                                                inplace_final_state=use_cache)
        else:
            o, new_state = ops.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=state,
                                                      output_final_state=use_cache, use_qk_l2norm_in_kernel=l2)
        if use_cache:
            if past_key_values is None:
                past_key_values = {}
            past_key_values[self.layer_idx] = {"recurrent_state": new_state, "conv_state": conv_out}
        gate = gp[0].reshape(B, T, H, DV) if self.use_gate else None
        o = self.o_norm(o, gate)
        return _linear(o.reshape(B, T, -1), self.o_proj.weight), None, past_key_values
