"""CPU oracle for the short causal convolution + SiLU (+ per-group L2 normalisation) in front of the GDN op.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package ``archbench_amd`` imports, calls or links this
module; ``tests/`` use it as the checker.

What it restates (reference file:line, paths relative to the archbench tree):

* ``short_conv_fwd`` -- ``ShortConv.forward`` (archbench/layers/nsgdn.py:457-470): a depthwise causal conv1d of
  kernel size W over the channel-last activations followed by SiLU (the CPU branch, nsgdn.py:467-470, and the
  causal_conv1d op with activation=True, nsgdn.py:425-428), extended with fla ShortConvolution's optional bias
  and conv state (the previous W-1 inputs, used by decode), and with the per-head L2 normalisation that the
  GatedDeltaNet layer applies to q and k (nsgdn.py:527-528; F.normalize, eps 1e-12).  Written as an explicit
  sum over the W taps.
* ``short_conv_bwd`` -- the gradient of ``short_conv_fwd`` by autograd in the oracle's dtype (the reference's
  backward is causal_conv1d_bwd_function, nsgdn.py:433-437).

Conventions: x [B, T, D]; w [D, W]; bias [D] or None; state [B, D, W-1] (oldest input first); the
normalisation group is ``norm_group`` consecutive channels (0 = none).

Parity status: pinned in tests/test_conv_oracle.py against torch.nn.functional.conv1d (groups = D, the
reference's own CPU path), the W = 1 pointwise case, state passing, unit group norms, and fp64 gradcheck.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def short_conv_fwd(x, w, bias=None, state=None, norm_group: int = 0, dtype=torch.float64):
    """(y [B,T,D], new_state [B,D,W-1]) in ``dtype``."""
    B, T, D = x.shape
    W = w.shape[-1]
    x = x.to("cpu", dtype)
    w = w.to("cpu", dtype)
    prev = torch.zeros(B, W - 1, D, dtype=dtype) if state is None else state.to("cpu", dtype).transpose(1, 2)
    xp = torch.cat([prev, x], dim=1)  # [B, W-1+T, D]; position t of x is index t + W-1
    z = torch.zeros(B, T, D, dtype=dtype)
    for i in range(W):
        z = z + w[:, i] * xp[:, i:i + T]
    if bias is not None:
        z = z + bias.to("cpu", dtype)
    y = F.silu(z)
    if norm_group:
        y = F.normalize(y.view(B, T, D // norm_group, norm_group), dim=-1, eps=1e-12).view(B, T, D)
    new_state = xp[:, -(W - 1):].transpose(1, 2) if W > 1 else xp[:, :0].transpose(1, 2)
    return y, new_state


def short_conv_bwd(x, w, bias, state, dy, norm_group: int = 0, dtype=torch.float64):
    """(dx, dw, dbias | None, dstate | None) of sum(y * dy) in ``dtype``."""
    xs = x.detach().to("cpu", dtype).requires_grad_()
    ws = w.detach().to("cpu", dtype).requires_grad_()
    bs = None if bias is None else bias.detach().to("cpu", dtype).requires_grad_()
    ss = None if state is None else state.detach().to("cpu", dtype).requires_grad_()
    y, _ = short_conv_fwd(xs, ws, bs, ss, norm_group, dtype)
    (y * dy.to("cpu", dtype)).sum().backward()
    return xs.grad, ws.grad, (None if bs is None else bs.grad), (None if ss is None else ss.grad)
