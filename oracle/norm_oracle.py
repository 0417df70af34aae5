"""CPU oracle for the elementwise work on either side of the GDN op: the output gated RMSNorm and the g / beta
gate functions.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package ``archbench_amd`` imports, calls or links this
module; ``tests/`` use it as the checker.

What it restates (reference file:line, paths relative to the archbench tree):

* ``gated_rmsnorm_fwd`` -- the mixer's output normalisation: ``self.norm(y)`` (an ``nn.RMSNorm(DV, eps)`` over
  each head, nsgdn.py:510, :539) followed by ``y * F.silu(g)`` (nsgdn.py:540-541); fla's FusedRMSNormGated in
  GatedDeltaNet computes the same product in one pass.  Written out as x / sqrt(mean(x^2) + eps) * w * g *
  sigmoid(g) over the last dimension, in the oracle's dtype (no intermediate rounding).
* ``gates_fwd`` -- ``la = -softplus(ab[..., :H] + dt_bias) * exp(A_log)``, ``la.clamp_min(la_min)``,
  ``beta = sigmoid(ab[..., H:] + b_bias)`` (nsgdn.py:531-534), with fla GatedDeltaNet's ``beta * 2`` option
  (allow_neg_eigval) as ``beta_scale``.  softplus is log(1 + e^x), and x itself above 20 (torch's threshold).
* ``l2norm_fwd`` -- the per-head normalisation of q and k, ``F.normalize(.) * DK**-0.5`` (nsgdn.py:527-528):
  scale * x / max(||x||, eps).
* ``*_bwd`` -- gradients of the above by autograd in the oracle's dtype.

Parity status: pinned in tests/test_norm_oracle.py against torch's own F.rms_norm / F.silu / F.softplus /
torch.sigmoid / F.normalize composition (the reference's code path), closed forms (constant rows, unit weight,
zero gate, unit-norm rows), scale invariance of the norms, and fp64 gradcheck.
"""

from __future__ import annotations

import torch


def gated_rmsnorm_fwd(x, gate=None, weight=None, eps: float = 1e-5, dtype=torch.float64):
    x = x.to("cpu", dtype)
    r = 1.0 / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
    y = x * r
    if weight is not None:
        y = y * weight.to("cpu", dtype)
    if gate is not None:
        gt = gate.to("cpu", dtype)
        y = y * gt * torch.sigmoid(gt)
    return y


def gated_rmsnorm_bwd(x, gate, weight, dy, eps: float = 1e-5, dtype=torch.float64):
    """(dx, dgate | None, dweight | None) of sum(y * dy)."""
    xs = x.detach().to("cpu", dtype).requires_grad_()
    gs = None if gate is None else gate.detach().to("cpu", dtype).requires_grad_()
    ws = None if weight is None else weight.detach().to("cpu", dtype).requires_grad_()
    y = gated_rmsnorm_fwd(xs, gs, ws, eps, dtype)
    (y * dy.to("cpu", dtype)).sum().backward()
    return xs.grad, (None if gs is None else gs.grad), (None if ws is None else ws.grad)


def _softplus(x):
    return torch.where(x > 20, x, torch.log1p(torch.exp(torch.clamp(x, max=20))))


def gates_fwd(a, b, A_log, dt_bias=None, b_bias=None, beta_scale: float = 1.0, g_min: float = float("-inf"),
              dtype=torch.float64):
    """(g, beta) in ``dtype``."""
    a, b = a.to("cpu", dtype), b.to("cpu", dtype)
    xa = a if dt_bias is None else a + dt_bias.to("cpu", dtype)
    g = -torch.exp(A_log.to("cpu", dtype)) * _softplus(xa)
    if g_min != float("-inf"):
        g = g.clamp_min(g_min)
    xb = b if b_bias is None else b + b_bias.to("cpu", dtype)
    return g, beta_scale * torch.sigmoid(xb)


def gates_bwd(a, b, A_log, dt_bias, b_bias, dg, dbeta, beta_scale: float = 1.0, g_min: float = float("-inf"),
              dtype=torch.float64):
    """(da, db, dA_log, ddt_bias | None, db_bias | None) of sum(g * dg + beta * dbeta)."""
    leaves = [None if t is None else t.detach().to("cpu", dtype).requires_grad_()
              for t in (a, b, A_log, dt_bias, b_bias)]
    g, beta = gates_fwd(*leaves, beta_scale=beta_scale, g_min=g_min, dtype=dtype)
    (g * dg.to("cpu", dtype) + beta * dbeta.to("cpu", dtype)).sum().backward()
    return tuple(None if t is None else t.grad for t in leaves)


def l2norm_fwd(x, eps: float = 1e-12, scale: float = 1.0, dtype=torch.float64):
    """scale * x / max(||x||, eps) over the last dimension (F.normalize, nsgdn.py:527-528)."""
    x = x.to("cpu", dtype)
    return scale * x / torch.clamp(x.norm(dim=-1, keepdim=True), min=eps)


def l2norm_bwd(x, dy, eps: float = 1e-12, scale: float = 1.0, dtype=torch.float64):
    xs = x.detach().to("cpu", dtype).requires_grad_()
    (l2norm_fwd(xs, eps, scale, dtype) * dy.to("cpu", dtype)).sum().backward()
    return xs.grad
