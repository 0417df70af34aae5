"""CPU oracle for the fused linear + cross-entropy (archbench/fused_ce.py:20-57).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package ``archbench_amd`` imports, calls or links this
module; ``tests/`` use it as the checker.

* ``ce_rows(logits, target, ignore_index, dloss)`` -- per-row loss logsumexp(x) - x_t (0 for ignored rows) and the
  in-place gradient dloss * (softmax - onehot) that fla's cross_entropy_fwd / cross_entropy_bwd produce on each
  chunk (fused_ce.py:33-45), written out with an explicit max-shifted logsumexp.
* ``linear_ce(x, target, weight, ignore_index)`` -- the whole op: mean over non-ignored tokens of the
  cross-entropy of x W^T (the divisor clamped to 1 as fused_ce.py:24-25), with dx and dW by autograd.

Parity status: pinned in tests/test_ce_oracle.py against torch.nn.functional.cross_entropy (the reference's
unfused path, archbench/model.py:142-147), closed forms (all-zero logits: loss log V and gradient 1/V - onehot),
the all-ignored case (loss 0, zero gradients), and gradcheck.
"""

from __future__ import annotations

import torch


def ce_rows(logits, target, ignore_index: int = -100, dloss: float = 1.0, dtype=torch.float64):
    x = logits.to("cpu", dtype)
    t = target.to("cpu")
    m = x.max(-1, keepdim=True).values
    lse = (m + (x - m).exp().sum(-1, keepdim=True).log()).squeeze(-1)
    ign = t == ignore_index
    tt = torch.where(ign, torch.zeros_like(t), t)
    loss = torch.where(ign, torch.zeros_like(lse), lse - x.gather(1, tt[:, None]).squeeze(1))
    grad = (x - lse[:, None]).exp()
    grad[torch.arange(x.shape[0]), tt] -= 1.0
    grad = torch.where(ign[:, None], torch.zeros_like(grad), grad * dloss)
    return loss, lse, grad


def linear_ce(x, target, weight, ignore_index: int = -100, dtype=torch.float64):
    """(loss, dx, dW)."""
    xs = x.detach().to("cpu", dtype).requires_grad_()
    ws = weight.detach().to("cpu", dtype).requires_grad_()
    t = target.to("cpu")
    loss_rows, _, _ = ce_rows(xs @ ws.T, t, ignore_index, 1.0, dtype)
    total = (t != ignore_index).sum().clamp_min(1)
    loss = loss_rows.sum() / total
    loss.backward()
    return loss.detach(), xs.grad, ws.grad
