"""Pins oracle/ce_oracle.py on the CPU (see its header)."""

import math

import torch
import torch.nn.functional as F

from oracle import ce_oracle as CE


def test_matches_torch_cross_entropy():
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(37, 24, generator=gen, dtype=torch.float64)
    w = torch.randn(104, 24, generator=gen, dtype=torch.float64) * 0.3
    t = torch.randint(0, 104, (37,), generator=gen)
    t[3] = t[20] = -100
    loss, dx, dw = CE.linear_ce(x, t, w)
    xs, ws = x.clone().requires_grad_(), w.clone().requires_grad_()
    ref = F.cross_entropy(xs @ ws.T, t, ignore_index=-100)  # archbench/model.py:146
    ref.backward()
    torch.testing.assert_close(loss, ref.detach())
    torch.testing.assert_close(dx, xs.grad)
    torch.testing.assert_close(dw, ws.grad)
    rows, lse, g = CE.ce_rows(x @ w.T, t, -100, 0.5)
    torch.testing.assert_close(lse, torch.logsumexp(x @ w.T, -1))
    assert rows[3] == 0 and not g[3].any()


def test_closed_forms():
    V = 16
    rows, lse, g = CE.ce_rows(torch.zeros(3, V), torch.tensor([0, 5, 15]), -100, 1.0)
    torch.testing.assert_close(rows, torch.full((3,), math.log(V), dtype=torch.float64))
    want = torch.full((3, V), 1.0 / V, dtype=torch.float64)
    want[0, 0] -= 1
    want[1, 5] -= 1
    want[2, 15] -= 1
    torch.testing.assert_close(g, want)
    loss, dx, dw = CE.linear_ce(torch.randn(4, 8), torch.full((4,), -100), torch.randn(V, 8))
    assert loss == 0 and not dx.any() and not dw.any()


def test_gradcheck():
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(5, 6, generator=gen, dtype=torch.float64, requires_grad=True)
    w = torch.randn(8, 6, generator=gen, dtype=torch.float64, requires_grad=True)
    t = torch.tensor([1, 7, -100, 0, 3])
    f = lambda a, b: CE.ce_rows(a @ b.T, t)[0].sum() / 4
    assert torch.autograd.gradcheck(f, (x, w))
