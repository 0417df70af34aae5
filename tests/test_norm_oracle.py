"""Pins oracle/norm_oracle.py (gated RMSNorm and the g / beta gates) on the CPU: against torch's own
F.rms_norm / F.silu / F.softplus / sigmoid composition (the reference's code path, nsgdn.py:531-541), closed forms
and invariants, and fp64 gradcheck."""

import math

import torch
import torch.nn.functional as F

from oracle import norm_oracle as N


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_norm_matches_torch_composition():
    x = torch.randn(3, 5, 2, 128, generator=_g(0), dtype=torch.float64)
    gate = torch.randn(3, 5, 2, 128, generator=_g(1), dtype=torch.float64)
    w = torch.rand(128, generator=_g(2), dtype=torch.float64) + 0.5
    ref = F.rms_norm(x, (128,), w, 1e-5) * F.silu(gate)  # nn.RMSNorm then y * silu(g), nsgdn.py:539-541
    torch.testing.assert_close(N.gated_rmsnorm_fwd(x, gate, w, 1e-5), ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(N.gated_rmsnorm_fwd(x, None, w, 1e-5), F.rms_norm(x, (128,), w, 1e-5),
                               rtol=1e-12, atol=1e-12)


def test_norm_closed_forms():
    # a constant row c: mean(x^2) = c^2, y = c / sqrt(c^2 + eps) * w * silu(g)
    c, eps = 0.3, 1e-5
    x = torch.full((1, 64), c, dtype=torch.float64)
    gate = torch.full((1, 64), 0.7, dtype=torch.float64)
    y = N.gated_rmsnorm_fwd(x, gate, None, eps)
    want = c / math.sqrt(c * c + eps) * 0.7 / (1 + math.exp(-0.7))
    assert torch.allclose(y, torch.full_like(y, want), rtol=1e-14)
    # zero gate -> zero output; scale invariance (eps -> 0)
    assert not N.gated_rmsnorm_fwd(x, torch.zeros_like(x), None, eps).any()
    z = torch.randn(4, 256, generator=_g(3), dtype=torch.float64)
    torch.testing.assert_close(N.gated_rmsnorm_fwd(7.5 * z, None, None, 0.0), N.gated_rmsnorm_fwd(z, None, None, 0.0))
    # unit RMS rows come back unchanged
    u = z / z.pow(2).mean(-1, keepdim=True).sqrt()
    torch.testing.assert_close(N.gated_rmsnorm_fwd(u, None, None, 0.0), u)


def test_norm_gradcheck():
    x = torch.randn(2, 3, 64, generator=_g(4), dtype=torch.float64)
    gate = torch.randn(2, 3, 64, generator=_g(5), dtype=torch.float64)
    w = torch.rand(64, generator=_g(6), dtype=torch.float64) + 0.5
    dy = torch.randn(2, 3, 64, generator=_g(7), dtype=torch.float64)
    dx, dgate, dw = N.gated_rmsnorm_bwd(x, gate, w, dy, 1e-5)
    xs, gs, ws = (t.clone().requires_grad_() for t in (x, gate, w))
    ((F.rms_norm(xs, (64,), ws, 1e-5) * F.silu(gs)) * dy).sum().backward()
    torch.testing.assert_close(dx, xs.grad)
    torch.testing.assert_close(dgate, gs.grad)
    torch.testing.assert_close(dw, ws.grad)
    assert torch.autograd.gradcheck(lambda a, b, c: N.gated_rmsnorm_fwd(a, b, c, 1e-5),
                                    (xs.detach().requires_grad_(), gs.detach().requires_grad_(),
                                     ws.detach().requires_grad_()))


def test_gates_match_torch_composition():
    H = 6
    a = torch.randn(4, 9, H, generator=_g(8), dtype=torch.float64) * 3
    b = torch.randn(4, 9, H, generator=_g(9), dtype=torch.float64) * 3
    A_log = torch.rand(H, generator=_g(10), dtype=torch.float64).mul(15).add(1).log()
    dt_bias = torch.randn(H, generator=_g(11), dtype=torch.float64)
    b_bias = torch.randn(H, generator=_g(12), dtype=torch.float64)
    g, beta = N.gates_fwd(a, b, A_log, dt_bias, b_bias)
    torch.testing.assert_close(g, -F.softplus(a + dt_bias) * A_log.exp())  # nsgdn.py:531
    torch.testing.assert_close(beta, torch.sigmoid(b + b_bias))  # nsgdn.py:534
    g2, beta2 = N.gates_fwd(a, b, A_log, dt_bias, None, beta_scale=2.0, g_min=-1.0)
    torch.testing.assert_close(g2, (-F.softplus(a + dt_bias) * A_log.exp()).clamp_min(-1.0))  # nsgdn.py:533
    torch.testing.assert_close(beta2, 2 * torch.sigmoid(b))
    # softplus threshold: above 20 the input itself
    big = torch.full((1, H), 25.0, dtype=torch.float64)
    torch.testing.assert_close(N.gates_fwd(big, big, torch.zeros(H, dtype=torch.float64))[0], -big)


def test_gates_gradients():
    H = 5
    a = torch.randn(3, 7, H, generator=_g(13), dtype=torch.float64) * 3
    b = torch.randn(3, 7, H, generator=_g(14), dtype=torch.float64)
    A_log = torch.rand(H, generator=_g(15), dtype=torch.float64)
    dt_bias = torch.randn(H, generator=_g(16), dtype=torch.float64)
    b_bias = torch.randn(H, generator=_g(17), dtype=torch.float64)
    dg = torch.randn(3, 7, H, generator=_g(18), dtype=torch.float64)
    dbeta = torch.randn(3, 7, H, generator=_g(19), dtype=torch.float64)
    got = N.gates_bwd(a, b, A_log, dt_bias, b_bias, dg, dbeta, beta_scale=2.0, g_min=-2.0)
    leaves = [t.clone().requires_grad_() for t in (a, b, A_log, dt_bias, b_bias)]
    la = (-F.softplus(leaves[0] + leaves[3]) * leaves[2].exp()).clamp_min(-2.0)
    be = 2 * torch.sigmoid(leaves[1] + leaves[4])
    (la * dg + be * dbeta).sum().backward()
    for x, l in zip(got, leaves):
        torch.testing.assert_close(x, l.grad)
    # dA_log = sum of g * dg where unclamped (d/dA_log of -e^A sp = itself)
    g_unc = -F.softplus(a + dt_bias) * A_log.exp()
    want = torch.where(g_unc >= -2.0, g_unc * dg, torch.zeros_like(dg)).sum((0, 1))
    torch.testing.assert_close(got[2], want)


def test_l2norm_matches_normalize():
    x = torch.randn(3, 4, 128, generator=_g(20), dtype=torch.float64)
    torch.testing.assert_close(N.l2norm_fwd(x, 1e-12, 128 ** -0.5), F.normalize(x, dim=-1) * 128 ** -0.5)  # :527
    # unit rows unchanged at scale 1; rows below eps are divided by eps, not by their norm
    u = F.normalize(x, dim=-1)
    torch.testing.assert_close(N.l2norm_fwd(u), u)
    tiny = torch.full((1, 64), 1e-8, dtype=torch.float64)
    torch.testing.assert_close(N.l2norm_fwd(tiny, 1e-3), tiny / 1e-3)
    # gradient: orthogonal to x for rows above eps (the projection (I - x x^T / |x|^2) / |x|)
    dy = torch.randn(3, 4, 128, generator=_g(21), dtype=torch.float64)
    dx = N.l2norm_bwd(x, dy)
    assert (dx * x).sum(-1).abs().max() < 1e-12
    assert torch.autograd.gradcheck(lambda a: N.l2norm_fwd(a, 1e-12, 0.5), (x[:1, :1].clone().requires_grad_(),))
