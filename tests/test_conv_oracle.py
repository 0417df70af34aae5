"""Pins the short-conv oracle (oracle/conv_oracle.py) on the CPU."""

import pytest
import torch
import torch.nn.functional as F

from oracle import conv_oracle as C


def _inputs(B=2, T=37, D=16, W=4, seed=0, state=True, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    w = torch.randn(D, W, generator=g, dtype=torch.float64) * 0.5
    b = torch.randn(D, generator=g, dtype=torch.float64) * 0.1 if bias else None
    s = torch.randn(B, D, W - 1, generator=g, dtype=torch.float64) if state else None
    return x, w, b, s


def test_matches_torch_conv1d():
    """The explicit tap sum equals the reference's own CPU path: F.conv1d(groups=D, padding=W-1)[:T] + SiLU."""
    x, w, b, _ = _inputs(state=False)
    y, _ = C.short_conv_fwd(x, w, b)
    T, D, W = x.shape[1], x.shape[2], w.shape[1]
    ref = F.conv1d(x.transpose(1, 2), w.unsqueeze(1), b, padding=W - 1, groups=D)[..., :T]
    assert torch.allclose(y, F.silu(ref.transpose(1, 2)), atol=1e-12)


def test_width_one_is_pointwise():
    x, w, b, _ = _inputs(W=1, state=False)
    y, _ = C.short_conv_fwd(x, w, b)
    assert torch.allclose(y, F.silu(x * w[:, 0] + b), atol=1e-12)


def test_state_passing():
    x, w, b, s = _inputs(T=41)
    y, s_end = C.short_conv_fwd(x, w, b, s)
    y1, s1 = C.short_conv_fwd(x[:, :17], w, b, s)
    y2, s2 = C.short_conv_fwd(x[:, 17:], w, b, s1)
    assert torch.allclose(torch.cat([y1, y2], 1), y, atol=1e-12)
    assert torch.allclose(s2, s_end, atol=0)
    assert torch.equal(s_end, x[:, -3:].transpose(1, 2))


def test_short_sequence_state_keeps_old_inputs():
    x, w, b, s = _inputs(T=2)
    _, s_end = C.short_conv_fwd(x, w, b, s)
    assert torch.equal(s_end[..., 0], s[..., 2])  # the oldest surviving input comes from the old state
    assert torch.equal(s_end[..., 1:], x.transpose(1, 2))


@pytest.mark.parametrize("G", [4, 8, 16])
def test_group_norm_unit(G):
    x, w, b, s = _inputs()
    y, _ = C.short_conv_fwd(x, w, b, s, norm_group=G)
    n = y.view(*y.shape[:2], -1, G).norm(dim=-1)
    assert torch.allclose(n, torch.ones_like(n), atol=1e-12)


def test_gradcheck():
    x, w, b, s = _inputs(B=1, T=9, D=8)
    for G in (0, 4):
        f = lambda x_, w_, b_, s_: C.short_conv_fwd(x_, w_, b_, s_, norm_group=G)[0]
        assert torch.autograd.gradcheck(f, (x.requires_grad_(), w.requires_grad_(), b.requires_grad_(),
                                            s.requires_grad_()))


def test_bwd_matches_finite_differences_on_dw():
    x, w, b, s = _inputs(B=1, T=12, D=8)
    dy = torch.randn_like(x)
    _, dw, _, _ = C.short_conv_bwd(x, w, b, s, dy, norm_group=4)
    eps = 1e-6
    for c, i in [(0, 0), (3, 2), (7, 3)]:
        wp, wm = w.clone(), w.clone()
        wp[c, i] += eps
        wm[c, i] -= eps
        fp = (C.short_conv_fwd(x, wp, b, s, 4)[0] * dy).sum()
        fm = (C.short_conv_fwd(x, wm, b, s, 4)[0] * dy).sum()
        assert abs(((fp - fm) / (2 * eps)).item() - dw[c, i].item()) < 1e-6
