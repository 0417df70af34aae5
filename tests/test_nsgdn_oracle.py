"""Pins oracle/nsgdn_oracle.py (separate read / write vectors) on the CPU: reduction to the pinned gated delta
rule oracle at u = beta k, chunk form = token recurrence, brute-force affine-map products, the T = 1 closed
form, fp64 gradcheck, and write_direction's invariant, per-step contraction and two-step closed form, with planted
mistakes that the pins must catch (nsgdn.py:61-75, :240-249, :408-417)."""

import torch
import torch.nn.functional as F

from oracle import gdn_oracle as G
from oracle import nsgdn_oracle as NS


def _inputs(B=2, T=37, H=2, K=8, V=6, seed=0, h0=True):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen, dtype=torch.float64)
    q, k = F.normalize(r(B, T, H, K), dim=-1), F.normalize(r(B, T, H, K), dim=-1)
    u = 0.5 * r(B, T, H, K)
    v = r(B, T, H, V)
    la = F.logsigmoid(r(B, T, H) + 3)
    h = 0.1 * r(B, H, K, V) if h0 else None
    return q, k, u, v, la, h


def test_reduces_to_gated_delta_rule():
    q, k, _, v, la, h0 = _inputs()
    beta = torch.rand(*la.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    u = beta[..., None] * k
    y, hT = NS.recurrent_fwd(q, k, u, v, la, 0.7, h0)
    y2, hT2 = G.recurrent_fwd(q, k, v, la, beta, 0.7, h0)
    torch.testing.assert_close(y, y2)
    torch.testing.assert_close(hT, hT2)


def test_chunk_form_equals_recurrence():
    q, k, u, v, la, h0 = _inputs(T=70)
    y, hT = NS.recurrent_fwd(q, k, u, v, la, 0.5, h0)
    for c in (1, 16, 64):
        yc, hc = NS.chunk_fwd(q, k, u, v, la, 0.5, h0, chunk=c)
        torch.testing.assert_close(yc, y)
        torch.testing.assert_close(hc, hT)


def test_brute_force_affine_maps():
    q, k, u, v, la, h0 = _inputs(B=1, T=9, H=1)
    S = h0[0, 0].clone()
    for t in range(9):
        a = la[0, t, 0].exp()
        kt, ut, vt = k[0, t, 0], u[0, t, 0], v[0, t, 0]
        # S_t = a (I - u k^T) S_{t-1} + u v^T  (K x V form)
        S = a * (torch.eye(8, dtype=torch.float64) - torch.outer(ut, kt)) @ S + torch.outer(ut, vt)
    _, hT = NS.recurrent_fwd(q, k, u, v, la, 1.0, h0)
    torch.testing.assert_close(hT[0, 0], S)


def test_t1_closed_form():
    q, k, u, v, la, h0 = _inputs(T=1)
    a = la[:, 0].exp()[..., None, None]
    S1 = a * h0 + u[:, 0][..., :, None] * (v[:, 0] - torch.einsum("bhkv,bhk->bhv", a * h0, k[:, 0]))[..., None, :]
    y, hT = NS.recurrent_fwd(q, k, u, v, la, 2.0, h0)
    torch.testing.assert_close(hT, S1)
    torch.testing.assert_close(y[:, 0], 2.0 * torch.einsum("bhkv,bhk->bhv", S1, q[:, 0]))


def test_gradcheck():
    q, k, u, v, la, h0 = _inputs(B=1, T=5, H=1, K=3, V=2)
    args = tuple(x.clone().requires_grad_() for x in (q, k, u, v, la, h0))
    assert torch.autograd.gradcheck(lambda *a: NS.chunk_fwd(*a[:5], 0.9, a[5], chunk=2)[0], args)
    dy = torch.randn(1, 5, 1, 2, dtype=torch.float64)
    got = NS.recurrent_bwd(q, k, u, v, la, dy, 0.9, h0)
    leaves = [x.clone().requires_grad_() for x in (q, k, u, v, la, h0)]
    (NS.chunk_fwd(*leaves[:5], 0.9, leaves[5], chunk=2)[0] * dy).sum().backward()
    for a, b in zip(got, leaves):
        torch.testing.assert_close(a, b.grad)


def test_write_direction():
    q, k, _, _, la, _ = _inputs(T=12)
    beta = torch.sigmoid(torch.randn(*la.shape, generator=torch.Generator().manual_seed(2), dtype=torch.float64))
    p = F.pad(k[:, :-1], (0, 0, 0, 0, 1, 0))
    lam = torch.tensor([0.5, 1.5], dtype=torch.float64)
    torch.testing.assert_close(NS.write_direction(k, p, beta, lam, 1), beta[..., None] * k)
    u3 = NS.write_direction(k, p, beta, lam, 3)
    torch.testing.assert_close((u3 * k).sum(-1), beta)  # the current-key gain is kept for unit k
    assert not torch.allclose(u3, beta[..., None] * k)


def _wd_case(T=20):
    q, k, _, _, la, _ = _inputs(T=T, K=8)
    gen = torch.Generator().manual_seed(5)
    beta = torch.rand(*la.shape, generator=gen, dtype=torch.float64)
    lam = torch.tensor([0.7, 1.8], dtype=torch.float64)
    p = torch.randn(*k.shape, generator=gen, dtype=torch.float64)  # any p (the layer passes the previous key)
    return k, p, beta, lam


def _wd_pins(wd) -> None:
    """Properties that fix write_direction's step coefficient (the reference states the first at nsgdn.py:64-66):
    * contraction: for unit k each step scales p . u by (1 - lam beta |p_perp|^2), so
      p . u_n = beta (p . k) (1 - lam beta |p_perp|^2)^(n-1);
    * the n = 2 closed form u_2 = beta k - lam beta^2 (p . k) p_perp;
    * u_n - beta k lies along p_perp (every step moves u along p_perp only)."""
    k, p, beta, lam = _wd_case()
    b, lm = beta[..., None], lam[None, None, :, None]
    pk = (p * k).sum(-1, keepdim=True)
    p_perp = p - pk * k
    shrink = 1 - lm * b * (p_perp * p_perp).sum(-1, keepdim=True)
    for n in (2, 3, 4):
        u = wd(k, p, beta, lam, n)
        torch.testing.assert_close((p * u).sum(-1, keepdim=True), b * pk * shrink ** (n - 1))
        resid = u - b * k
        along = (resid * p_perp).sum(-1, keepdim=True) / (p_perp * p_perp).sum(-1, keepdim=True)
        torch.testing.assert_close(resid, along * p_perp)
    torch.testing.assert_close(wd(k, p, beta, lam, 2), b * k - lm * b * b * pk * p_perp)


def test_write_direction_pinned_for_several_steps():
    _wd_pins(NS.write_direction)


def test_write_direction_pins_catch_planted_mistakes():
    """Restatements with a flipped step sign, a dropped lam, a dropped beta (all three keep the k . u = beta
    invariant of test_write_direction) or p in place of p_perp must each fail the pins."""
    def mutant(kind):
        def wd(k, p, beta, lam, n_steps):
            b, lm = beta[..., None], lam[None, None, :, None]
            u = b * k
            p_perp = p - (p * k).sum(-1, keepdim=True) * k
            for _ in range(n_steps - 1):
                c = {"sign": -lm * b, "lam": b, "beta": lm, "p": lm * b}[kind]
                d = p if kind == "p" else p_perp
                u = u - c * (p * u).sum(-1, keepdim=True) * d
            return u
        return wd

    for kind in ("sign", "lam", "beta", "p"):
        try:
            _wd_pins(mutant(kind))
        except AssertionError:
            continue
        raise AssertionError(f"planted write_direction mistake {kind!r} passed the pins")
