"""Pins the CPU oracle (oracle/gdn_oracle.py) with closed forms, invariants and brute force.

The reference ships no tests or golden vectors for this path, so each check below is chosen so that a
plausible slip in the restatement (output read before the write, beta on the wrong side, a transposed state,
a dropped decay, a wrong sign in the reverse recurrence) fails at least one of them.
"""

import math

import pytest
import torch

from archbench_amd.synthetic import make_inputs
from oracle import gdn_oracle as O

D = torch.float64


def _inp(B=2, T=16, H=3, K=8, V=6, seed=0, **kw):
    x = make_inputs(B, T, H, K, V, seed=seed, **kw)
    return x


def test_t1_closed_form():
    # S1 = a S0 + beta k (v - a S0^T k)^T ;  o = S1^T (s q)
    x = _inp(T=1, h0_std=0.5)
    s = 0.37
    o, S = O.recurrent_fwd(x.q, x.k, x.v, x.g, x.beta, s, x.h0)
    a = x.g[:, 0].double().exp()[..., None, None]
    S0 = x.h0.double()
    k, q, v, b = x.k[:, 0].double(), x.q[:, 0].double(), x.v[:, 0].double(), x.beta[:, 0].double()
    r = b[..., None] * (v - (a * S0 * k[..., :, None]).sum(-2))
    S1 = a * S0 + k[..., :, None] * r[..., None, :]
    o1 = (S1 * (s * q)[..., :, None]).sum(-2)
    torch.testing.assert_close(S, S1, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(o[:, 0], o1, rtol=1e-12, atol=1e-12)


def test_beta_zero_is_pure_decay():
    x = _inp(T=20, h0_std=1.0)
    beta = torch.zeros_like(x.beta)
    o, S = O.recurrent_fwd(x.q, x.k, x.v, x.g, beta, 1.0, x.h0)
    G = x.g.double().cumsum(1)  # [B,T,H]
    S_exp = G[:, -1].exp()[..., None, None] * x.h0.double()
    torch.testing.assert_close(S, S_exp, rtol=1e-12, atol=1e-12)
    o_exp = torch.einsum("bhkv,bthk->bthv", x.h0.double(), x.q.double()) * G.exp()[..., None]
    torch.testing.assert_close(o, o_exp, rtol=1e-12, atol=1e-12)


def test_delta_rule_exact_write_and_orthogonal_keys():
    # g = 0, beta = 1, unit k  =>  S_t^T k_t = v_t exactly; with orthonormal keys earlier writes are untouched.
    B, T, H, K, V = 1, 6, 2, 8, 5
    x = _inp(B, T, H, K, V, h0_std=1.0)
    Qm, _ = torch.linalg.qr(torch.randn(H, K, K, generator=torch.Generator().manual_seed(3), dtype=D))
    k = Qm[:, :, :T].permute(2, 0, 1)[None].contiguous()  # [1,T,H,K], orthonormal over t
    g = torch.zeros(B, T, H, dtype=D)
    beta = torch.ones(B, T, H, dtype=D)
    _, S = O.recurrent_fwd(x.q, k, x.v, g, beta, 1.0, x.h0)
    for t in range(T):
        torch.testing.assert_close(torch.einsum("bhkv,bhk->bhv", S, k[:, t]), x.v[:, t].double(),
                                   rtol=1e-12, atol=1e-12)
    # directions orthogonal to every key keep their initial content
    P = torch.eye(K, dtype=D) - torch.einsum("thk,thj->hkj", k[0], k[0])
    torch.testing.assert_close(P @ S[0], P @ x.h0[0].double(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 8, 16, 32, 64])
@pytest.mark.parametrize("T", [1, 37, 64, 100])
def test_chunk_form_equals_token_recurrence(chunk, T):
    x = _inp(B=2, T=T, H=2, K=16, V=8, h0_std=0.3)
    o_r, S_r = O.recurrent_fwd(x.q, x.k, x.v, x.g, x.beta, 0.5, x.h0)
    o_c, S_c = O.chunk_fwd(x.q, x.k, x.v, x.g, x.beta, 0.5, x.h0, chunk=chunk)
    torch.testing.assert_close(o_c, o_r, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(S_c, S_r, rtol=1e-10, atol=1e-10)


def test_chunk_form_strong_decay_no_overflow():
    # large negative g: pairwise exp(G_i - G_j) stays <= 1 (no exp(G_i)/exp(G_j) overflow)
    x = _inp(B=1, T=128, H=2, K=16, V=8, g_shift=-6.0)
    o_r, S_r = O.recurrent_fwd(x.q, x.k, x.v, x.g * 20, x.beta, 1.0)
    o_c, S_c = O.chunk_fwd(x.q, x.k, x.v, x.g * 20, x.beta, 1.0, chunk=64)
    assert torch.isfinite(o_c).all()
    torch.testing.assert_close(o_c, o_r, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(S_c, S_r, rtol=1e-9, atol=1e-9)


def test_state_passing():
    x = _inp(B=2, T=50, H=2, K=8, V=8, h0_std=0.2)
    o, S = O.recurrent_fwd(x.q, x.k, x.v, x.g, x.beta, 1.0, x.h0)
    t1 = 23
    o1, S1 = O.recurrent_fwd(x.q[:, :t1], x.k[:, :t1], x.v[:, :t1], x.g[:, :t1], x.beta[:, :t1], 1.0, x.h0)
    o2, S2 = O.chunk_fwd(x.q[:, t1:], x.k[:, t1:], x.v[:, t1:], x.g[:, t1:], x.beta[:, t1:], 1.0, S1, chunk=16)
    torch.testing.assert_close(torch.cat([o1, o2], 1), o, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(S2, S, rtol=1e-10, atol=1e-10)


def test_linearity_in_v():
    x = _inp(B=1, T=30, H=2, K=8, V=4)
    v1 = x.v.double()
    v2 = torch.randn(x.v.shape, generator=torch.Generator().manual_seed(9), dtype=D)
    a, b = 0.7, -1.3
    o1, S1 = O.recurrent_fwd(x.q, x.k, v1, x.g, x.beta)
    o2, S2 = O.recurrent_fwd(x.q, x.k, v2, x.g, x.beta)
    o3, S3 = O.recurrent_fwd(x.q, x.k, a * v1 + b * v2, x.g, x.beta)
    torch.testing.assert_close(o3, a * o1 + b * o2, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(S3, a * S1 + b * S2, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("T", [1, 5, 12])
def test_brute_force_transition_products(T):
    x = _inp(B=1, T=T, H=2, K=6, V=5, h0_std=0.4)
    o_r, S_r = O.recurrent_fwd(x.q, x.k, x.v, x.g, x.beta, 0.8, x.h0)
    o_b, S_b = O.transition_fwd(x.q, x.k, x.v, x.g, x.beta, 0.8, x.h0)
    torch.testing.assert_close(o_r, o_b, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(S_r, S_b, rtol=1e-10, atol=1e-10)


def test_step_equals_one_token():
    x = _inp(B=3, T=1, H=2, K=8, V=8, h0_std=0.1)
    o, S = O.step(x.q[:, 0], x.k[:, 0], x.v[:, 0], x.g[:, 0], x.beta[:, 0], x.h0, 0.5)
    o_r, S_r = O.recurrent_fwd(x.q, x.k, x.v, x.g, x.beta, 0.5, x.h0)
    torch.testing.assert_close(o, o_r[:, 0])
    torch.testing.assert_close(S, S_r)


@pytest.mark.parametrize("T,ckpt", [(1, 64), (9, 4), (20, 64), (33, 8)])
def test_reverse_recurrence_matches_autograd(T, ckpt):
    x = _inp(B=2, T=T, H=2, K=6, V=5, h0_std=0.3, with_do=True)
    s = 0.6
    leaves = [t.double().requires_grad_() for t in (x.q, x.k, x.v, x.g, x.beta, x.h0)]
    q, k, v, g, beta, h0 = leaves
    dhT = torch.randn(h0.shape, generator=torch.Generator().manual_seed(5), dtype=D)
    o, S = O.recurrent_fwd(q, k, v, g, beta, s, h0)
    L = (o * x.do.double()).sum() + (S * dhT).sum()
    auto = torch.autograd.grad(L, leaves)
    hand = O.recurrent_bwd(x.q, x.k, x.v, x.g, x.beta, x.do, s, x.h0, dhT, ckpt=ckpt)
    names = ["dq", "dk", "dv", "dg", "dbeta", "dh0"]
    for n, a, b in zip(names, auto, hand):
        torch.testing.assert_close(b, a, rtol=1e-10, atol=1e-10, msg=n)


def test_gradcheck_forward_fp64():
    x = _inp(B=1, T=5, H=1, K=4, V=3, h0_std=0.3)
    leaves = tuple(t.double().requires_grad_() for t in (x.q, x.k, x.v, x.g, x.beta, x.h0))
    f = lambda q, k, v, g, b, h: O.chunk_fwd(q, k, v, g, b, 0.9, h, chunk=2)
    assert torch.autograd.gradcheck(f, leaves, eps=1e-6, atol=1e-7)


def test_finite_differences_dg_dbeta():
    x = _inp(B=1, T=7, H=1, K=4, V=3, h0_std=0.3, with_do=True)
    hand = O.recurrent_bwd(x.q, x.k, x.v, x.g, x.beta, x.do, 1.0, x.h0)
    loss = lambda g, b: (O.recurrent_fwd(x.q, x.k, x.v, g, b, 1.0, x.h0)[0] * x.do.double()).sum().item()
    eps = 1e-6
    g0, b0 = x.g.double(), x.beta.double()
    for t in range(7):
        e = torch.zeros_like(g0)
        e[0, t, 0] = eps
        fd_g = (loss(g0 + e, b0) - loss(g0 - e, b0)) / (2 * eps)
        fd_b = (loss(g0, b0 + e) - loss(g0, b0 - e)) / (2 * eps)
        assert math.isclose(hand[3][0, t, 0].item(), fd_g, rel_tol=1e-6, abs_tol=1e-8)
        assert math.isclose(hand[4][0, t, 0].item(), fd_b, rel_tol=1e-6, abs_tol=1e-8)


def test_planted_mistake_is_caught():
    """A restatement that reads the output before the write must fail the T=1 closed form."""
    x = _inp(T=1, h0_std=0.5)

    def wrong(q, k, v, g, beta, s, h0):
        S = g[:, 0].double().exp()[..., None, None] * h0.double()
        o = torch.einsum("bhkv,bhk->bhv", S, s * q[:, 0].double())  # read before write
        return o

    o_ok, _ = O.recurrent_fwd(x.q, x.k, x.v, x.g, x.beta, 1.0, x.h0)
    assert not torch.allclose(wrong(x.q, x.k, x.v, x.g, x.beta, 1.0, x.h0), o_ok[:, 0], atol=1e-6)


@pytest.mark.parametrize("T,chunk", [(1, 64), (37, 16), (64, 64), (100, 32), (130, 64)])
def test_chunk_backward_equals_reverse_recurrence(T, chunk):
    x = _inp(B=2, T=T, H=2, K=8, V=6, h0_std=0.3, with_do=True)
    dhT = torch.randn(2, 2, 8, 6, generator=torch.Generator().manual_seed(11), dtype=D)
    ref = O.recurrent_bwd(x.q, x.k, x.v, x.g, x.beta, x.do, 0.7, x.h0, dhT)
    got = O.chunk_bwd(x.q, x.k, x.v, x.g, x.beta, x.do, 0.7, x.h0, dhT, chunk=chunk)
    for n, a, b in zip(["dq", "dk", "dv", "dg", "dbeta", "dh0"], got, ref):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-9, msg=n)
