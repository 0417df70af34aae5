"""CPU oracle for the chunk op with separate read and write vectors (archbench's n-step GDN family).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package ``archbench_amd`` imports, calls or links this
module; ``tests/`` use it as the checker.

What it restates (reference file:line, paths relative to the archbench tree):

* ``recurrent_fwd`` -- ``nsgdn_ref`` (archbench/layers/nsgdn.py:408-417): per token S~ = e^la S, r = v - S~^T k,
  S = S~ + u r^T, y = S^T q, extended with a query scale and initial / final states.  The reference keeps S as
  [V, K]; here S is [K, V] (the chunk op's convention).
* ``chunk_fwd`` -- the chunked form of the same recurrence (nsgdn.py:240-249): within a chunk
  L_ij = (k_i . u_j) gamma_i / gamma_j (i > j), T = (I + L)^-1, R = T (V - diag(gamma) K S0),
  S_C = gamma_C S0 + sum_j (gamma_C / gamma_j) u_j r_j^T, y_t = gamma_t S0^T q_t + sum_{j<=t} (gamma_t / gamma_j)
  (u_j . q_t) r_j -- written with exponent differences so it cannot overflow.
* ``recurrent_bwd`` -- gradients of ``recurrent_fwd`` by autograd in the oracle's dtype (the reference's backward
  is _nsgdn_bwd_kernel / archbench::nsgdn_chunk_bwd, nsgdn.py:108-154, :369-382).
* ``write_direction`` -- nsgdn.py:61-75: u_1 = beta k, then n-1 steps u <- u - lam beta (p . u) p_perp with
  p_perp = p - (p . k) k.

Parity status: pinned in tests/test_nsgdn_oracle.py: with u = beta k every function reduces to the gated delta
rule oracle (oracle/gdn_oracle.py, itself pinned); chunk form = token recurrence for several chunk sizes and
ragged T; brute-force products of the per-token affine maps S -> e^la (I - u k^T)^T ... ; the T = 1 closed form;
fp64 gradcheck; write_direction's k . u = beta invariant for unit k.
"""

from __future__ import annotations

import torch


def _to(dtype, *xs):
    return [None if x is None else x.to("cpu", dtype) for x in xs]


def recurrent_fwd(q, k, u, v, la, scale: float = 1.0, h0=None, dtype=torch.float64):
    """(y [B,T,H,V], hT [B,H,K,V])."""
    q, k, u, v, la, h0 = _to(dtype, q, k, u, v, la, h0)
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=dtype) if h0 is None else h0.clone()
    ys = []
    for t in range(T):
        S = la[:, t].exp()[..., None, None] * S  # nsgdn.py:413
        r = v[:, t] - torch.einsum("bhkv,bhk->bhv", S, k[:, t])  # :414 (read with k)
        S = S + u[:, t][..., :, None] * r[..., None, :]  # :415 (write with u)
        ys.append(torch.einsum("bhkv,bhk->bhv", S, scale * q[:, t]))  # :416 (output after the write)
    return torch.stack(ys, 1), S


def chunk_fwd(q, k, u, v, la, scale: float = 1.0, h0=None, chunk: int = 64, dtype=torch.float64):
    q, k, u, v, la, h0 = _to(dtype, q, k, u, v, la, h0)
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=dtype) if h0 is None else h0.clone()
    ys = []
    for t0 in range(0, T, chunk):
        t1 = min(T, t0 + chunk)
        n = t1 - t0
        qc, kc, uc, vc = (x[:, t0:t1].transpose(1, 2) for x in (q, k, u, v))  # [B,H,n,*]
        G = la[:, t0:t1].transpose(1, 2).cumsum(-1)  # [B,H,n]
        D = G[..., :, None] - G[..., None, :]  # G_i - G_j
        strict = torch.tril(torch.ones(n, n, dtype=torch.bool), -1)
        incl = torch.tril(torch.ones(n, n, dtype=torch.bool))
        E_s = torch.where(strict, D.clamp(max=0).exp(), torch.zeros((), dtype=dtype))
        E_i = torch.where(incl, D.clamp(max=0).exp(), torch.zeros((), dtype=dtype))
        L = (kc @ uc.transpose(-1, -2)) * E_s
        Tm = torch.linalg.inv(torch.eye(n, dtype=dtype) + L)
        gam = G.exp()
        R = Tm @ (vc - gam[..., None] * (kc @ S))
        y = scale * gam[..., None] * (qc @ S) + ((scale * qc @ uc.transpose(-1, -2)) * E_i) @ R
        lam = (G[..., -1:] - G).exp()  # gamma_C / gamma_j
        S = gam[..., -1, None, None] * S + uc.transpose(-1, -2) @ (lam[..., None] * R)
        ys.append(y.transpose(1, 2))
    return torch.cat(ys, 1), S


def recurrent_bwd(q, k, u, v, la, dy, scale: float = 1.0, h0=None, dhT=None, dtype=torch.float64):
    """(dq, dk, du, dv, dla, dh0 | None) of sum(y * dy) + sum(hT * dhT)."""
    leaves = [None if x is None else x.detach().to("cpu", dtype).requires_grad_() for x in (q, k, u, v, la, h0)]
    y, hT = recurrent_fwd(*leaves[:5], scale=scale, h0=leaves[5], dtype=dtype)
    loss = (y * dy.to("cpu", dtype)).sum()
    if dhT is not None:
        loss = loss + (hT * dhT.to("cpu", dtype)).sum()
    loss.backward()
    return tuple(None if x is None else x.grad for x in leaves)


def write_direction(k, p, beta, lam, n_steps: int):
    """nsgdn.py:61-75.  k, p [B,T,H,K]; beta [B,T,H]; lam [H]."""
    b = beta[..., None]
    lm = lam[None, None, :, None]
    u = b * k
    if n_steps > 1:
        p_perp = p - (p * k).sum(-1, keepdim=True) * k
        for _ in range(n_steps - 1):
            u = u - lm * b * (p * u).sum(-1, keepdim=True) * p_perp
    return u
