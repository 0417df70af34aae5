"""CPU oracle for the gated DeltaNet (GDN) token-mixing op.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package ``archbench_amd`` imports, calls or links this
module.  It is used by ``tests/`` (as the checker), by ``__graft_entry__.smoke()`` (as the checker) and by the
``cpu_baseline`` leg of ``bench.py`` (as the reported CPU baseline, kind "port").

What it restates (reference file:line, paths relative to the archbench tree):

* ``recurrent_fwd``  -- the token recurrence of ``nsgdn_ref`` (archbench/layers/nsgdn.py:408-417) with the
  plain-GDN write vector ``u = beta * k`` (``write_direction`` with n_steps=1, nsgdn.py:67-69), extended with an
  initial/final state and a query scale.  The reference keeps S as [V, K] (nsgdn.py:410); here S is stored
  transposed, [K, V], which is the fla / decode-cache convention.  Order inside a step is decay -> read ->
  write -> output-after-write (nsgdn.py:413-416).
* ``recurrent_bwd`` -- the exact reverse-time gradient of ``_nsgdn_bwd_kernel`` (nsgdn.py:108-154), with the
  chain rule through ``u = beta * k`` (nsgdn.py:69) giving dbeta and the extra dk term, and gradients for the
  initial state (dh0) and the final state (dhT).  States are recomputed from checkpoints every ``ckpt``
  tokens, the way the reference stores one state per chunk (nsgdn.py:94, :123).
* ``chunk_fwd`` -- the chunkwise WY/UT form used by the reference's tensor-core pipeline
  (nsgdn.py:240-249 algebra; nsgdn.py:357-362 call order), for any chunk size and ragged tails.
* ``transition_fwd`` -- brute force: the explicit product of per-token transition matrices
  ``alpha_t (I - beta_t k_t k_t^T)``; an independent formulation used only to pin the others.
* ``step`` -- one recurrent decode step (the per-token body of nsgdn.py:413-416), state updated out of place.

Conventions: q, k [B, T, H, K]; v [B, T, H, V]; g (natural-log decay), beta [B, T, H]; states [B, H, K, V].
Every function computes in ``dtype`` (float64 by default) and returns tensors in that dtype.

Parity status: every function here is pinned by the closed forms, invariants and brute-force checks in
tests/test_oracle.py (T=1 closed form, beta=0 pure decay, exact delta-rule write, chunk-size invariance,
state passing, linearity in v, brute-force transition products, fp64 autograd gradcheck of recurrent_bwd).
The reference ships no tests, golden vectors or fixtures for this path, and fla (the external package that
carries archbench's ``gdn`` arithmetic) is absent, so agreement with fla's own kernels is unpinned.
"""

from __future__ import annotations

import torch


def _prep(dtype, *xs):
    # .to() keeps the autograd graph, so the fp64 gradient tests can differentiate through the forward
    return [None if x is None else x.to("cpu", dtype) for x in xs]


def recurrent_fwd(q, k, v, g, beta, scale: float = 1.0, h0=None, dtype=torch.float64):
    """Token recurrence (nsgdn.py:408-417 with u = beta*k, nsgdn.py:69).

    S~_t = exp(g_t) S_{t-1};  r_t = beta_t (v_t - S~_t^T k_t);  S_t = S~_t + k_t r_t^T;  o_t = S_t^T (scale q_t).
    Returns (o [B,T,H,V], hT [B,H,K,V]).
    """
    q, k, v, g, beta, h0 = _prep(dtype, q, k, v, g, beta, h0)
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=dtype) if h0 is None else h0.clone()
    o = torch.empty(B, T, H, V, dtype=dtype)
    for t in range(T):
        S = g[:, t].exp()[..., None, None] * S  # decay  (nsgdn.py:413)
        kt = k[:, t]
        read = torch.einsum("bhkv,bhk->bhv", S, kt)  # S^T k  (nsgdn.py:414)
        r = beta[:, t][..., None] * (v[:, t] - read)
        S = S + kt[..., :, None] * r[..., None, :]  # write  (nsgdn.py:415, u = beta k)
        o[:, t] = torch.einsum("bhkv,bhk->bhv", S, scale * q[:, t])  # output after write  (nsgdn.py:416)
    return o, S


def step(q, k, v, g, beta, state, scale: float = 1.0, dtype=torch.float64):
    """One decode step: q,k [B,H,K], v [B,H,V], g,beta [B,H], state [B,H,K,V]. Returns (o [B,H,V], new state)."""
    o, S = recurrent_fwd(q[:, None], k[:, None], v[:, None], g[:, None], beta[:, None], scale, state, dtype)
    return o[:, 0], S


def _checkpoints(k, v, g, beta, h0, ckpt):
    """States at token boundaries 0, ckpt, 2*ckpt, ... (the reference stores one state per CT tokens, nsgdn.py:94)."""
    B, T, H, K = k.shape
    S = h0.clone()
    cps = []
    for t in range(T):
        if t % ckpt == 0:
            cps.append(S.clone())
        S = g[:, t].exp()[..., None, None] * S
        r = beta[:, t][..., None] * (v[:, t] - torch.einsum("bhkv,bhk->bhv", S, k[:, t]))
        S = S + k[:, t][..., :, None] * r[..., None, :]
    return cps, S


def recurrent_bwd(q, k, v, g, beta, do, scale: float = 1.0, h0=None, dhT=None, ckpt: int = 64,
                  dtype=torch.float64):
    """Exact reverse-time gradient of ``recurrent_fwd`` (restates nsgdn.py:108-154 in [K,V] form).

    With Ĝ = dL/dS_t, stepping t = T-1 .. 0 (u = beta k, r_ref = v - S~^T k):
        dq_t  = scale * S_t do_t                          (nsgdn.py:134)
        Ĝ    += scale * q_t do_t^T                         (nsgdn.py:146)
        rho   = Ĝ^T u_t  -> dv_t = rho                     (nsgdn.py:147-148)
        du_t  = Ĝ r_ref,t                                   (nsgdn.py:149)
        Ĝ    -= k_t rho^T      (now dL/dS~_t)               (nsgdn.py:150)
        dk_t  = -S~_t rho + beta_t du_t,  dbeta_t = k_t . du_t   (nsgdn.py:151 + chain rule through u, nsgdn.py:69)
        dg_t  = <Ĝ, S~_t>_F                                 (nsgdn.py:152)
        Ĝ    <- exp(g_t) Ĝ     (dL/dS_{t-1})                (nsgdn.py:153)
    Returns (dq, dk, dv, dg, dbeta, dh0).
    """
    q, k, v, g, beta, do, h0, dhT = _prep(dtype, q, k, v, g, beta, do, h0, dhT)
    B, T, H, K = q.shape
    V = v.shape[-1]
    if h0 is None:
        h0 = torch.zeros(B, H, K, V, dtype=dtype)
    cps, _ = _checkpoints(k, v, g, beta, h0, ckpt)
    Gh = torch.zeros(B, H, K, V, dtype=dtype) if dhT is None else dhT.clone()
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    dv = torch.empty_like(v)
    dg, db = torch.empty_like(g), torch.empty_like(beta)
    for c in reversed(range(len(cps))):
        t0, t1 = c * ckpt, min(T, (c + 1) * ckpt)
        # recompute S~_t and S_t inside the checkpoint window (nsgdn.py:126-135)
        S = cps[c].clone()
        St, Sw, rr = [], [], []
        for t in range(t0, t1):
            S = g[:, t].exp()[..., None, None] * S
            St.append(S)
            r_ref = v[:, t] - torch.einsum("bhkv,bhk->bhv", S, k[:, t])
            S = S + (beta[:, t][..., None] * k[:, t])[..., :, None] * r_ref[..., None, :]
            Sw.append(S)
            rr.append(r_ref)
        for i in reversed(range(t1 - t0)):
            t = t0 + i
            kt, qt = k[:, t], scale * q[:, t]
            ut = beta[:, t][..., None] * kt
            dq[:, t] = scale * torch.einsum("bhkv,bhv->bhk", Sw[i], do[:, t])
            Gh = Gh + qt[..., :, None] * do[:, t][..., None, :]
            rho = torch.einsum("bhkv,bhk->bhv", Gh, ut)
            dv[:, t] = rho
            du = torch.einsum("bhkv,bhv->bhk", Gh, rr[i])
            Gh = Gh - kt[..., :, None] * rho[..., None, :]
            dk[:, t] = -torch.einsum("bhkv,bhv->bhk", St[i], rho) + beta[:, t][..., None] * du
            db[:, t] = (kt * du).sum(-1)
            dg[:, t] = (Gh * St[i]).sum((-1, -2))
            Gh = g[:, t].exp()[..., None, None] * Gh
    return dq, dk, dv, dg, db, Gh


def chunk_fwd(q, k, v, g, beta, scale: float = 1.0, h0=None, chunk: int = 64, dtype=torch.float64):
    """Chunkwise WY/UT form (nsgdn.py:240-249; call order nsgdn.py:357-362), ragged tail allowed.

    Per chunk (local i, j; G = chunk-local cumsum of g (nsgdn.py:357), gamma = exp(G)):
        A_ij = beta_i (k_i.k_j) exp(G_i - G_j)  (i > j)            (L of nsgdn.py:243, column-beta form)
        Tm   = (I + A)^-1                                            (solve_tril, nsgdn.py:337)
        W    = Tm diag(beta gamma) K,  U = Tm diag(beta) V          (recompute_w_u_fwd, nsgdn.py:360)
        R    = U - W S0                                              (chunk_gated_delta_rule_fwd_h, nsgdn.py:361)
        O    = scale [diag(gamma) Q S0 + (M o Q K^T) R],  M_ij = exp(G_i - G_j) (i >= j)   (chunk_fwd_o, :362)
        S_C  = gamma_C S0 + (diag(gamma_C / gamma) K)^T R
    """
    q, k, v, g, beta, h0 = _prep(dtype, q, k, v, g, beta, h0)
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=dtype) if h0 is None else h0.clone()
    o = torch.empty(B, T, H, V, dtype=dtype)
    for t0 in range(0, T, chunk):
        t1 = min(T, t0 + chunk)
        n = t1 - t0
        # [B,H,n,*]
        qc, kc = q[:, t0:t1].transpose(1, 2), k[:, t0:t1].transpose(1, 2)
        vc = v[:, t0:t1].transpose(1, 2)
        gc, bc = g[:, t0:t1].transpose(1, 2), beta[:, t0:t1].transpose(1, 2)
        G = gc.cumsum(-1)
        Gam = (G[..., :, None] - G[..., None, :])
        low = torch.tril(torch.ones(n, n, dtype=torch.bool), -1)
        lowd = torch.tril(torch.ones(n, n, dtype=torch.bool), 0)
        E = torch.where(lowd, Gam, torch.full_like(Gam, float("-inf"))).exp()
        A = torch.where(low, bc[..., :, None] * (kc @ kc.transpose(-1, -2)) * E, torch.zeros_like(E))
        I = torch.eye(n, dtype=dtype)
        Tm = torch.linalg.solve_triangular(I + A, I.expand_as(A), upper=False, unitriangular=True)
        gam = G.exp()
        W = Tm @ ((bc * gam)[..., None] * kc)
        U = Tm @ (bc[..., None] * vc)
        R = U - W @ S
        P = E * (qc @ kc.transpose(-1, -2))
        O = scale * (gam[..., None] * (qc @ S) + P @ R)
        o[:, t0:t1] = O.transpose(1, 2)
        gC = gam[..., -1]
        decay_to_end = (G[..., -1:] - G).exp()  # gamma_C / gamma_j as one exp, never a ratio of underflowing exps
        S = gC[..., None, None] * S + (decay_to_end[..., None] * kc).transpose(-1, -2) @ R
    return o, S


def transition_fwd(q, k, v, g, beta, scale: float = 1.0, h0=None, dtype=torch.float64):
    """Brute force for tiny T, from the transition form of one step:
        S_t = M_t S_{t-1} + X_t,   M_t = exp(g_t) (I - beta_t k_t k_t^T),   X_t = beta_t k_t v_t^T,
    so  S_t = sum_{j<=t} (M_t ... M_{j+1}) X_j + (M_t ... M_0) S0.

    Every S_t is rebuilt from scratch with explicit K x K products (no r vector, no WY algebra); the cost is
    O(T^2 K^3), so only for T <= 16.
    """
    q, k, v, g, beta, h0 = _prep(dtype, q, k, v, g, beta, h0)
    B, T, H, K = q.shape
    V = v.shape[-1]
    I = torch.eye(K, dtype=dtype)
    # per-token transition  M_t = exp(g_t) (I - beta_t k_t k_t^T),  input  X_t = beta_t k_t v_t^T
    Mt = [g[:, t].exp()[..., None, None] * (I - beta[:, t][..., None, None] * k[:, t][..., :, None] * k[:, t][..., None, :])
          for t in range(T)]
    Xt = [beta[:, t][..., None, None] * k[:, t][..., :, None] * v[:, t][..., None, :] for t in range(T)]
    S0 = torch.zeros(B, H, K, V, dtype=dtype) if h0 is None else h0
    o = torch.empty(B, T, H, V, dtype=dtype)
    S = None
    for t in range(T):
        # Phi(t, j) for every j <= t, built fresh each t (brute force)
        S = torch.zeros(B, H, K, V, dtype=dtype)
        Phi = I.expand(B, H, K, K).clone()
        for j in range(t, -1, -1):
            S = S + Phi @ Xt[j]
            Phi = Phi @ Mt[j]
        S = S + Phi @ S0
        o[:, t] = torch.einsum("bhkv,bhk->bhv", S, scale * q[:, t])
    return o, (S if S is not None else S0.clone())


def _chunk_factors(qc, kc, vc, gc, bc, scale):
    """Per-chunk WY factors in [.., n, .] layout (the quantities the chunk kernels build in LDS)."""
    n = qc.shape[-2]
    dtype = qc.dtype
    G = gc.cumsum(-1)
    Gam = G[..., :, None] - G[..., None, :]
    lowd = torch.tril(torch.ones(n, n, dtype=torch.bool), 0)
    low = torch.tril(torch.ones(n, n, dtype=torch.bool), -1)
    E = torch.where(lowd, Gam, torch.full_like(Gam, float("-inf"))).exp()  # exp(G_i - G_j), i >= j
    KK = kc @ kc.transpose(-1, -2)
    A = torch.where(low, bc[..., :, None] * KK * E, torch.zeros_like(E))
    I = torch.eye(n, dtype=dtype)
    Tm = torch.linalg.solve_triangular(I + A, I.expand_as(A).contiguous(), upper=False, unitriangular=True)
    gam = G.exp()
    X = (bc * gam)[..., None] * kc
    Y = bc[..., None] * vc
    P = scale * E * (qc @ kc.transpose(-1, -2))
    dte = (G[..., -1:] - G).exp()
    return dict(G=G, E=E, KK=KK, A=A, Tm=Tm, gam=gam, X=X, Y=Y, W=Tm @ X, U=Tm @ Y, P=P, dte=dte, low=low)


def chunk_bwd(q, k, v, g, beta, do, scale: float = 1.0, h0=None, dhT=None, chunk: int = 64,
              dtype=torch.float64, return_states: bool = False):
    """Chunkwise backward (the pipeline of nsgdn.py:369-382: recompute states, reverse state-gradient sweep,
    intra-chunk gradients, WY backward (nsgdn.py:279-330), reverse chunk-local cumsum of dG (nsgdn.py:381)).

    Per chunk, with S0 the state entering it and dSC = dL/d(state leaving it):
        dR  = P^T dO + Kd dSC                               Kd = diag(exp(G_C - G)) K
        dS0 = scale (diag(gamma) Q)^T dO + gamma_C dSC - W^T dR
        dq  = scale gamma (dO S0^T) + (dP o scale E) K       dP = dO R^T (lower incl. diagonal)
        dk  = dte (R dSC^T) + (dP o scale E)^T Q + beta gamma (Tm^T dW) + (D + D^T) K
              dW = -dR S0^T,  dA = -Tm^T (dW X^T + dR Y^T) Tm^T (strict lower),  D = dA o beta_i E
        dv  = beta (Tm^T dR)
        dbeta = gamma (Tm^T dW . k) + (Tm^T dR . v) + rowsum(dA o KK o E)
        dG  = scale gamma (dO S0^T . q) - dte (R dSC^T . k) + [last] (sum dte (R dSC^T . k) + gamma_C <dSC, S0>)
              + beta gamma (Tm^T dW . k) + rowsum - colsum of (dP o P) and of (dA o A)
        dg  = reverse chunk-local cumsum of dG
    Returns (dq, dk, dv, dg, dbeta, dh0) and, with return_states, also the per-chunk entering states h,
    the per-chunk dSC, R and dR (chunk-major lists) for debugging kernel intermediates.
    """
    q, k, v, g, beta, do, h0, dhT = _prep(dtype, q, k, v, g, beta, do, h0, dhT)
    B, T, H, K = q.shape
    V = v.shape[-1]
    S = torch.zeros(B, H, K, V, dtype=dtype) if h0 is None else h0.clone()
    tr = lambda x: x.transpose(1, 2)  # [B,n,H,*] -> [B,H,n,*]
    chunks = []
    for t0 in range(0, T, chunk):
        t1 = min(T, t0 + chunk)
        f = _chunk_factors(tr(q[:, t0:t1]), tr(k[:, t0:t1]), tr(v[:, t0:t1]), tr(g[:, t0:t1]), tr(beta[:, t0:t1]),
                           scale)
        R = f["U"] - f["W"] @ S
        chunks.append((t0, t1, f, S, R))
        kc = tr(k[:, t0:t1])
        S = f["gam"][..., -1, None, None] * S + (f["dte"][..., None] * kc).transpose(-1, -2) @ R
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    dv = torch.empty_like(v)
    dg, db = torch.empty_like(g), torch.empty_like(beta)
    dS = torch.zeros(B, H, K, V, dtype=dtype) if dhT is None else dhT.clone()
    dSCs, dRs = [], []
    for (t0, t1, f, S0, R) in reversed(chunks):
        qc, kc, vc = tr(q[:, t0:t1]), tr(k[:, t0:t1]), tr(v[:, t0:t1])
        bc, dOc = tr(beta[:, t0:t1]), tr(do[:, t0:t1])
        gam, dte, Tm, W, P, E = f["gam"], f["dte"], f["Tm"], f["W"], f["P"], f["E"]
        gC = gam[..., -1]
        dSC = dS
        Kd = dte[..., None] * kc
        dR = P.transpose(-1, -2) @ dOc + Kd @ dSC
        dS = scale * (gam[..., None] * qc).transpose(-1, -2) @ dOc + gC[..., None, None] * dSC \
            - W.transpose(-1, -2) @ dR
        dSCs.append(dSC)
        dRs.append(dR)
        dQg = dOc @ S0.transpose(-1, -2)
        dP = torch.tril(dOc @ R.transpose(-1, -2))
        dKd = R @ dSC.transpose(-1, -2)
        dW = -dR @ S0.transpose(-1, -2)
        dTm = dW @ f["X"].transpose(-1, -2) + dR @ f["Y"].transpose(-1, -2)
        dX = Tm.transpose(-1, -2) @ dW
        dY = Tm.transpose(-1, -2) @ dR
        dA = -(Tm.transpose(-1, -2) @ dTm @ Tm.transpose(-1, -2))
        dA = torch.where(f["low"], dA, torch.zeros_like(dA))
        D_ = dA * bc[..., :, None] * E
        dPm = dP * scale * E
        dqc = scale * gam[..., None] * dQg + dPm @ kc
        dkc = dte[..., None] * dKd + dPm.transpose(-1, -2) @ qc + (bc * gam)[..., None] * dX \
            + D_ @ kc + D_.transpose(-1, -2) @ kc
        dvc = bc[..., None] * dY
        dX_k = (dX * kc).sum(-1)
        dbc = gam * dX_k + (dY * vc).sum(-1) + (dA * f["KK"] * E).sum(-1)
        dKd_k = dte * (dKd * kc).sum(-1)
        dPP = dP * P
        dAA = dA * f["A"]
        dG = scale * gam * (dQg * qc).sum(-1) - dKd_k + bc * gam * dX_k \
            + dPP.sum(-1) - dPP.sum(-2) + dAA.sum(-1) - dAA.sum(-2)
        dG[..., -1] += dKd_k.sum(-1) + gC * (dSC * S0).sum((-1, -2))
        dgc = dG.flip(-1).cumsum(-1).flip(-1)
        dq[:, t0:t1], dk[:, t0:t1], dv[:, t0:t1] = tr(dqc), tr(dkc), tr(dvc)
        dg[:, t0:t1], db[:, t0:t1] = tr(dgc), tr(dbc)
    out = (dq, dk, dv, dg, db, dS)
    if return_states:
        return out, dict(h=[c[3] for c in chunks], R=[c[4] for c in chunks], dSC=dSCs[::-1], dR=dRs[::-1])
    return out
