"""The exact fp32 token scan (ops.nsgdn_scan: archbench::nsgdn_fwd / nsgdn_bwd, nsgdn.py:80-216) against the
oracle's token recurrence (oracle/nsgdn_oracle.py::recurrent_fwd / recurrent_bwd, fp64 on the CPU): y and every
gradient (dq, dk, du, dv, dla) at fp32 accuracy -- max-abs error <= 1e-4 for y and rel-L2 <= 1e-6 for y and each
gradient, the achieved errors printed -- over K in {64, 128}, V below, at and above one 64-row block (96: a
partial block), T around the 32-token checkpoint interval and the backward's 4-token groups (1, 31, 32, 33, 45, 100)
and over 32 checkpoint chunks (1024), B and H > 1."""

import pytest
import torch
import torch.nn.functional as F

from archbench_amd import ops
from oracle import nsgdn_oracle as NS
from tests.gpu_util import banner, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, K, V, seed):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, K, generator=g), dim=-1) * K ** -0.5
    k = F.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    u = k * torch.rand(B, T, H, 1, generator=g) + 0.1 * torch.randn(B, T, H, K, generator=g) / K ** 0.5
    v = torch.randn(B, T, H, V, generator=g)
    la = -F.softplus(torch.randn(B, T, H, generator=g)) * 0.5
    dy = torch.randn(B, T, H, V, generator=g)
    return q, k, u, v, la, dy


CASES = [  # B, T, H, K, V
    (2, 100, 2, 64, 64),
    (1, 33, 3, 128, 128),
    (2, 32, 2, 128, 256),
    (1, 31, 2, 64, 96),
    (3, 1, 2, 128, 64),
    (1, 45, 2, 64, 64),
    (1, 1024, 1, 128, 64),
]


@pytest.mark.parametrize("B,T,H,K,V", CASES)
def test_token_scan_matches_recurrence(B, T, H, K, V):
    banner(f"token scan B={B} T={T} H={H} K={K} V={V}")
    q, k, u, v, la, dy = _inputs(B, T, H, K, V, seed=B * 100 + T + K + V)
    leaves = [t.cuda().requires_grad_() for t in (q, k, u, v, la)]
    y = ops.nsgdn_scan(*leaves)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    y_ref, _ = NS.recurrent_fwd(q, k, u, v, la)
    grads_ref = NS.recurrent_bwd(q, k, u, v, la, dy)[:5]
    assert y.dtype == torch.float32
    errs = {"y": (max_abs(y, y_ref), rel_l2(y, y_ref))}
    for n, t, gr in zip(("dq", "dk", "du", "dv", "dla"), leaves, grads_ref):
        errs[n] = (max_abs(t.grad, gr), rel_l2(t.grad, gr))
    print("[max-abs, rel-L2] " + ", ".join(f"{n} {a:.1e} {r:.1e}" for n, (a, r) in errs.items()), flush=True)
    assert errs["y"][0] <= 1e-4
    for n, (a, r) in errs.items():
        assert r <= 1e-6, (n, r)


def test_token_scan_edges():
    banner("token scan: empty batch, unsupported K, shape errors")
    q, k, u, v, la, _ = _inputs(1, 8, 2, 64, 64, seed=1)
    d = [t.cuda() for t in (q, k, u, v, la)]
    e = ops.nsgdn_scan(*(t[:0] for t in d))
    assert e.shape == (0, 8, 2, 64)
    with pytest.raises(ValueError, match="K=96"):
        z = torch.zeros(1, 8, 2, 96, device="cuda")
        ops.nsgdn_scan(z, z, z, d[3], d[4])
    with pytest.raises(ValueError, match="la"):
        ops.nsgdn_scan(d[0], d[1], d[2], d[3], d[4][:, :4])


def test_gdn_op_fp32_k128_runs_exact_token_scan(monkeypatch):
    """chunk_gated_delta_rule with fp32 inputs at K = 128 (no fp32 chunk kernels there) runs the token scan with
    u = beta k: o, the final state and every gradient including dh0 (with a final-state gradient) against the gated
    delta rule oracle (fp64), rel-L2 <= 1e-6; T = 0 returns the initial state."""
    from oracle import gdn_oracle as O
    banner("gdn op fp32 K=128 V=256 through the token scan, with h0 / hT")
    monkeypatch.setattr(ops, "_TOKEN_ROUTE_WARNED", [False])
    B, T, H, K, V = 2, 70, 2, 128, 256
    g_ = torch.Generator().manual_seed(12)
    q = F.normalize(torch.randn(B, T, H, K, generator=g_), dim=-1)
    k = F.normalize(torch.randn(B, T, H, K, generator=g_), dim=-1)
    v = torch.randn(B, T, H, V, generator=g_)
    g = F.logsigmoid(torch.randn(B, T, H, generator=g_) + 3)
    beta = torch.rand(B, T, H, generator=g_)
    h0 = torch.randn(B, H, K, V, generator=g_) * 0.1
    do = torch.randn(B, T, H, V, generator=g_)
    dhT = torch.randn(B, H, K, V, generator=g_) * 0.1
    leaves = [t.cuda().requires_grad_() for t in (q, k, v, g, beta, h0)]
    with pytest.warns(UserWarning, match="token scan"):
        o, hT = ops.chunk_gated_delta_rule(*leaves[:5], scale=0.5, initial_state=leaves[5], output_final_state=True)
    torch.autograd.backward((o, hT), (do.cuda(), dhT.cuda()))
    o_ref, hT_ref = O.chunk_fwd(q, k, v, g, beta, 0.5, h0)
    grads_ref = O.chunk_bwd(q, k, v, g, beta, do, 0.5, h0, dhT)
    errs = {"o": rel_l2(o, o_ref), "hT": rel_l2(hT, hT_ref)}
    for n, t, gr in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), leaves, grads_ref):
        errs[n] = rel_l2(t.grad, gr)
    print("[rel-L2] " + ", ".join(f"{n} {e:.1e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert e <= 1e-6, (n, e)
    o0, hT0 = ops.chunk_gated_delta_rule(*(t[:, :0].detach() for t in leaves[:5]), scale=0.5,
                                         initial_state=leaves[5].detach(), output_final_state=True)
    assert o0.shape == (B, 0, H, V) and torch.equal(hT0, leaves[5].detach())


def test_token_scan_is_deterministic():
    """Row sums are added in a fixed order (no atomics): two runs of the forward and backward on the same inputs agree
    bit for bit, at a shape with several 64-row blocks, checkpoint chunks and a short last group."""
    banner("token scan determinism B=2 T=77 H=3 K=128 V=192")
    q, k, u, v, la, dy = (t.cuda() for t in _inputs(2, 77, 3, 128, 192, seed=5))
    runs = []
    for _ in range(2):
        y, r, st, _ = ops.nsgdn_token_fwd(q, k, u, v, la, None, False)
        grads = ops.nsgdn_token_bwd(q, k, u, la, r, st, dy, None, False)
        runs.append([y, r] + [g for g in grads if g is not None])
    torch.cuda.synchronize()
    for a, b in zip(*runs):
        assert torch.equal(a, b)
