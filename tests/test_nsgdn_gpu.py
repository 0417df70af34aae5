"""The chunk op with separate read / write vectors (archbench's nsgdn_chunk_fwd / _bwd) on the GPU: against the
CPU oracle (oracle/nsgdn_oracle.py, fp64 on the same bf16-rounded inputs; rel-L2 <= 1e-2 for y, hT and every
gradient), against the gated delta rule kernels at u = beta k (dk_gdn = dk + beta du, dbeta = du . k), and
through autograd."""

import pytest
import torch
import torch.nn.functional as F

from archbench_amd import ops
from oracle import nsgdn_oracle as NS
from tests.gpu_util import banner, rel_l2

pytestmark = pytest.mark.gpu
bf = torch.bfloat16


def _inputs(B, T, H, K, V, seed, h0=False, dhT=False):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    q = (F.normalize(r(B, T, H, K), dim=-1) * K ** -0.5).to(bf).float()
    k = F.normalize(r(B, T, H, K), dim=-1).to(bf).float()
    beta = torch.sigmoid(r(B, T, H))
    u = (beta[..., None] * k + 0.05 * r(B, T, H, K)).to(bf).float()
    v = r(B, T, H, V).to(bf).float()
    la = F.logsigmoid(r(B, T, H) + 4)
    dy = r(B, T, H, V).to(bf).float()
    S0 = 0.1 * r(B, H, K, V) if h0 else None
    dS = 0.1 * r(B, H, K, V) if dhT else None
    return q, k, u, v, la, dy, S0, dS


def _dev(t, dt=bf):
    return None if t is None else t.to("cuda", dt)


CASES = [(1, 64, 64, False), (63, 128, 128, True), (64, 64, 128, False), (65, 128, 128, True),
         (200, 128, 128, True), (130, 128, 256, False), (100, 64, 64, True)]


@pytest.mark.parametrize("T,K,V,states", CASES)
def test_nsgdn_matches_oracle(T, K, V, states):
    B, H = 1, 2
    banner(f"nsgdn chunk B={B} T={T} H={H} K={K} V={V} states={states}")
    q, k, u, v, la, dy, S0, dS = _inputs(B, T, H, K, V, seed=T + K, h0=states, dhT=states)
    y, hT, stash = ops.nsgdn_chunk_fwd(_dev(q), _dev(k), _dev(u), _dev(v), _dev(la, torch.float32),
                                       _dev(S0, torch.float32), 1.0)
    grads = ops.nsgdn_chunk_bwd(_dev(q), _dev(k), _dev(u), _dev(v), _dev(la, torch.float32),
                                _dev(S0, torch.float32), _dev(dy), _dev(dS, torch.float32), stash, 1.0)
    torch.cuda.synchronize()
    y_r, hT_r = NS.chunk_fwd(q, k, u, v, la, 1.0, S0)
    assert rel_l2(y, y_r) <= 1e-2
    assert rel_l2(hT, hT_r) <= 1e-2
    ref = NS.recurrent_bwd(q, k, u, v, la, dy, 1.0, S0, dS)
    for n, got, r in zip(("dq", "dk", "du", "dv", "dla", "dh0"), grads, ref):
        if r is not None:
            assert rel_l2(got, r) <= 1e-2, n


def test_nsgdn_equals_gdn_at_u_beta_k():
    """With u = beta k the n-step op is the gated delta rule: same output, and the gradients map as
    dk_gdn = dk + beta du, dbeta = du . k (the chain rule through u = beta k, nsgdn.py:69)."""
    banner("nsgdn vs gdn kernels at u = beta k")
    B, T, H, K, V = 2, 150, 2, 128, 128
    q, k, _, v, la, dy, _, _ = _inputs(B, T, H, K, V, seed=5)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=torch.Generator().manual_seed(6)))
    u = (beta[..., None] * k).to(bf).float()
    y, _, stash = ops.nsgdn_chunk_fwd(_dev(q), _dev(k), _dev(u), _dev(v), _dev(la, torch.float32), None, 1.0)
    dq, dk, du, dv, dla, _ = ops.nsgdn_chunk_bwd(_dev(q), _dev(k), _dev(u), _dev(v), _dev(la, torch.float32),
                                                 None, _dev(dy), None, stash, 1.0)
    o, _, st2 = ops.chunk_fwd_stash(_dev(q), _dev(k), _dev(v), _dev(la, torch.float32),
                                    _dev(beta, torch.float32), None, 1.0)
    g = ops.chunk_bwd_stashed(_dev(q), _dev(k), _dev(v), _dev(la, torch.float32), _dev(beta, torch.float32),
                              None, _dev(dy), None, st2, 1.0)
    torch.cuda.synchronize()
    assert rel_l2(y, o) <= 1e-2
    bet = beta.cuda()[..., None]
    assert rel_l2(dq, g[0]) <= 1e-2
    assert rel_l2(dk.float() + bet * du.float(), g[1]) <= 1e-2
    assert rel_l2(dv, g[2]) <= 1e-2
    assert rel_l2(dla, g[3]) <= 1e-2
    assert rel_l2((du.float() * k.cuda()).sum(-1), g[4]) <= 1e-2


def test_nsgdn_autograd_and_errors():
    banner("nsgdn autograd")
    B, T, H, K, V = 1, 90, 2, 64, 64
    q, k, u, v, la, dy, S0, _ = _inputs(B, T, H, K, V, seed=9, h0=True)
    leaves = [_dev(x, bf).requires_grad_() for x in (q, k, u, v)] + [_dev(la, torch.float32).requires_grad_(),
                                                                     _dev(S0, torch.float32).requires_grad_()]
    y, hT = ops.nsgdn_scan_chunk(*leaves[:5], 1.0, leaves[5], output_final_state=True)
    (y.float() * dy.cuda()).sum().backward()
    ref = NS.recurrent_bwd(q, k, u, v, la, dy, 1.0, S0)
    for n, leaf, r in zip(("dq", "dk", "du", "dv", "dla", "dh0"), leaves, ref):
        assert rel_l2(leaf.grad, r) <= 1e-2, n
    with pytest.raises(ValueError):
        ops.nsgdn_chunk_fwd(q.cuda(), k.cuda(), u.cuda(), v.cuda(), la.cuda(), None, 1.0)  # fp32 inputs
