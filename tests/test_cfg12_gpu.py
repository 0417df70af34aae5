"""Configs 1 and 2 at their full sizes on the GPU, bf16, zero initial state, seed 0 (the benchmarked shapes).

Config 2 (the headline training shape): B=8, T=4096, H=16, K=V=128 through the training pair (stashing forward +
stashed backward, the path autograd and the benchmark take).  With 8192 chunks the persistent gradient kernel
runs 32 chunks per workgroup.  Config 1: B=8, T=2048, H=8, K=V=128, forward only (gdn_chunk_fwd).

(b, h) pairs are independent, so three of them are checked against the fp64 chunk oracle at the full length
(rel-L2 <= 1e-2 for o, hT and every gradient); every head is checked by a size-independent property, state
passing: the sequence run as two segments cut at a ragged point and chained through the final state (and,
backward, through dh0 -> dhT) gives the same outputs and gradients as the one-shot run.
"""

import pytest
import torch

from archbench_amd import ops
from oracle import gdn_oracle as O
from tests.gpu_util import banner, device_inputs, rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-2
GRADS = ("dq", "dk", "dv", "dg", "dbeta")


def _pairs(B, H):
    return ((0, 0), (B // 2, H // 2 + 1), (B - 1, H - 1))


def _train(dev, h0, dhT, t0, t1):
    sl = lambda x: x[:, t0:t1].contiguous()
    o, hT, stash = ops.chunk_fwd_stash(sl(dev.q), sl(dev.k), sl(dev.v), sl(dev.g), sl(dev.beta), h0, 1.0)
    grads = ops.chunk_bwd_stashed(sl(dev.q), sl(dev.k), sl(dev.v), sl(dev.g), sl(dev.beta), h0, sl(dev.do), dhT,
                                  stash, 1.0)
    return o, hT, grads


def test_cfg2_full_size_training_pair():
    B, T, H, K, V = 8, 4096, 16, 128, 128
    banner(f"config 2 full size B={B} T={T} H={H} K={K} V={V} bf16, training pair")
    host, dev = device_inputs(B, T, H, K, V, torch.bfloat16, seed=0, with_do=True)
    o, hT, (dq, dk, dv, dg, db, dh0) = _train(dev, None, None, 0, T)
    torch.cuda.synchronize()
    for t in (o, hT, dq, dk, dv, dg, db, dh0):
        assert torch.isfinite(t).all()
    for bi, h in _pairs(B, H):
        s = lambda x: x[bi:bi + 1, :, h:h + 1]
        o_r, hT_r = O.chunk_fwd(s(host.q), s(host.k), s(host.v), s(host.g), s(host.beta), 1.0)
        ref = O.chunk_bwd(s(host.q), s(host.k), s(host.v), s(host.g), s(host.beta), s(host.do), 1.0)
        errs = {"o": rel_l2(s(o), o_r), "hT": rel_l2(hT[bi:bi + 1, h:h + 1], hT_r)}
        errs.update({n: rel_l2(s(got), r) for n, got, r in zip(GRADS, (dq, dk, dv, dg, db), ref)})
        errs["dh0"] = rel_l2(dh0[bi:bi + 1, h:h + 1], ref[5])
        print(f"[cfg2 b={bi} h={h}] rel-L2 " + ", ".join(f"{n} {e:.2e}" for n, e in errs.items()), flush=True)
        assert all(e <= TOL for e in errs.values()), (bi, h, errs)

    # all heads: two segments cut at 1000 (a ragged chunk boundary), chained through the states
    cut = 1000
    o1, h1, _ = ops.chunk_fwd_stash(*(x[:, :cut].contiguous() for x in (dev.q, dev.k, dev.v, dev.g, dev.beta)),
                                    None, 1.0)
    o2, h2, g2 = _train(dev, h1, None, cut, T)
    _, _, g1 = _train(dev, None, g2[5], 0, cut)
    errs = {"o": rel_l2(torch.cat([o1, o2], 1), o), "hT": rel_l2(h2, hT)}
    for j, (n, full) in enumerate(zip(GRADS, (dq, dk, dv, dg, db))):
        errs[n] = rel_l2(torch.cat([g1[j], g2[j]], 1), full)
    print("[cfg2 state passing, all heads] rel-L2 " + ", ".join(f"{n} {e:.2e}" for n, e in errs.items()),
          flush=True)
    assert all(e <= TOL for e in errs.values()), errs


def test_cfg1_full_size_forward():
    B, T, H, K, V = 8, 2048, 8, 128, 128
    banner(f"config 1 full size B={B} T={T} H={H} K={K} V={V} bf16, forward")
    host, dev = device_inputs(B, T, H, K, V, torch.bfloat16, seed=0)
    o, hT = ops.chunk_fwd(dev.q, dev.k, dev.v, dev.g, dev.beta, None, 1.0)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(hT).all()
    for bi, h in _pairs(B, H):
        s = lambda x: x[bi:bi + 1, :, h:h + 1]
        o_r, hT_r = O.chunk_fwd(s(host.q), s(host.k), s(host.v), s(host.g), s(host.beta), 1.0)
        e_o, e_h = rel_l2(s(o), o_r), rel_l2(hT[bi:bi + 1, h:h + 1], hT_r)
        print(f"[cfg1 b={bi} h={h}] rel-L2 o {e_o:.2e}, hT {e_h:.2e}", flush=True)
        assert e_o <= TOL and e_h <= TOL, (bi, h, e_o, e_h)
    cut = 777
    sl = lambda x, a, b: x[:, a:b].contiguous()
    o1, h1 = ops.chunk_fwd(*(sl(x, 0, cut) for x in (dev.q, dev.k, dev.v, dev.g, dev.beta)), None, 1.0)
    o2, h2 = ops.chunk_fwd(*(sl(x, cut, T) for x in (dev.q, dev.k, dev.v, dev.g, dev.beta)), h1, 1.0)
    e_o, e_h = rel_l2(torch.cat([o1, o2], 1), o), rel_l2(h2, hT)
    print(f"[cfg1 state passing, all heads] rel-L2 o {e_o:.2e}, hT {e_h:.2e}", flush=True)
    assert e_o <= TOL and e_h <= TOL
