"""HIP kernels (through the C ABI via the custom ops) against the CPU oracle on identical seeded inputs.

Tolerances (stated by the workload definition): fp32 runs max-abs <= 1e-4 (absolute, for the output, the final
state and every gradient; the achieved errors are printed); bf16 runs relative L2 <= 1e-2 for the output, the final
state and every gradient, against the fp64 oracle on the same (bf16-rounded) inputs.
"""

import pytest
import torch

from archbench_amd import ops
from oracle import gdn_oracle as O
from tests.gpu_util import assert_fp32_close, banner, device_inputs, max_abs, rel_l2

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
BF16_TOL = 1e-2


def _fwd_case(B, T, H, K, V, dtype, scale=1.0, h0_std=None, g_shift=4.0, seed=0):
    banner(f"chunk fwd B={B} T={T} H={H} K={K} V={V} {dtype} scale={scale} h0={h0_std}")
    host, dev = device_inputs(B, T, H, K, V, dtype, seed=seed, g_shift=g_shift, h0_std=h0_std)
    o, hT = ops.chunk_gated_delta_rule(dev.q, dev.k, dev.v, dev.g, dev.beta, scale=scale,
                                       initial_state=dev.h0, output_final_state=True)
    torch.cuda.synchronize()
    o_ref, hT_ref = O.chunk_fwd(host.q, host.k, host.v, host.g, host.beta, scale, host.h0)
    return o, hT, o_ref, hT_ref


def test_fp32_cfg0_forward():
    """Config 0: fp32 B=2 T=512 H=4 K=V=64, zero initial state; max-abs <= 1e-4."""
    o, hT, o_ref, hT_ref = _fwd_case(2, 512, 4, 64, 64, torch.float32)
    assert max_abs(o, o_ref) <= FP32_TOL
    assert max_abs(hT, hT_ref) <= FP32_TOL


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200])
def test_fp32_ragged_lengths(T):
    o, hT, o_ref, hT_ref = _fwd_case(1, T, 2, 64, 64, torch.float32, scale=0.125, h0_std=0.1)
    assert max_abs(o, o_ref) <= FP32_TOL
    assert max_abs(hT, hT_ref) <= FP32_TOL


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128), (128, 256), (64, 128)])
def test_bf16_forward_shapes(K, V):
    o, hT, o_ref, hT_ref = _fwd_case(2, 256, 3, K, V, torch.bfloat16, h0_std=0.1)
    assert rel_l2(o, o_ref) <= BF16_TOL
    assert rel_l2(hT, hT_ref) <= BF16_TOL


def test_bf16_cfg1_slice_forward():
    """Config 1 shape per head (K=V=128, H=8), T cut to 1024 so the fp64 oracle stays fast."""
    o, hT, o_ref, hT_ref = _fwd_case(2, 1024, 8, 128, 128, torch.bfloat16)
    assert rel_l2(o, o_ref) <= BF16_TOL
    assert rel_l2(hT, hT_ref) <= BF16_TOL


def _bwd_case(B, T, H, K, V, dtype, scale=1.0, h0_std=None, g_shift=4.0, seed=0, with_dhT=True):
    banner(f"chunk bwd B={B} T={T} H={H} K={K} V={V} {dtype} scale={scale} h0={h0_std}")
    host, dev = device_inputs(B, T, H, K, V, dtype, seed=seed, g_shift=g_shift, h0_std=h0_std, with_do=True)
    dhT = torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(seed + 1)) * 0.1 if with_dhT else None
    h0 = dev.h0
    got = ops.chunk_bwd(dev.q, dev.k, dev.v, dev.g, dev.beta, h0, dev.do,
                        None if dhT is None else dhT.cuda(), scale)
    torch.cuda.synchronize()
    ref = O.chunk_bwd(host.q, host.k, host.v, host.g, host.beta, host.do, scale, host.h0, dhT)
    return got, ref


NAMES = ["dq", "dk", "dv", "dg", "dbeta", "dh0"]


def test_fp32_backward_cfg0_shape():
    got, ref = _bwd_case(2, 512, 4, 64, 64, torch.float32, h0_std=0.1)
    assert_fp32_close("cfg0 bwd", NAMES, got, ref, FP32_TOL)


@pytest.mark.parametrize("T", [1, 50, 64, 130])
def test_fp32_backward_ragged(T):
    got, ref = _bwd_case(1, T, 2, 64, 64, torch.float32, scale=0.125, h0_std=0.1)
    assert_fp32_close(f"ragged bwd T={T}", NAMES, got, ref, FP32_TOL)


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128), (128, 256)])
def test_bf16_backward_shapes(K, V):
    got, ref = _bwd_case(2, 256, 2, K, V, torch.bfloat16, h0_std=0.1)
    for n, a, b in zip(NAMES, got, ref):
        assert rel_l2(a, b) <= BF16_TOL, (n, rel_l2(a, b))


def test_bf16_cfg3_like_backward():
    """Config 3 conventions (K=128, V=256, h0 ~ N(0, 0.1^2), slow decay g_shift=6), T cut to 1024."""
    got, ref = _bwd_case(1, 1024, 2, 128, 256, torch.bfloat16, h0_std=0.1, g_shift=6.0)
    for n, a, b in zip(NAMES, got, ref):
        assert rel_l2(a, b) <= BF16_TOL, (n, rel_l2(a, b))


def test_autograd_matches_backward_op():
    banner("autograd through chunk_gated_delta_rule")
    host, dev = device_inputs(1, 100, 2, 64, 64, torch.float32, h0_std=0.1, with_do=True)
    leaves = [t.clone().requires_grad_() for t in (dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0)]
    q, k, v, g, b, h0 = leaves
    o, hT = ops.chunk_gated_delta_rule(q, k, v, g, b, scale=0.3, initial_state=h0, output_final_state=True)
    dhT = torch.full_like(hT, 0.05)
    ((o * dev.do).sum() + (hT * dhT).sum()).backward()
    ref = O.chunk_bwd(host.q, host.k, host.v, host.g, host.beta, host.do, 0.3, host.h0, dhT.cpu())
    assert_fp32_close("autograd", NAMES, [leaf.grad for leaf in leaves], ref, FP32_TOL)


def test_autograd_recompute_path(monkeypatch):
    """The same gradients through the recompute path (no stash kept by the forward)."""
    monkeypatch.setenv("ARCHBENCH_AMD_GDN_STASH", "0")
    banner("autograd through chunk_gated_delta_rule, recompute path")
    host, dev = device_inputs(1, 100, 2, 64, 64, torch.float32, h0_std=0.1, with_do=True)
    leaves = [t.clone().requires_grad_() for t in (dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0)]
    q, k, v, g, b, h0 = leaves
    o, hT = ops.chunk_gated_delta_rule(q, k, v, g, b, scale=0.3, initial_state=h0, output_final_state=True)
    dhT = torch.full_like(hT, 0.05)
    ((o * dev.do).sum() + (hT * dhT).sum()).backward()
    ref = O.chunk_bwd(host.q, host.k, host.v, host.g, host.beta, host.do, 0.3, host.h0, dhT.cpu())
    assert_fp32_close("autograd", NAMES, [leaf.grad for leaf in leaves], ref, FP32_TOL)


@pytest.mark.parametrize("dtype,T,K,V", [(torch.float32, 130, 64, 64), (torch.bfloat16, 200, 128, 128),
                                         (torch.bfloat16, 64, 64, 256), (torch.bfloat16, 64, 128, 128),
                                         (torch.bfloat16, 130, 128, 128), (torch.bfloat16, 190, 64, 128)])
def test_stash_pair_equals_plain_and_recompute(dtype, T, K, V):
    """fwd_stash gives the plain forward's o and hT bit for bit, and bwd_stashed the recompute backward's
    gradients bit for bit (the stash holds exactly what the recompute sweep rebuilds); both against the oracle.
    bf16 at V <= 128 keeps every second state: one chunk (no pair), and three chunks (the last one unpaired,
    ragged at T = 190) walk the pairs' edge cases."""
    banner(f"stash pair {dtype} T={T} K={K} V={V}")
    host, dev = device_inputs(2, T, 2, K, V, dtype, h0_std=0.1, with_do=True, seed=3)
    dhT = (torch.randn(2, 2, K, V, generator=torch.Generator().manual_seed(9)) * 0.1).cuda()
    o_s, hT_s, stash = ops.chunk_fwd_stash(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, 0.5)
    o_p, hT_p = ops.chunk_fwd(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, 0.5)
    got = ops.chunk_bwd_stashed(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, dev.do, dhT, stash, 0.5)
    plain = ops.chunk_bwd(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, dev.do, dhT, 0.5)
    torch.cuda.synchronize()
    assert torch.equal(o_s, o_p) and torch.equal(hT_s, hT_p)
    for n, a, b in zip(NAMES, got, plain):
        assert torch.equal(a, b), n
    o_ref, hT_ref = O.chunk_fwd(host.q, host.k, host.v, host.g, host.beta, 0.5, host.h0)
    ref = O.chunk_bwd(host.q, host.k, host.v, host.g, host.beta, host.do, 0.5, host.h0, dhT.cpu())
    if dtype == torch.float32:
        assert_fp32_close("stash pair", ["o", "hT", *NAMES], [o_s, hT_s, *got], [o_ref, hT_ref, *ref], FP32_TOL)
    else:
        assert rel_l2(o_s, o_ref) <= BF16_TOL
        for n, a, b in zip(NAMES, got, ref):
            assert rel_l2(a, b) <= BF16_TOL, (n, rel_l2(a, b))


def test_training_pair_repeatable_bitwise():
    """Every reduction is in a fixed order (no atomics): two runs of the training pair on the same inputs give
    identical bits, at a shape with thousands of workgroups and a ragged last chunk."""
    banner("training pair repeatability B=4 T=1000 H=8 K=V=128 bf16")
    _, dev = device_inputs(4, 1000, 8, 128, 128, torch.bfloat16, h0_std=0.1, with_do=True, seed=21)
    runs = []
    for _ in range(2):
        o, hT, stash = ops.chunk_fwd_stash(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, 0.7)
        grads = ops.chunk_bwd_stashed(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, dev.do, None, stash, 0.7)
        torch.cuda.synchronize()
        runs.append((o, hT) + tuple(grads))
    for n, a, b in zip(("o", "hT", *NAMES), runs[0], runs[1]):
        assert torch.equal(a, b), n


@pytest.mark.parametrize("K,V", [(128, 128), (128, 64), (64, 256), (64, 128)])
def test_training_pair_many_chunks_per_workgroup(K, V):
    """The gradient kernel's workgroups are persistent (at most one per CU, each looping over chunks and
    prefetching the next one during the current one): with 768 chunks of which the last of every sequence is
    ragged (T = 1000), each workgroup runs several chunks, ragged ones included.  Two heads are checked against
    the fp64 oracle, every head against the plain (recompute) backward."""
    B, T, H = 4, 1000, 12
    banner(f"training pair, many chunks per workgroup B={B} T={T} H={H} K={K} V={V} bf16")
    host, dev = device_inputs(B, T, H, K, V, torch.bfloat16, seed=31, h0_std=0.1, with_do=True)
    dhT = torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(32)) * 0.1
    o, hT, stash = ops.chunk_fwd_stash(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, 0.6)
    grads = ops.chunk_bwd_stashed(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, dev.do, dhT.cuda(), stash, 0.6)
    plain = ops.chunk_bwd(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, dev.do, dhT.cuda(), 0.6)
    torch.cuda.synchronize()
    for n, a, b in zip(NAMES, grads, plain):
        assert rel_l2(a, b) <= BF16_TOL, (n, rel_l2(a, b))
    for bi, h in ((0, 0), (3, 11)):
        s = lambda x: x[bi:bi + 1, :, h:h + 1]
        ref = O.chunk_bwd(s(host.q), s(host.k), s(host.v), s(host.g), s(host.beta), s(host.do), 0.6,
                          host.h0[bi:bi + 1, h:h + 1], dhT[bi:bi + 1, h:h + 1])
        for n, got, r in zip(NAMES[:5], grads[:5], ref[:5]):
            assert rel_l2(s(got), r) <= BF16_TOL, (bi, h, n, rel_l2(s(got), r))
        assert rel_l2(grads[5][bi:bi + 1, h:h + 1], ref[5]) <= BF16_TOL, (bi, h, "dh0")


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_training_pair(seed):
    """Seeded random shapes (ragged T, one to four heads, every compiled K x V pair, random scale, with and
    without states) through the training pair against the fp64 oracle (rel-L2 <= 1e-2)."""
    rng = torch.Generator().manual_seed(1000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=rng))]
    B, T, H = pick([1, 2, 3]), int(torch.randint(1, 300, (1,), generator=rng)), pick([1, 2, 4])
    K, V = pick([(64, 64), (64, 128), (64, 256), (128, 64), (128, 128), (128, 256)])
    scale = float(torch.empty(1).uniform_(0.3, 1.2, generator=rng))
    states = bool(seed % 2)
    banner(f"random training pair seed={seed} B={B} T={T} H={H} K={K} V={V} scale={scale:.3f} states={states}")
    host, dev = device_inputs(B, T, H, K, V, torch.bfloat16, seed=seed, h0_std=0.1 if states else None,
                              with_do=True)
    dhT = (torch.randn(B, H, K, V, generator=rng) * 0.1).cuda() if states else None
    o, hT, stash = ops.chunk_fwd_stash(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, scale)
    got = ops.chunk_bwd_stashed(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, dev.do, dhT, stash, scale)
    torch.cuda.synchronize()
    o_ref, hT_ref = O.chunk_fwd(host.q, host.k, host.v, host.g, host.beta, scale, host.h0)
    ref = O.chunk_bwd(host.q, host.k, host.v, host.g, host.beta, host.do, scale, host.h0,
                      None if dhT is None else dhT.cpu())
    assert rel_l2(o, o_ref) <= BF16_TOL
    assert rel_l2(hT, hT_ref) <= BF16_TOL
    for n, a, b in zip(NAMES, got, ref):
        if b is not None:
            assert rel_l2(a, b) <= BF16_TOL, (n, rel_l2(a, b))


def test_state_passing_on_gpu():
    banner("state passing")
    host, dev = device_inputs(2, 300, 2, 128, 128, torch.bfloat16, h0_std=0.1)
    o, hT = ops.chunk_gated_delta_rule(dev.q, dev.k, dev.v, dev.g, dev.beta, 1.0, dev.h0, True)
    t1 = 130
    sl = lambda x, a, b: x[:, a:b]
    o1, h1 = ops.chunk_gated_delta_rule(sl(dev.q, 0, t1), sl(dev.k, 0, t1), sl(dev.v, 0, t1), sl(dev.g, 0, t1),
                                        sl(dev.beta, 0, t1), 1.0, dev.h0, True)
    o2, h2 = ops.chunk_gated_delta_rule(sl(dev.q, t1, 300), sl(dev.k, t1, 300), sl(dev.v, t1, 300),
                                        sl(dev.g, t1, 300), sl(dev.beta, t1, 300), 1.0, h1, True)
    assert rel_l2(torch.cat([o1, o2], 1), o) <= BF16_TOL
    assert rel_l2(h2, hT) <= BF16_TOL


def test_strong_decay_is_finite():
    banner("strong decay")
    host, dev = device_inputs(1, 256, 2, 64, 64, torch.float32, g_shift=-6.0)
    g = dev.g * 20
    o, hT = ops.chunk_gated_delta_rule(dev.q, dev.k, dev.v, g, dev.beta, 1.0, None, True)
    o_ref, hT_ref = O.chunk_fwd(host.q, host.k, host.v, host.g * 20, host.beta, 1.0)
    assert torch.isfinite(o).all() and torch.isfinite(hT).all()
    assert max_abs(o, o_ref) <= FP32_TOL


def test_empty_sequence():
    banner("T = 0")
    dev = device_inputs(2, 1, 2, 64, 64, torch.bfloat16, h0_std=0.1)[1]
    z = lambda x: x[:, :0]
    o, hT = ops.chunk_gated_delta_rule(z(dev.q), z(dev.k), z(dev.v), z(dev.g), z(dev.beta), 1.0, dev.h0, True)
    assert o.shape == (2, 0, 2, 64)
    torch.testing.assert_close(hT, dev.h0)


# ----------------------------------------------------------------------------------------------- decode step
def _step_case(B, H, K, V, dtype, scale=1.0):
    from archbench_amd.synthetic import make_step_inputs
    banner(f"decode step B={B} H={H} K={K} V={V} {dtype}")
    q, k, v, g, b, S = make_step_inputs(B, H, K, V)
    r = lambda t: t.to(dtype).float()
    o_ref, S_ref = O.step(r(q), r(k), r(v), g, b, S, scale)
    Sd = S.cuda()
    o = ops.recurrent_step(q.to("cuda", dtype), k.to("cuda", dtype), v.to("cuda", dtype), g.cuda(), b.cuda(), Sd,
                           scale)
    torch.cuda.synchronize()
    return o, Sd, o_ref, S_ref


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128), (128, 256), (64, 128)])
def test_step_fp32(K, V):
    o, S, o_ref, S_ref = _step_case(8, 4, K, V, torch.float32, 0.5)
    assert max_abs(o, o_ref) <= FP32_TOL
    assert max_abs(S, S_ref) <= FP32_TOL


def test_step_cfg4_bf16_full_shape():
    """Config 4: B=256 H=16 K=V=128, fp32 state updated in place, bf16 token."""
    o, S, o_ref, S_ref = _step_case(256, 16, 128, 128, torch.bfloat16)
    assert rel_l2(o, o_ref) <= BF16_TOL
    assert max_abs(S, S_ref) <= FP32_TOL  # state arithmetic is fp32 on rounded inputs


def test_step_matches_chunk_single_token():
    banner("step vs chunk at T=1")
    host, dev = device_inputs(4, 1, 4, 128, 128, torch.bfloat16, h0_std=0.1)
    o_c, h_c = ops.chunk_gated_delta_rule(dev.q, dev.k, dev.v, dev.g, dev.beta, 1.0, dev.h0, True)
    with torch.no_grad():
        o_s, h_s = ops.fused_recurrent_gated_delta_rule(dev.q, dev.k, dev.v, dev.g, dev.beta, 1.0, dev.h0, True)
    # the chunk path rounds the state to bf16 as an MFMA operand; the step keeps it fp32: compare at the bf16 bar
    assert rel_l2(o_s, o_c) <= BF16_TOL
    assert rel_l2(h_s, h_c) <= BF16_TOL
