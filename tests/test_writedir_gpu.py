"""ops.write_direction (gdn_writedir.hip) against the oracle's write_direction (nsgdn.py:61-75) with the
reference's shift p = k[:, t-1] (nsgdn.py:535), in fp64 on the CPU: u, and dk, dbeta, dlam through autograd.
fp32 inputs: rel-L2 <= 2e-6 for u, dk and dbeta, 2e-5 for dlam (a sum over every token).  bf16 k: the oracle runs
on the bf16-rounded k and du, and the bar is bf16 output rounding (rel-L2 <= 4e-3 for u and dk; the fp32 dbeta and
dlam <= 2e-5, 1e-4)."""

import pytest
import torch
import torch.nn.functional as F

from archbench_amd import ops
from oracle import nsgdn_oracle as NS
from tests.gpu_util import banner, rel_l2

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, K, seed, unit=True):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, T, H, K, generator=g)
    k = F.normalize(k, dim=-1) if unit else k * (1.5 / K ** 0.5)
    beta = torch.rand(B, T, H, generator=g)
    lam = F.softplus(torch.randn(H, generator=g))
    du = torch.randn(B, T, H, K, generator=g)
    return k, beta, lam, du


def _oracle(k, beta, lam, du, n):
    k, beta, lam = (t.double().requires_grad_() for t in (k, beta, lam))
    p = F.pad(k[:, :-1], (0, 0, 0, 0, 1, 0))
    u = NS.write_direction(k, p, beta, lam, n)
    u.backward(du.double())
    # at one step lam takes no part (u = beta k) and autograd leaves its gradient unset
    return u.detach(), k.grad, beta.grad, lam.grad if lam.grad is not None else torch.zeros_like(lam)


def _run(k, beta, lam, du, n, dtype):
    kd = k.to("cuda", dtype).requires_grad_()
    bd, ld = beta.cuda().requires_grad_(), lam.cuda().requires_grad_()
    u = ops.write_direction(kd, bd, ld, n)
    u.backward(du.to("cuda", dtype))
    torch.cuda.synchronize()
    return u.detach(), kd.grad, bd.grad, ld.grad


CASES = [  # B, T, H, K, n_steps, unit-norm keys
    (2, 64, 4, 64, 2, True),
    (1, 37, 3, 128, 3, True),
    (3, 1, 2, 64, 2, True),
    (2, 100, 2, 256, 4, False),
    (1, 50, 5, 128, 8, False),
    (2, 33, 2, 64, 1, True),
    (2, 40, 3, 64, 9, True),  # past the unrolled range the earlier kernel had: any n_steps runs
    (1, 33, 2, 128, 16, True),
    (2, 20, 2, 64, 9, False),
]


@pytest.mark.parametrize("B,T,H,K,n,unit", CASES)
def test_write_direction_fp32(B, T, H, K, n, unit):
    banner(f"write_direction fp32 B={B} T={T} H={H} K={K} n_steps={n} unit={unit}")
    k, beta, lam, du = _inputs(B, T, H, K, seed=B * 1000 + T + n, unit=unit)
    got = _run(k, beta, lam, du, n, torch.float32)
    ref = _oracle(k, beta, lam, du, n)
    errs = [rel_l2(a, b) for a, b in zip(got[:3], ref[:3])]
    errs.append(rel_l2(got[3], ref[3]) if n > 1 else got[3].abs().max().item())
    print(f"[rel-L2] u {errs[0]:.1e} dk {errs[1]:.1e} dbeta {errs[2]:.1e} dlam {errs[3]:.1e}", flush=True)
    assert got[0].dtype == torch.float32 and got[1].dtype == torch.float32
    assert errs[0] <= 2e-6 and errs[1] <= 2e-6 and errs[2] <= 2e-6 and errs[3] <= 2e-5


@pytest.mark.parametrize("B,T,H,K,n", [(2, 130, 4, 128, 2), (1, 65, 2, 64, 3), (2, 17, 3, 256, 2)])
def test_write_direction_bf16(B, T, H, K, n):
    banner(f"write_direction bf16 B={B} T={T} H={H} K={K} n_steps={n}")
    k, beta, lam, du = _inputs(B, T, H, K, seed=7 + T)
    kb, dub = k.bfloat16().float(), du.bfloat16().float()
    got = _run(kb, beta, lam, dub, n, torch.bfloat16)
    ref = _oracle(kb, beta, lam, dub, n)
    errs = [rel_l2(a, b) for a, b in zip(got, ref)]
    print(f"[rel-L2] u {errs[0]:.1e} dk {errs[1]:.1e} dbeta {errs[2]:.1e} dlam {errs[3]:.1e}", flush=True)
    assert got[0].dtype == torch.bfloat16 and got[1].dtype == torch.bfloat16
    assert errs[0] <= 4e-3 and errs[1] <= 4e-3 and errs[2] <= 2e-5 and errs[3] <= 1e-4


def test_write_direction_one_step_and_edges():
    banner("write_direction n_steps <= 1, empty batch, unsupported shapes")
    k, beta, lam, _ = _inputs(2, 20, 2, 64, seed=3)
    for n in (0, 1):
        u = ops.write_direction(k.cuda(), beta.cuda(), lam.cuda(), n)
        torch.testing.assert_close(u.cpu(), beta[..., None] * k, rtol=1e-6, atol=1e-7)
    e = ops.write_direction(k[:0].cuda(), beta[:0].cuda(), lam.cuda(), 2)
    assert e.shape == (0, 20, 2, 64)
    with pytest.raises(ValueError, match="K=96"):
        ops.write_direction(torch.randn(1, 4, 2, 96, device="cuda"), beta[:1, :4].cuda(), lam.cuda(), 2)
    with pytest.raises(ValueError, match="beta must be"):
        ops.write_direction(k.cuda(), beta[:, :3].cuda(), lam.cuda(), 2)
