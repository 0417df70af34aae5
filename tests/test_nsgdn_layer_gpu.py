"""The nsgdn mixer (archbench_amd/layers/nsgdn.py) on the GPU against a CPU fp64 restatement of the reference's
NStepGDN.forward (archbench/layers/nsgdn.py:518-542: conv1d + SiLU, F.normalize, softplus / sigmoid gates,
write_direction, the token scan with its bf16 boundary, RMSNorm * silu(g), o_proj) with the same parameters:
output, input gradient and every parameter gradient within rel-L2 2e-2 (3e-2 for parameter gradients)."""

import pytest
import torch
import torch.nn.functional as F

from archbench_amd import layers
from oracle import nsgdn_oracle as NS
from tests.gpu_util import banner, rel_l2

pytestmark = pytest.mark.gpu


def _reference_forward(P, x, H, DK, DV, n_steps, size, eps, bf16_scan=True):
    """NStepGDN.forward restated on CPU fp64 from the module's parameters P (name -> tensor); with bf16_scan the
    scan's inputs and output are rounded to bf16 as the reference's nsgdn_scan_chunk does (nsgdn.py:404)."""
    B, T, _ = x.shape
    qk, vd = H * DK, H * DV
    proj = x @ P["in_proj.weight"].T
    qkv, g, ab = proj[..., :2 * qk + vd], proj[..., 2 * qk + vd:2 * qk + 2 * vd], proj[..., 2 * qk + 2 * vd:]
    y = F.conv1d(qkv.transpose(1, 2), P["conv.weight"], padding=size - 1, groups=qkv.shape[-1])
    qkv = F.silu(y[..., :T].transpose(1, 2))
    q = F.normalize(qkv[..., :qk].reshape(B, T, H, DK), dim=-1) * DK ** -0.5
    k = F.normalize(qkv[..., qk:2 * qk].reshape(B, T, H, DK), dim=-1)
    v = qkv[..., 2 * qk:].reshape(B, T, H, DV)
    la = -F.softplus(ab[..., :H] + P["dt_bias"]) * P["A_log"].exp()
    beta = torch.sigmoid(ab[..., H:2 * H] + P["b_bias"])
    p = F.pad(k[:, :-1], (0, 0, 0, 0, 1, 0))
    u = NS.write_direction(k, p, beta, F.softplus(P["lam"]), n_steps)
    # the reference's scan takes and returns bf16 (nsgdn_scan_chunk, nsgdn.py:404): round there as it does
    bf = (lambda t: t.to(torch.bfloat16).to(torch.float64)) if bf16_scan else (lambda t: t)
    yk, _ = NS.chunk_fwd(bf(q), bf(k), bf(u), bf(v), la, 1.0)
    yk = bf(yk)
    yk = F.rms_norm(yk, (DV,), P["norm.weight"], eps) * F.silu(g.reshape(B, T, H, DV))
    return yk.reshape(B, T, -1) @ P["o_proj.weight"].T


def test_nsgdn_layer_matches_reference_forward_backward():
    banner("nsgdn layer vs reference forward (fp64 CPU)")
    torch.manual_seed(0)
    H, DK, DV, d = 2, 64, 128, 192
    m = layers.build_mixer("nsgdn", d, 0, 2, num_heads=H, head_dim=DK, expand_v=2.0, n_steps=2, lam=1.0).cuda()
    for n, p in m.named_parameters():
        if p.dim() == 2:
            torch.nn.init.normal_(p, std=0.05)
    x = torch.randn(2, 100, d, generator=torch.Generator().manual_seed(1))
    xd = x.cuda().requires_grad_()
    y = m(xd)
    dy = torch.randn(*y.shape, generator=torch.Generator().manual_seed(2))
    y.backward(dy.cuda())
    refs = []
    for bf16_scan in (True, False):
        P = {n: p.detach().cpu().double().requires_grad_() for n, p in m.named_parameters()}
        xr = x.double().requires_grad_()
        yr = _reference_forward(P, xr, H, DK, DV, 2, 4, 1e-5, bf16_scan)
        yr.backward(dy.double())
        refs.append((yr.detach(), xr.grad, {n: t.grad for n, t in P.items()}))
    (yr, dxr, gr), (_, _, gr_exact) = refs
    assert rel_l2(y, yr) <= 2e-2
    assert rel_l2(xd.grad, dxr) <= 2e-2
    for n, p in m.named_parameters():
        # the per-head vectors' gradients (A_log, dt_bias, b_bias, lam) are sums over every token that largely
        # cancel; the reference itself moves by rel_l2(exact, bf16) when only the bf16 rounding point changes,
        # so that sensitivity widens the bound
        noise = rel_l2(gr_exact[n], gr[n])
        assert rel_l2(p.grad, gr[n]) <= 3e-2 + 4 * noise, (n, noise)


@pytest.mark.parametrize("impl,DK", [("triton", 64), ("ref", 128)])
def test_nsgdn_layer_exact_scan_matches_in_fp32(impl, DK):
    """scan_impl "triton" / "ref" run the reference's exact fp32 token scan (ops.nsgdn_scan).  Without autocast
    every pass of the layer is fp32 (projections, conv, gates, write direction, scan, norm), so the whole mixer
    must match the fp64 restatement of NStepGDN.forward to fp32 accuracy: output and input gradient rel-L2
    <= 1e-5, every parameter gradient <= 1e-4 (the per-head vectors' are cancelling sums over every token)."""
    banner(f"nsgdn layer, scan_impl={impl}, fp32 vs fp64 restatement")
    torch.manual_seed(3)
    H, DV, d = 2, 2 * DK, 192
    m = layers.build_mixer("nsgdn", d, 0, 2, num_heads=H, head_dim=DK, expand_v=2.0, n_steps=2, lam=1.0,
                           scan_impl=impl).cuda()
    for n, p in m.named_parameters():
        if p.dim() == 2:
            torch.nn.init.normal_(p, std=0.05)
    x = torch.randn(2, 70, d, generator=torch.Generator().manual_seed(4))
    xd = x.cuda().requires_grad_()
    y = m(xd)
    assert y.dtype == torch.float32
    dy = torch.randn(*y.shape, generator=torch.Generator().manual_seed(5))
    y.backward(dy.cuda())
    P = {n: p.detach().cpu().double().requires_grad_() for n, p in m.named_parameters()}
    xr = x.double().requires_grad_()
    yr = _reference_forward(P, xr, H, DK, DV, 2, 4, m.norm.eps or 1e-5, bf16_scan=False)
    yr.backward(dy.double())
    errs = {"y": rel_l2(y, yr), "dx": rel_l2(xd.grad, xr.grad)}
    errs.update({n: rel_l2(p.grad, P[n].grad) for n, p in m.named_parameters()})
    print("rel-L2:", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    assert errs["y"] <= 1e-5 and errs["dx"] <= 1e-5, errs
    for n, _ in m.named_parameters():
        assert errs[n] <= 1e-4, (n, errs[n])


@pytest.mark.parametrize("impl", ["chunk", "triton"])
def test_nsgdn_layer_under_torch_compile(impl):
    """The n-step mixer compiled as the reference trainer compiles the model (torch.compile(dynamic=False), bf16
    autocast): forward and backward match eager through the custom ops' fake implementations (write direction,
    input stage, gates, the chunk op or the exact token scan, gated RMSNorm)."""
    banner(f"nsgdn layer under torch.compile(dynamic=False), scan_impl={impl}")
    torch.manual_seed(6)
    m = layers.build_mixer("nsgdn", 192, 0, 2, num_heads=2, head_dim=64, expand_v=2.0, n_steps=2, lam=1.0,
                           scan_impl=impl).cuda()
    for p in m.parameters():
        if p.dim() == 2:
            torch.nn.init.normal_(p, std=0.05)
    x = torch.randn(2, 96, 192, device="cuda", generator=torch.Generator("cuda").manual_seed(7))

    def run(fn):
        for p in m.parameters():
            p.grad = None
        xi = x.clone().requires_grad_()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = fn(xi)
        y.float().square().sum().backward()
        return y.float(), xi.grad, {n: p.grad.clone() for n, p in m.named_parameters()}

    y0, gx0, gp0 = run(m)
    y1, gx1, gp1 = run(torch.compile(m, dynamic=False))
    assert rel_l2(y1, y0) <= 1e-2 and rel_l2(gx1, gx0) <= 1e-2
    for n in gp0:
        assert rel_l2(gp1[n], gp0[n]) <= 2e-2, n
