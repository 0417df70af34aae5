"""The gdn mixer layer and the op boundary on the GPU: layer output/gradients against the same layer whose
token mixing runs in the CPU oracle and against an fp64 restatement of fla's GatedDeltaNet, prefill + decode
through the cache, torch.compile(dynamic=False) and torch.library.opcheck."""

import pytest
import torch

from archbench_amd import _lib, layers, ops
from oracle import gdn_oracle as O
from tests.gpu_util import banner, rel_l2

pytestmark = pytest.mark.gpu


def _oracle_op(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
               use_qk_l2norm_in_kernel=False, **kw):
    """The oracle (fp64, CPU, differentiable) in place of the HIP op: test infrastructure only."""
    dev, dt = q.device, q.dtype
    if use_qk_l2norm_in_kernel:
        q, k = ops._l2norm(q), ops._l2norm(k)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    h0 = None if initial_state is None else initial_state.cpu()
    o, hT = O.chunk_fwd(q.cpu(), k.cpu(), v.cpu(), g.cpu(), beta.cpu(), scale, h0)
    return o.to(dev, dt), (hT.to(dev, torch.float32) if output_final_state else None)


def _layer(seed=0):
    torch.manual_seed(seed)
    m = layers.build_mixer("gdn", 256, 0, 2, num_heads=2, head_dim=64, expand_v=2.0).cuda()
    for p in m.parameters():  # the model's init keeps fla-layer params; give the projections a usable scale
        if p.dim() == 2:
            torch.nn.init.normal_(p, std=0.05)
    return m


def test_layer_matches_oracle_forward_backward(monkeypatch):
    banner("layer fwd/bwd vs oracle-backed layer")
    m = _layer()
    x = torch.randn(2, 100, 256, device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    x1 = x.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y1 = m(x1)
    y1.float().square().sum().backward()
    g1 = {n: p.grad.clone() for n, p in m.named_parameters()}
    m.zero_grad()
    monkeypatch.setattr("archbench_amd.layers.gdn.ops.chunk_gated_delta_rule", _oracle_op)
    x2 = x.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y2 = m(x2)
    y2.float().square().sum().backward()
    assert rel_l2(y1.float(), y2.float()) <= 1e-2
    assert rel_l2(x1.grad, x2.grad) <= 1e-2
    for n, p in m.named_parameters():
        assert rel_l2(g1[n], p.grad) <= 2e-2, n


GDN_YAML = dict(head_dim=128, expand_v=2.0, use_gate=True, use_short_conv=True, conv_size=4)  # arch/gdn.yaml


# archbench's model sizes (configs/{40m,65m,130m,380m}/gdn.yaml and nsgdn.yaml): d_model and num_heads; every size
# uses head_dim 128 and expand_v 2 (configs/arch/gdn.yaml, nsgdn.yaml), so K = 128 and V = 256
REFERENCE_SIZES = [("40m", 384, 3), ("65m", 512, 4), ("130m", 768, 6), ("380m", 1024, 8)]


@pytest.mark.parametrize("size,d_model,heads", REFERENCE_SIZES)
def test_reference_config_under_autocast(monkeypatch, size, d_model, heads):
    """The mixer exactly as archbench's model builds it for configs/<size>/gdn.yaml (head_dim 128, expand_v 2 ->
    K = 128, V = 256), fed fp32 hidden states under bf16 autocast as Block.forward does under the trainer
    (model.py:44-45, trainer.py:66): the op must run its bf16 kernels, and output, input gradient and every weight
    matrix's gradient must match the same layer with the token mixing in the fp64 oracle within rel-L2 1e-2 (the
    per-head vectors A_log and dt_bias within 3e-2)."""
    banner(f"layer at configs/{size}/gdn.yaml (d_model {d_model}, {heads} heads) under bf16 autocast vs "
           "oracle-backed layer")
    torch.manual_seed(5)
    m = layers.build_mixer("gdn", d_model, 0, 10, num_heads=heads, **GDN_YAML).cuda()
    for p in m.parameters():
        if p.dim() == 2:
            torch.nn.init.normal_(p, std=0.03)
    seen = []
    real = ops.chunk_gated_delta_rule

    def spy(q, k, v, *a, **kw):
        seen.append((q.dtype, k.dtype, v.dtype, q.shape[-1], v.shape[-1]))
        return real(q, k, v, *a, **kw)

    monkeypatch.setattr("archbench_amd.layers.gdn.ops.chunk_gated_delta_rule", spy)
    x = torch.randn(2, 200, d_model, device="cuda", generator=torch.Generator("cuda").manual_seed(2))
    x1 = x.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y1 = m(x1)
    dy = torch.randn(y1.shape, device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    (y1.float() * dy).sum().backward()
    assert seen == [(torch.bfloat16, torch.bfloat16, torch.bfloat16, 128, 256)], seen
    g1 = {n: p.grad.clone() for n, p in m.named_parameters()}
    m.zero_grad()
    monkeypatch.setattr("archbench_amd.layers.gdn.ops.chunk_gated_delta_rule", _oracle_op)
    x2 = x.clone().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y2 = m(x2)
    (y2.float() * dy).sum().backward()
    errs = {"y": rel_l2(y1.float(), y2.float()), "dx": rel_l2(x1.grad, x2.grad)}
    errs.update({n: rel_l2(g1[n], p.grad) for n, p in m.named_parameters()})
    print("rel-L2 vs oracle-backed layer:", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    assert errs["y"] <= 1e-2 and errs["dx"] <= 1e-2, errs
    for n, p in m.named_parameters():
        # the per-head vectors' gradients are sums over every token that largely cancel: bf16 rounding inside the
        # op (a few 1e-3 per token) shows several times larger in their relative error
        bar = 3e-2 if n.rsplit(".", 1)[-1] in ("A_log", "dt_bias") else 1e-2
        assert errs[n] <= bar, (n, errs[n])


def test_fp32_layer_at_k128_runs_the_exact_scan(monkeypatch):
    """Without autocast the projections are fp32; the fp32 chunk kernels exist for K = 64 only, so at the reference
    config's K = 128 the op runs the exact fp32 token scan (saying so once, with the bf16 route named) and the
    layer matches its oracle-backed copy to fp32 accuracy."""
    banner("fp32 layer at K = 128 through the exact token scan")
    monkeypatch.setattr(ops, "_TOKEN_ROUTE_WARNED", [False])
    torch.manual_seed(9)
    m = layers.build_mixer("gdn", 256, 0, 2, num_heads=2, **GDN_YAML).cuda()
    for p in m.parameters():
        if p.dim() == 2:
            torch.nn.init.normal_(p, std=0.05)
    x = torch.randn(2, 80, 256, device="cuda", generator=torch.Generator("cuda").manual_seed(10))
    x1 = x.clone().requires_grad_()
    with pytest.warns(UserWarning, match="bf16"):
        y1 = m(x1)
    assert y1.dtype == torch.float32
    y1.square().sum().backward()
    g1 = {n: p.grad.clone() for n, p in m.named_parameters()}
    m.zero_grad()
    monkeypatch.setattr("archbench_amd.layers.gdn.ops.chunk_gated_delta_rule", _oracle_op)
    x2 = x.clone().requires_grad_()
    y2 = m(x2)
    y2.square().sum().backward()
    errs = {"y": rel_l2(y1, y2), "dx": rel_l2(x1.grad, x2.grad)}
    errs.update({n: rel_l2(g1[n], p.grad) for n, p in m.named_parameters()})
    print("rel-L2 vs oracle-backed layer:", {n: f"{e:.1e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= 1e-5, (n, e)


def test_prefill_then_decode_matches_full_sequence():
    banner("prefill + decode cache")
    m = _layer(3).eval()
    x = torch.randn(2, 65, 256, device="cuda")
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        full, _, _ = m.layer(x)
        cache = {}
        pre, _, cache = m.layer(x[:, :64], use_cache=True, past_key_values=cache)
        outs = [pre]
        step, _, cache = m.layer(x[:, 64:65], use_cache=True, past_key_values=cache)
        outs.append(step)
    assert rel_l2(torch.cat(outs, 1).float(), full.float()) <= 1e-2


def test_torch_compile_static():
    banner("torch.compile(dynamic=False)")
    q = torch.nn.functional.normalize(torch.randn(1, 128, 2, 64, device="cuda"), dim=-1).bfloat16()
    v = torch.randn(1, 128, 2, 64, device="cuda").bfloat16()
    g = torch.nn.functional.logsigmoid(torch.randn(1, 128, 2, device="cuda") + 4)
    b = torch.rand(1, 128, 2, device="cuda")

    def f(q, k, v, g, b):
        o, _ = ops.chunk_gated_delta_rule(q, k, v, g, b, scale=1.0)
        return o.float().sum(-1)

    eager = f(q, q, v, g, b)
    compiled = torch.compile(f, dynamic=False, fullgraph=True)(q, q, v, g, b)
    torch.testing.assert_close(compiled, eager)


def test_opcheck():
    banner("opcheck")
    torch.manual_seed(0)
    q = torch.nn.functional.normalize(torch.randn(1, 70, 2, 64, device="cuda"), dim=-1)
    v = torch.randn(1, 70, 2, 64, device="cuda")
    g = torch.nn.functional.logsigmoid(torch.randn(1, 70, 2, device="cuda") + 4)
    b = torch.rand(1, 70, 2, device="cuda")
    h0 = torch.randn(1, 2, 64, 64, device="cuda") * 0.1
    args = (q.requires_grad_(), q.detach().clone().requires_grad_(), v.requires_grad_(), g.requires_grad_(),
            b.requires_grad_(), h0.requires_grad_(), 0.5)
    torch.library.opcheck(torch.ops.archbench_amd.gdn_chunk_fwd.default, args,
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
    # the ops added around the chunk op: write direction, fp32 token scan, mixer input stage
    utils = ("test_schema", "test_faketensor", "test_autograd_registration")
    k = torch.nn.functional.normalize(torch.randn(1, 70, 2, 64, device="cuda"), dim=-1).requires_grad_()
    beta, lam = torch.rand(1, 70, 2, device="cuda").requires_grad_(), torch.rand(2, device="cuda").requires_grad_()
    torch.library.opcheck(torch.ops.archbench_amd.write_direction.default, (k, beta, lam, 2), test_utils=utils)
    la = (-torch.rand(1, 70, 2, device="cuda")).requires_grad_()
    qs = [torch.randn(1, 70, 2, 64, device="cuda").requires_grad_() for _ in range(3)]
    h0t = (torch.randn(1, 2, 64, 64, device="cuda") * 0.1).requires_grad_()
    for h0a, fin in ((None, False), (h0t, True)):
        torch.library.opcheck(torch.ops.archbench_amd.nsgdn_token_fwd.default,
                              (*qs, v.detach().requires_grad_(), la, h0a, fin), test_utils=utils)
    y = torch.randn(1, 70, 512, device="cuda", dtype=torch.bfloat16).requires_grad_()
    w = (torch.randn(512, 4, device="cuda") * 0.5).requires_grad_()
    torch.library.opcheck(torch.ops.archbench_amd.mixer_input_stage.default, (y, w, 128, 256, 64), test_utils=utils)


def test_decode_advances_cache_state_in_place(monkeypatch):
    """A cached decode step advances the cache's own fp32 state tensor (same storage, no copy of the state) and
    equals the oracle's step from the state before it."""
    banner("decode step in place on the cache state")
    m = _layer(4).eval()
    x = torch.randn(2, 65, 256, device="cuda", generator=torch.Generator("cuda").manual_seed(6))
    seen = []
    real = ops.fused_recurrent_gated_delta_rule

    def spy(q, k, v, g, beta, **kw):
        seen.append((q.detach().float().cpu(), k.detach().float().cpu(), v.detach().float().cpu(), g.cpu(),
                     beta.cpu(), kw["initial_state"].clone().cpu()))
        return real(q, k, v, g, beta, **kw)

    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        cache = {}
        _, _, cache = m.layer(x[:, :64], use_cache=True, past_key_values=cache)
        S = cache[0]["recurrent_state"]
        ptr = S.data_ptr()
        monkeypatch.setattr("archbench_amd.layers.gdn.ops.fused_recurrent_gated_delta_rule", spy)
        _, _, cache = m.layer(x[:, 64:65], use_cache=True, past_key_values=cache)
    S1 = cache[0]["recurrent_state"]
    assert S1 is S and S1.data_ptr() == ptr
    q, k, v, g, beta, S0 = seen[0]
    o_ref, S_ref = O.step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0], S0, 64 ** -0.5)
    assert rel_l2(S1, S_ref) <= 1e-5


@pytest.mark.parametrize("K,V", [(64, 256), (128, 64)])
def test_decode_shapes_without_step_kernel(K, V):
    """Decode at (K, V) pairs the step kernel is not compiled for runs through the chunk kernels (which cover
    them), in place when asked, and agrees with the oracle step."""
    banner(f"decode without a step kernel K={K} V={V}")
    assert not _lib.supported("step", K, V, torch.bfloat16) and _lib.supported("chunk", K, V, torch.bfloat16)
    B, H = 3, 2
    gen = torch.Generator().manual_seed(7)
    q = torch.nn.functional.normalize(torch.randn(B, 1, H, K, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, 1, H, K, generator=gen), dim=-1)
    v = torch.randn(B, 1, H, V, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(B, 1, H, generator=gen) + 4)
    b = torch.sigmoid(torch.randn(B, 1, H, generator=gen))
    S0 = torch.randn(B, H, K, V, generator=gen) * 0.1
    r = lambda t: t.to(torch.bfloat16).float()
    o_ref, S_ref = O.step(r(q[:, 0]), r(k[:, 0]), r(v[:, 0]), g[:, 0], b[:, 0], S0, 0.5)
    S = S0.cuda()
    with torch.no_grad():
        o, S1 = ops.fused_recurrent_gated_delta_rule(*(t.cuda().to(torch.bfloat16) for t in (q, k, v)), g.cuda(),
                                                     b.cuda(), scale=0.5, initial_state=S,
                                                     output_final_state=True, inplace_final_state=True)
    assert S1 is S
    assert rel_l2(o[:, 0], o_ref) <= 1e-2 and rel_l2(S, S_ref) <= 1e-2


def test_layer_under_torch_compile():
    """The mixer compiled as the reference trainer compiles the model (torch.compile(dynamic=False), bf16
    autocast): forward and backward match eager, through the custom ops' fake implementations."""
    banner("layer under torch.compile(dynamic=False)")
    m = _layer()
    x = torch.randn(2, 128, 256, device="cuda", generator=torch.Generator("cuda").manual_seed(3))

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


@pytest.mark.parametrize("N,K", [(8, 512), (512, 1024), (3072, 512), (24, 40)])
def test_split_weight_gradient(N, K):
    """The layer's weight gradient split over the tokens equals dy^T x to fp32 accumulation (both operand orders,
    and the single-product fallback for short inputs), and the layer's linear backward returns it in the
    weight's dtype."""
    from archbench_amd.layers.gdn import _linear, _weight_grad
    banner(f"split weight gradient N={N} K={K}")
    M = 16384 if N != 24 else 1000
    gen = torch.Generator("cuda").manual_seed(7)
    dy = torch.randn(M, N, device="cuda", generator=gen).to(torch.bfloat16)
    x = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16)
    ref = dy.double().t() @ x.double()
    got = _weight_grad(dy, x)
    assert got.dtype == torch.float32 and got.shape == (N, K)
    assert rel_l2(got.double(), ref) <= 1e-5
    w = torch.randn(N, K, device="cuda", generator=gen).requires_grad_()
    xa = x.clone().requires_grad_()
    y = _linear(xa, w)
    assert torch.equal(y, torch.nn.functional.linear(x, w.to(torch.bfloat16)))
    y.backward(dy)
    assert w.grad.dtype == torch.float32 and rel_l2(w.grad.double(), ref) <= 1e-5
    assert torch.equal(xa.grad, dy @ w.detach().to(torch.bfloat16))


def test_grouped_linear_groups_and_gradients():
    """The layers' grouped projection: one output per row group of one weight (each equal to F.linear against
    those rows), the input gradient summed over the groups inside their GEMMs, each group's weight gradient in its
    rows and zero in rows no group covers (the padding rows of nsgdn's in_proj)."""
    from archbench_amd.layers.gdn import _grouped_linear
    banner("grouped linear: three groups and padding rows")
    M, K = 16384, 512
    bounds = (0, 2048, 3072, 3080)
    gen = torch.Generator("cuda").manual_seed(11)
    x = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16).requires_grad_()
    w = (torch.randn(3088, K, device="cuda", generator=gen) * 0.05).requires_grad_()
    outs = _grouped_linear(x, w, bounds)
    wb = w.detach().to(torch.bfloat16)
    dys = []
    for (r0, r1), y in zip(zip(bounds[:-1], bounds[1:]), outs):
        assert y.is_contiguous() and torch.equal(y, torch.nn.functional.linear(x.detach(), wb[r0:r1]))
        dys.append(torch.randn(y.shape, device="cuda", generator=gen).to(torch.bfloat16))
    torch.autograd.backward(outs, dys)
    dx_ref = sum(dy.double() @ wb[r0:r1].double() for dy, r0, r1 in zip(dys, bounds[:-1], bounds[1:]))
    assert x.grad.dtype == torch.bfloat16 and rel_l2(x.grad.double(), dx_ref) <= 5e-3
    for dy, r0, r1 in zip(dys, bounds[:-1], bounds[1:]):
        ref = dy.double().t() @ x.detach().double()
        assert rel_l2(w.grad[r0:r1].double(), ref) <= 1e-5, (r0, r1)
    assert torch.count_nonzero(w.grad[bounds[-1]:]) == 0


def _gdn_restatement(P, x, H, DK, DV, use_gate, eps, bf16_op):
    """fla's GatedDeltaNet.forward as the gdn arch builds it (separate q/k/v/a/b/g linears; causal depthwise conv
    + SiLU; q, k L2-normalised per head; g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b); the chunk rule
    at scale DK^-1/2; RMSNorm(o) * silu(gate); o_proj), restated on the CPU in fp64 from the module's parameters
    P.  With bf16_op the op's inputs and output are rounded to bf16, where the layer under autocast hands them
    over."""
    F = torch.nn.functional
    B, T, _ = x.shape
    lin = lambda n: x @ P[n + ".weight"].T
    bf = (lambda t: t.to(torch.bfloat16).to(torch.float64)) if bf16_op else (lambda t: t)

    def conv(y, n):
        w = P[n + ".weight"]
        z = F.conv1d(y.transpose(1, 2), w, padding=w.shape[-1] - 1, groups=y.shape[-1])[..., :T]
        return F.silu(z.transpose(1, 2))
    q = F.normalize(conv(lin("layer.q_proj"), "layer.q_conv1d").reshape(B, T, H, DK), dim=-1)
    k = F.normalize(conv(lin("layer.k_proj"), "layer.k_conv1d").reshape(B, T, H, DK), dim=-1)
    v = conv(lin("layer.v_proj"), "layer.v_conv1d").reshape(B, T, H, DV)
    g = -P["layer.A_log"].exp() * F.softplus(lin("layer.a_proj") + P["layer.dt_bias"])
    beta = torch.sigmoid(lin("layer.b_proj"))
    o, _ = O.chunk_fwd(bf(q), bf(k), bf(v), g, beta, DK ** -0.5)
    o = F.rms_norm(bf(o), (DV,), P["layer.o_norm.weight"], eps)
    if use_gate:
        o = o * F.silu(lin("layer.g_proj").reshape(B, T, H, DV))
    return o.reshape(B, T, -1) @ P["layer.o_proj.weight"].T


@pytest.mark.parametrize("use_gate", [True, False])
def test_gdn_layer_matches_restatement(use_gate):
    """The whole gdn mixer under bf16 autocast (grouped projection GEMMs, the fused input stage, gates, the chunk
    kernels, gated RMSNorm) against an fp64 CPU restatement of fla's GatedDeltaNet with the same parameters:
    output and input gradient within rel-L2 1e-2, every parameter gradient within 3e-2 plus four times the
    restatement's own movement when only the op's bf16 rounding point changes (the per-head vectors' gradients
    are cancelling sums over every token)."""
    banner(f"gdn layer vs fp64 restatement, use_gate={use_gate}")
    torch.manual_seed(7)
    H, DK, DV, d = 2, 64, 128, 192
    m = layers.build_mixer("gdn", d, 0, 2, num_heads=H, head_dim=DK, expand_v=2.0, use_gate=use_gate).cuda()
    for p in m.parameters():
        if p.dim() == 2:
            torch.nn.init.normal_(p, std=0.05)
    x = torch.randn(2, 100, d, generator=torch.Generator().manual_seed(8))
    xd = x.cuda().requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = m(xd)
    dy = torch.randn(*y.shape, generator=torch.Generator().manual_seed(9))
    y.float().backward(dy.cuda())
    refs = []
    for bf16_op in (True, False):
        P = {n: p.detach().cpu().double().requires_grad_() for n, p in m.named_parameters()}
        xr = x.double().requires_grad_()
        yr = _gdn_restatement(P, xr, H, DK, DV, use_gate, m.layer.o_norm.eps, bf16_op)
        yr.backward(dy.double())
        refs.append((yr.detach(), xr.grad, {n: t.grad for n, t in P.items()}))
    (yr, dxr, gr), (_, _, gr_exact) = refs
    errs = {"y": rel_l2(y.float(), yr), "dx": rel_l2(xd.grad, dxr)}
    print("rel-L2 vs restatement:", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    assert errs["y"] <= 1e-2 and errs["dx"] <= 1e-2, errs
    for n, p in m.named_parameters():
        noise = rel_l2(gr_exact[n], gr[n])
        assert rel_l2(p.grad, gr[n]) <= 3e-2 + 4 * noise, (n, rel_l2(p.grad, gr[n]), noise)
