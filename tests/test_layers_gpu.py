"""The gdn mixer layer and the op boundary on the GPU: layer output/gradients against the same layer whose
token mixing runs in the CPU oracle, prefill + decode through the cache, torch.compile(dynamic=False) and
torch.library.opcheck."""

import pytest
import torch

from archbench_amd import layers, ops
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
