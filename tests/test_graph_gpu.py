"""HIP graph capture of the kernels (torch.cuda.graph on the ROCm build): the training pair (stashing forward +
stashed backward), the short conv, the gated RMSNorm and a decode step are captured once and replayed several
times with eager work and synchronisations between replays; every replay must equal the eager result bit for
bit.  The library enqueues only kernels (no hipMemsetAsync, no host synchronisation), so capture is safe."""

import pytest
import torch

from archbench_amd import ops
from archbench_amd.synthetic import make_step_inputs
from tests.gpu_util import banner, device_inputs

pytestmark = pytest.mark.gpu


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def test_training_pair_conv_and_norm_replay():
    banner("HIP graph: training pair, conv, norm")
    _, dev = device_inputs(2, 300, 2, 128, 128, torch.bfloat16, seed=1, h0_std=0.1, with_do=True)
    xc = torch.randn(2, 300, 512, device="cuda").bfloat16()
    wc = torch.randn(512, 4, device="cuda")
    xn, gn = torch.randn(1200, 128, device="cuda").bfloat16(), torch.randn(1200, 128, device="cuda").bfloat16()
    wn = torch.rand(128, device="cuda")

    def step():
        o, hT, stash = ops.chunk_fwd_stash(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, 1.0)
        grads = ops.chunk_bwd_stashed(dev.q, dev.k, dev.v, dev.g, dev.beta, dev.h0, dev.do, None, stash, 1.0)
        y, st = ops.short_conv(xc, wc, None, None, 128)
        cg = ops.short_conv_bwd(xc, wc, None, None, y, 128)
        yn = ops.gated_rmsnorm(xn, gn, wn, 1e-5)
        ng = ops.gated_rmsnorm_bwd(xn, gn, wn, yn, 1e-5)
        return (o, hT, *grads, y, st, *cg, yn, *ng)

    eager = [t.clone() for t in step()]
    torch.cuda.synchronize()
    g, out = _capture(step)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(out, eager)):
            assert torch.equal(a, b), i
        step()  # eager work between replays
        torch.cuda.synchronize()


def test_decode_step_replay_advances_state():
    banner("HIP graph: decode step")
    q, k, v, gg, b, S = make_step_inputs(8, 4, 128, 128)
    q, k, v = (t.cuda().bfloat16() for t in (q, k, v))
    gg, b = gg.cuda(), b.cuda()
    S_graph, S_eager = S.cuda(), S.cuda()
    g, out = _capture(lambda: ops.recurrent_step(q, k, v, gg, b, S_graph, 1.0))
    S_graph.copy_(S.cuda())  # the warm-up and capture runs advanced it; start both from the same state
    for _ in range(4):
        g.replay()
        o_e = ops.recurrent_step(q, k, v, gg, b, S_eager, 1.0)
        torch.cuda.synchronize()
        assert torch.equal(out, o_e)
        assert torch.equal(S_graph, S_eager)
