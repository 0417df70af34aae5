"""Workload for the HBM-traffic counter runs (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE): two headline chunk
fwd+bwd training steps (B=8 T=4096 H=16 K=V=128 bf16; stashing forward + stashed backward), one step of the
recompute path (plain forward + backward with its recompute sweep), two decode steps (B=256 H=16 K=V=128), the
short conv (B=8 T=4096 D=2048, per-head normalisation) and the gated RMSNorm (524288 rows of 128) forward and
backward twice each, and two copies of a 256 MiB device buffer, whose known size calibrates the counters.  Not
collected by pytest."""
import sys, torch
import os
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
from archbench_amd import ops
from archbench_amd.synthetic import make_inputs, make_step_inputs
B,T,H,K,V = 8,4096,16,128,128
x = make_inputs(B,T,H,K,V, with_do=True).to("cuda", torch.bfloat16)
for _ in range(2):
    _, _, stash = ops.chunk_fwd_stash(x.q,x.k,x.v,x.g,x.beta,None,1.0)
    ops.chunk_bwd_stashed(x.q,x.k,x.v,x.g,x.beta,None,x.do,None,stash,1.0)
    del stash
ops.chunk_fwd(x.q,x.k,x.v,x.g,x.beta,None,1.0)
ops.chunk_bwd(x.q,x.k,x.v,x.g,x.beta,None,x.do,None,1.0)
q,k,v,g,b,S = make_step_inputs(256,16,128,128)
q,k,v = (t.to("cuda", torch.bfloat16) for t in (q,k,v)); g,b,S = g.cuda(), b.cuda(), S.cuda()
for _ in range(2): ops.recurrent_step(q,k,v,g,b,S,1.0)
del x
xc, dyc = (torch.randn(8, 4096, 2048, device="cuda").bfloat16() for _ in range(2))
wc = torch.randn(2048, 4, device="cuda")
for _ in range(2):
    ops.short_conv(xc, wc, None, None, 128); ops.short_conv_bwd(xc, wc, None, None, dyc, 128)
del xc, dyc
xn, gn, dyn = (torch.randn(8 * 4096 * 16, 128, device="cuda").bfloat16() for _ in range(3))
wn = torch.rand(128, device="cuda") + 0.5
for _ in range(2):
    ops.gated_rmsnorm(xn, gn, wn, 1e-5); ops.gated_rmsnorm_bwd(xn, gn, wn, dyn, 1e-5)
del xn, gn, dyn
a = torch.empty(256*2**20, dtype=torch.uint8, device="cuda").fill_(1)
c = torch.empty_like(a)
for _ in range(2): c.copy_(a)
torch.cuda.synchronize(); print("done", flush=True)
