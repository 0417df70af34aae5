"""Writes tests/golden/gdn_cfg0_slice.npz: a slice of the config-0 workload (fp32, B=2 T=512 H=4 K=V=64,
seed 0; here batch 0, heads 0-1, first 96 tokens = one full 64-token chunk plus a ragged 32-token tail) with
the fp64 oracle's outputs: o, final state, and the gradients for a seeded dO and dhT.

    python tests/golden/make_golden.py

The vectors come from this repository's oracle (the reference ships no golden vectors for this path); they pin
the oracle against regressions and give the GPU a fixed known-answer test that needs no oracle at run time.
"""

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from archbench_amd.synthetic import make_inputs  # noqa: E402
from oracle import gdn_oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gdn_cfg0_slice.npz")
T_SLICE, H_SLICE, SCALE = 96, 2, 1.0


def slice_inputs():
    x = make_inputs(2, 512, 4, 64, 64, seed=0)
    sl = lambda t: t[0:1, :T_SLICE, :H_SLICE].contiguous()
    gen = torch.Generator().manual_seed(1234)
    do = torch.randn(1, T_SLICE, H_SLICE, 64, generator=gen)
    dhT = torch.randn(1, H_SLICE, 64, 64, generator=gen) * 0.1
    return dict(q=sl(x.q), k=sl(x.k), v=sl(x.v), g=sl(x.g), beta=sl(x.beta), do=do, dhT=dhT)


def main():
    x = slice_inputs()
    o, hT = O.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], SCALE)
    dq, dk, dv, dg, db, dh0 = O.recurrent_bwd(x["q"], x["k"], x["v"], x["g"], x["beta"], x["do"], SCALE, None,
                                               x["dhT"])
    arrs = {k: v.numpy().astype(np.float32) for k, v in x.items()}
    out = dict(o=o, hT=hT, dq=dq, dk=dk, dv=dv, dg=dg, dbeta=db, dh0=dh0)
    arrs.update({k: v.detach().numpy().astype(np.float32) for k, v in out.items()})
    arrs["scale"] = np.float32(SCALE)
    np.savez_compressed(OUT, **arrs)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
