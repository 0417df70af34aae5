"""Known-answer vectors (tests/golden/gdn_cfg0_slice.npz, written by tests/golden/make_golden.py from the fp64
oracle on a slice of config 0): the input generator and the oracle must reproduce them on the CPU, and the
HIP kernels must match them on the GPU at the fp32 bar (absolute max-abs <= 1e-4 for the output, the final
state and every gradient)."""

import os

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "gdn_cfg0_slice.npz")


def load():
    z = np.load(FIX)  # allow_pickle stays False
    return {k: torch.from_numpy(z[k]) for k in z.files}


def test_generator_reproduces_fixture_inputs():
    from tests.golden.make_golden import slice_inputs

    x = slice_inputs()
    f = load()
    for k in ("q", "k", "v", "g", "beta", "do", "dhT"):
        torch.testing.assert_close(x[k], f[k], rtol=0, atol=0, msg=k)


def test_oracle_reproduces_fixture_outputs():
    f = load()
    s = float(f["scale"])
    o, hT = O.chunk_fwd(f["q"], f["k"], f["v"], f["g"], f["beta"], s)
    torch.testing.assert_close(o.float(), f["o"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(hT.float(), f["hT"], rtol=1e-5, atol=1e-6)
    grads = O.chunk_bwd(f["q"], f["k"], f["v"], f["g"], f["beta"], f["do"], s, None, f["dhT"])
    for n, a in zip(["dq", "dk", "dv", "dg", "dbeta", "dh0"], grads):
        torch.testing.assert_close(a.float(), f[n], rtol=1e-5, atol=1e-5, msg=n)


@pytest.mark.gpu
def test_kernels_match_fixture_fp32():
    from archbench_amd import ops
    from tests.gpu_util import assert_fp32_close

    f = {k: v.cuda() for k, v in load().items()}
    s = float(f["scale"])
    o, hT = ops.chunk_gated_delta_rule(f["q"], f["k"], f["v"], f["g"], f["beta"], scale=s, output_final_state=True)
    assert (o - f["o"]).abs().max().item() <= 1e-4
    assert (hT - f["hT"]).abs().max().item() <= 1e-4
    grads = ops.chunk_bwd(f["q"], f["k"], f["v"], f["g"], f["beta"], None, f["do"], f["dhT"], s)
    names = ["dq", "dk", "dv", "dg", "dbeta", "dh0"]
    assert_fp32_close("golden cfg0 slice", names, grads, [f[n] for n in names], 1e-4)
