"""Short causal conv + SiLU (+ per-group L2 norm) on the GPU against the CPU oracle (oracle/conv_oracle.py).

Forward y and the new conv state, backward dx, dw, dbias and dstate, through the C ABI via ops.short_conv /
ops.short_conv_bwd, for fp32 (max-abs error <= 1e-4 relative to the output scale) and bf16 (rel-L2 <= 1e-2),
over the ragged lengths the chunking has to handle (T = 1, shorter than the kernel, one chunk, one chunk + 1,
several chunks), with and without bias, conv state and normalisation."""

import pytest
import torch

from archbench_amd import _lib, ops
from oracle import conv_oracle as CO
from tests.gpu_util import banner, max_abs, rel_l2

pytestmark = pytest.mark.gpu

W = 4


def _inputs(B, T, D, dtype, seed, with_bias, with_state):
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=gen)
    x = r(B, T, D).to(dtype).float()
    w = (r(D, W) * 0.5).to(dtype).float()
    bias = (r(D) * 0.1) if with_bias else None
    state = r(B, D, W - 1).to(dtype).float() if with_state else None
    dy = r(B, T, D).to(dtype).float()
    return x, w, bias, state, dy


def _dev(t, dtype):
    return None if t is None else t.to("cuda", dtype)


def _check(got, ref, dtype, what):
    if dtype == torch.float32:
        err = max_abs(got, ref) / max(1.0, ref.abs().max().item())
        assert err <= 1e-4, f"{what}: max-abs error {err:.3g}"
    else:
        err = rel_l2(got, ref)
        assert err <= 1e-2, f"{what}: rel-L2 error {err:.3g}"


CASES = [(T, ng, bias, state) for T in (1, 3, 5, 64, 65, 200)
         for (ng, bias, state) in ((0, False, False), (128, True, True), (64, False, True))]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("T,ng,with_bias,with_state", CASES)
def test_conv_matches_oracle(dtype, T, ng, with_bias, with_state):
    B, D = 2, 640  # two channel blocks of 512, the second partly past D
    banner(f"short conv B={B} T={T} D={D} norm={ng} bias={with_bias} state={with_state} {dtype}")
    x, w, bias, state, dy = _inputs(B, T, D, dtype, 7 + T, with_bias, with_state)
    y, st = ops.short_conv(_dev(x, dtype), w.cuda(), _dev(bias, torch.float32), _dev(state, dtype), ng)
    dx, dw, db, dst = ops.short_conv_bwd(_dev(x, dtype), w.cuda(), _dev(bias, torch.float32), _dev(state, dtype),
                                         _dev(dy, dtype), ng)
    torch.cuda.synchronize()
    y_ref, st_ref = CO.short_conv_fwd(x, w, bias, state, ng)
    dx_ref, dw_ref, db_ref, dst_ref = CO.short_conv_bwd(x, w, bias, state, dy, ng)
    _check(y, y_ref, dtype, "y")
    assert torch.equal(st.float().cpu(), st_ref.float()), "new conv state must be the last inputs exactly"
    _check(dx, dx_ref, dtype, "dx")
    _check(dw, dw_ref, dtype, "dw")
    if with_bias:
        _check(db, db_ref, dtype, "dbias")
    if with_state:
        _check(dst, dst_ref, dtype, "dstate")


def test_conv_state_chains_across_calls():
    """Prefill in two pieces through the returned state equals one call over the whole sequence."""
    banner("short conv state chaining")
    B, T, D = 2, 130, 512
    x, w, bias, _, _ = _inputs(B, T, D, torch.float32, 3, True, False)
    xd, wd, bd = x.cuda(), w.cuda(), bias.cuda()
    full, st_full = ops.short_conv(xd, wd, bd, None, 128)
    a, st = ops.short_conv(xd[:, :70].contiguous(), wd, bd, None, 128)
    b1, st = ops.short_conv(xd[:, 70:71].contiguous(), wd, bd, st, 128)
    b2, st = ops.short_conv(xd[:, 71:].contiguous(), wd, bd, st, 128)
    assert max_abs(torch.cat([a, b1, b2], 1), full) <= 1e-6
    assert torch.equal(st, st_full)


def test_conv_autograd_with_state_grad():
    """The autograd wrapper routes the gradient of the returned state back into x (and into the old state for
    short inputs), as differentiating the oracle end to end does."""
    banner("short conv autograd through new_state")
    B, D = 2, 512
    for T in (2, 40):
        x, w, bias, state, dy = _inputs(B, T, D, torch.float32, 11 + T, True, True)
        dst_out = torch.randn(B, D, W - 1, generator=torch.Generator().manual_seed(5))
        leaves = [t.cuda().requires_grad_() for t in (x, w, bias, state)]
        y, st = ops.short_conv(*leaves, 64)
        ((y * dy.cuda()).sum() + (st * dst_out.cuda()).sum()).backward()
        ref = [t.double().requires_grad_() for t in (x, w, bias, state)]
        y_r, st_r = CO.short_conv_fwd(*ref, 64)
        ((y_r * dy.double()).sum() + (st_r * dst_out.double()).sum()).backward()
        for n, a, b in zip(("dx", "dw", "dbias", "dstate"), leaves, ref):
            assert max_abs(a.grad, b.grad) <= 1e-4 * max(1.0, b.grad.abs().max().item()), (T, n)


def test_conv_empty_sequence():
    banner("short conv T=0")
    x = torch.empty(2, 0, 512, device="cuda")
    w = torch.randn(512, W, device="cuda")
    state = torch.randn(2, 512, W - 1, device="cuda")
    y, st = ops.short_conv(x, w, None, state, 0)
    assert y.shape == (2, 0, 512) and torch.equal(st, state)
    dx, dw, db, dst = ops.short_conv_bwd(x, w, None, state, x, 0)
    assert dx.shape == x.shape and not dw.any() and not dst.any()


def test_conv_rejects_unsupported_shapes():
    banner("short conv shape errors")
    x = torch.randn(1, 8, 10, device="cuda")
    with pytest.raises(ValueError, match="not compiled"):
        ops.short_conv(x, torch.randn(10, W, device="cuda"), None, None, 0)  # D % 4 != 0
    x, w12 = torch.randn(2, 8, 12), torch.randn(12, W)  # D = 12: three lanes of one wave
    y, _ = ops.short_conv(x.cuda(), w12.cuda(), None, None, 0)
    y_ref, _ = CO.short_conv_fwd(x, w12, None, None, 0)
    assert max_abs(y, y_ref) <= 1e-5
    x = torch.randn(1, 8, 512, device="cuda")
    with pytest.raises(ValueError, match="not compiled"):
        ops.short_conv(x, torch.randn(512, W, device="cuda"), None, None, 96)  # unsupported group
    with pytest.raises(ValueError, match="not compiled"):
        ops.short_conv(x, torch.randn(512, 3, device="cuda"), None, None, 0)  # kernel size 3
    with pytest.raises(ValueError):
        ops.short_conv(x, torch.randn(256, W, device="cuda"), None, None, 0)  # weight rows != D


def test_conv_large_deterministic():
    """Layer shape (D = 2048, q/k normalisation per 128-channel head): the backward is deterministic (fixed-order
    partial sums), and dw matches the oracle on a bounded slice recomputed independently."""
    banner("short conv B=2 T=4096 D=2048 determinism")
    B, T, D = 2, 4096, 2048
    x, w, bias, _, dy = _inputs(B, T, D, torch.bfloat16, 1, False, False)
    args = (_dev(x, torch.bfloat16), w.cuda(), None, None, _dev(dy, torch.bfloat16), 128)
    r1 = ops.short_conv_bwd(*args)
    r2 = ops.short_conv_bwd(*args)
    for a, b in zip(r1, r2):
        assert torch.equal(a, b)
    # channels 0..255 only: the oracle on a channel slice is the same computation (depthwise)
    sl = slice(0, 256)
    _, dw_ref, _, _ = CO.short_conv_bwd(x[..., sl], w[sl], None, None, dy[..., sl], 128, dtype=torch.float32)
    assert rel_l2(r1[1][sl], dw_ref) <= 1e-2
    assert _lib.conv_ws_bytes(B, T, D, W) >= B * (T // 64) * D * W * 4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,ng", [(200, 128), (65, 0), (3, 64)])
def test_conv_reads_a_column_slice_in_place(dtype, T, ng):
    """x as a column slice of a wider [B, T, L] tensor (the q, k or v part of a fused projection's output): read in
    place with its token stride, bit-identical to the same values made contiguous, forward and backward, and the
    autograd path leaves the slice's storage untouched."""
    banner(f"conv column slice dtype={dtype} T={T} ng={ng}")
    B, D, L, off = 2, 256, 768, 128
    gen = torch.Generator().manual_seed(5)
    wide = torch.randn(B, T, L, generator=gen).to("cuda", dtype)
    w = (torch.randn(D, W, generator=gen) * 0.5).cuda()
    dy = torch.randn(B, T, D, generator=gen).to("cuda", dtype)
    xs = wide[..., off:off + D]
    assert not xs.is_contiguous() and ops._token_rows(xs)[1] == L
    xc = xs.contiguous()
    y_s, st_s = ops.short_conv(xs, w, None, None, ng)
    y_c, st_c = ops.short_conv(xc, w, None, None, ng)
    assert torch.equal(y_s, y_c) and torch.equal(st_s, st_c)
    g_s = ops.short_conv_bwd(xs, w, None, None, dy, ng)
    g_c = ops.short_conv_bwd(xc, w, None, None, dy, ng)
    for a, b in zip(g_s, g_c):
        assert torch.equal(a, b)
    before = wide.clone()
    xa = wide[..., off:off + D].detach().requires_grad_()
    y, _ = ops.short_conv(xa, w, None, None, ng)
    y.float().sum().backward()
    assert torch.equal(xa.grad, ops.short_conv_bwd(xc, w, None, None, torch.ones_like(dy), ng)[0])
    assert torch.equal(wide, before)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mixer_input_stage_equals_separate_convs(dtype):
    """The fused input stage (q, k, v convolved out of one projection output with one weight for the three) gives
    exactly the separate short convs' outputs, and its backward exactly their input gradients written into the
    column slices of one dy and their weight gradients into the row slices of one dw."""
    banner(f"mixer input stage dtype={dtype}")
    B, T, kd, vd, ng = 2, 130, 256, 512, 128
    L = 2 * kd + vd
    gen = torch.Generator().manual_seed(11)
    y = torch.randn(B, T, L, generator=gen).to("cuda", dtype)
    w = (torch.randn(L, W, generator=gen) * 0.5).cuda()
    outs = ops.mixer_input_stage(y, w, kd, vd, ng)
    cols = [(0, kd, ng), (kd, kd, ng), (2 * kd, vd, 0)]
    for o, (c0, d, g) in zip(outs, cols):
        assert torch.equal(o, ops.short_conv(y[..., c0:c0 + d].contiguous(), w[c0:c0 + d], None, None, g)[0])
    grads = [torch.randn(o.shape, generator=gen).to("cuda", dtype) for o in outs]
    dy, dw = ops.mixer_input_stage_bwd(y, w, *grads, kd, vd, ng)
    for (c0, d, g), gr in zip(cols, grads):
        dx_ref, dw_ref, _, _ = ops.short_conv_bwd(y[..., c0:c0 + d].contiguous(), w[c0:c0 + d], None, None, gr, g)
        assert torch.equal(dy[..., c0:c0 + d], dx_ref) and torch.equal(dw[c0:c0 + d], dw_ref)
    # through autograd: every input gradient of the stage at once
    ya, wa = y.detach().requires_grad_(), w.detach().requires_grad_()
    out = ops.mixer_input_stage(ya, wa, kd, vd, ng)
    torch.autograd.backward(out, grads)
    assert torch.equal(ya.grad, dy) and torch.equal(wa.grad, dw)
    with pytest.raises(ValueError, match="2 key_dim"):
        ops.mixer_input_stage(y[..., :-4], w, kd, vd, ng)


def test_conv_taps_rounded_to_activation_dtype():
    """With bf16 activations the kernels use the taps rounded to bf16 (as the reference's conv runs its fp32
    weight under bf16 autocast): an fp32 weight gives bit for bit what its bf16-rounded copy gives, forward and
    backward; with fp32 activations the taps are used as they are."""
    banner("short conv taps rounded to the activation dtype")
    B, T, D = 2, 100, 256
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(B, T, D, generator=gen).cuda()
    dy = torch.randn(B, T, D, generator=gen).cuda()
    w = (torch.randn(D, W, generator=gen) * 0.5).cuda()
    wr = w.bfloat16().float()
    assert not torch.equal(w, wr)
    for ng in (0, 128):
        xb, dyb = x.bfloat16(), dy.bfloat16()
        assert torch.equal(ops.short_conv(xb, w, None, None, ng)[0], ops.short_conv(xb, wr, None, None, ng)[0])
        a = ops.short_conv_bwd(xb, w, None, None, dyb, ng)
        b = ops.short_conv_bwd(xb, wr, None, None, dyb, ng)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
        assert not torch.equal(ops.short_conv(x, w, None, None, ng)[0], ops.short_conv(x, wr, None, None, ng)[0])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_conv_backward_long_chunks_match_oracle(dtype):
    """Without normalisation a large grid takes the backward's 128-token waves (at least four waves per CU): a
    ragged last chunk (T = 4000 = 31 * 128 + 32), bias and conv state, against the oracle."""
    B, T, D = 4, 4000, 2048
    waves_long = (D // 256) * B * -(-T // 128)
    if waves_long < 4 * torch.cuda.get_device_properties(0).multi_processor_count:
        pytest.skip("device has too many CUs for this grid to take the long-chunk backward")
    banner(f"short conv backward, 128-token waves: B={B} T={T} D={D} {dtype}")
    x, w, bias, state, dy = _inputs(B, T, D, dtype, 11, True, True)
    dx, dw, db, dst = ops.short_conv_bwd(_dev(x, dtype), w.cuda(), _dev(bias, torch.float32), _dev(state, dtype),
                                         _dev(dy, dtype), 0)
    torch.cuda.synchronize()
    dx_ref, dw_ref, db_ref, dst_ref = CO.short_conv_bwd(x, w, bias, state, dy, 0)
    _check(dx, dx_ref, dtype, "dx")
    _check(dw, dw_ref, dtype, "dw")
    _check(db, db_ref, dtype, "dbias")
    _check(dst, dst_ref, dtype, "dstate")
