"""Module-level drop-in surface on the CPU: registry semantics (archbench/layers/__init__.py:1-26), layer
construction from the reference's YAML kwargs, and shape propagation through the custom op's fake kernel."""

import pytest
import torch

from archbench_amd import layers
from archbench_amd.layers.fla import FLAMixer, build_fla
from archbench_amd.layers.gdn import GatedDeltaNet

GDN_YAML = dict(head_dim=128, expand_v=2.0, use_gate=True, use_short_conv=True, conv_size=4)  # arch/gdn.yaml


def test_registry_surface():
    assert "gdn" in layers.available()
    with pytest.raises(KeyError, match="unknown arch"):
        layers.build_mixer("nope", 64, 0, 2)
    with pytest.raises(ImportError):
        layers.build_mixer("fla:MesaNet", 64, 0, 2)


def test_build_gdn_like_model_py():
    m = layers.build_mixer("gdn", 512, 3, 10, num_heads=4, **GDN_YAML)  # 65m/gdn.yaml
    assert isinstance(m, FLAMixer) and isinstance(m.layer, GatedDeltaNet)
    L = m.layer
    assert L.hidden_size == 512 and L.layer_idx == 3
    assert (L.num_heads, L.head_k_dim, L.head_v_dim) == (4, 128, 256)
    names = dict(m.named_modules())
    assert any(n.endswith("o_proj") for n in names)  # zero-init rule of model.py:80-82 applies
    assert L.q_proj.weight.shape == (512, 512) and L.v_proj.weight.shape == (1024, 512)


def test_auto_kwargs_filtered_by_signature():
    m = build_fla("GatedDeltaNet", 256, 1, 4, num_heads=2, head_dim=64)
    assert m.layer.hidden_size == 256 and m.layer.layer_idx == 1


def test_no_cpu_fallback():
    m = layers.build_mixer("gdn", 64, 0, 2, num_heads=1, head_dim=64, expand_v=1.0)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        m(torch.randn(1, 8, 64))


def test_fake_tensor_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    from archbench_amd import ops

    with FakeTensorMode():
        q = torch.empty(2, 70, 3, 64, dtype=torch.bfloat16)
        v = torch.empty(2, 70, 3, 128, dtype=torch.bfloat16)
        g = torch.empty(2, 70, 3)
        o, hT = ops.chunk_fwd(q, q, v, g, g, None, 1.0)
        assert o.shape == (2, 70, 3, 128) and o.dtype == torch.bfloat16
        assert hT.shape == (2, 3, 64, 128) and hT.dtype == torch.float32
        grads = ops.chunk_bwd(q, q, v, g, g, None, o, None, 1.0)
        assert [tuple(t.shape) for t in grads] == [(2, 70, 3, 64), (2, 70, 3, 64), (2, 70, 3, 128), (2, 70, 3),
                                                   (2, 70, 3), (2, 3, 64, 128)]


def test_shape_errors_are_value_errors():
    from archbench_amd import ops

    q = torch.empty(1, 4, 2, 64, device="meta")
    with pytest.raises((ValueError, RuntimeError)):
        ops._shapes(q, q[..., :32], q, q[..., 0], q[..., 0], None)


def test_short_conv_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    from archbench_amd import ops

    with FakeTensorMode():
        x = torch.empty(2, 70, 512, dtype=torch.bfloat16)
        w = torch.empty(512, 4)
        y, st = ops.short_conv(x, w, None, None, 128)
        assert y.shape == x.shape and y.dtype == torch.bfloat16 and st.shape == (2, 512, 3)
        dx, dw, db, dst = ops.short_conv_bwd(x, w, None, None, x, 128)
        assert dx.shape == x.shape and dw.shape == (512, 4) and dw.dtype == torch.float32
        assert db.shape == (512,) and dst.shape == (2, 512, 3) and dst.dtype == torch.bfloat16


def test_short_conv_cpu_raises():
    from archbench_amd import ops

    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.short_conv(torch.randn(1, 4, 512), torch.randn(512, 4), None, None, 0)


def test_nsgdn_registered_and_no_cpu_fallback():
    assert "nsgdn" in layers.available()
    m = layers.build_mixer("nsgdn", 128, 0, 2, num_heads=2, head_dim=64, expand_v=2.0, n_steps=2, lam=1.0)
    names = {n for n, _ in m.named_parameters()}
    assert {"in_proj.weight", "conv.weight", "A_log", "dt_bias", "b_bias", "lam", "norm.weight",
            "o_proj.weight"} <= names
    assert m.conv.weight.shape == (2 * 128 + 256, 1, 4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        m(torch.randn(1, 8, 128))
    with pytest.raises(ValueError):
        layers.build_mixer("nsgdn", 128, 0, 2, num_heads=2, head_dim=48)


def test_nsgdn_token_scan_choices():
    """The reference's "triton" and "ref" scan_impl are its exact fp32 token scan, which this build runs for
    head_dim 64 and 128 (quietly, as for "chunk" and "dplr"); other head sizes fall back to the chunk kernels and
    say so."""
    import warnings

    with warnings.catch_warnings():
        warnings.simplefilter("error")
        for impl in ("chunk", "dplr", "triton", "ref"):
            for hd in (64, 128):
                m = layers.build_mixer("nsgdn", 128, 0, 2, num_heads=2, head_dim=hd, scan_impl=impl)
                assert m.scan_impl == impl
    for impl in ("triton", "ref"):
        with pytest.warns(UserWarning, match="fp32 token scan"):
            layers.build_mixer("nsgdn", 128, 0, 2, num_heads=2, head_dim=32, scan_impl=impl)
    with pytest.raises(ValueError):
        layers.build_mixer("nsgdn", 128, 0, 2, num_heads=2, head_dim=64, scan_impl="cuda")


@pytest.mark.parametrize("use_gate", [True, False])
def test_fused_input_projections_equal_the_separate_linears(use_gate):
    """The gdn mixer runs its six input linears as one GEMM on the concatenated weights: outputs and every
    weight and input gradient equal those of the separate nn.Linear modules (fp64 on the CPU)."""
    torch.manual_seed(0)
    m = layers.build_mixer("gdn", 64, 0, 2, num_heads=2, head_dim=16, expand_v=2.0, use_gate=use_gate).double()
    mods = [m.layer.q_proj, m.layer.k_proj, m.layer.v_proj, m.layer.a_proj, m.layer.b_proj]
    if use_gate:
        mods.append(m.layer.g_proj)
    x = torch.randn(2, 5, 64, dtype=torch.float64, requires_grad=True)
    outs = m.layer.input_projections(x)
    assert [o.shape[-1] for o in outs] == [md.out_features for md in mods]
    ws = [torch.randn(o.shape, dtype=torch.float64) for o in outs]
    sum((o * w).sum() for o, w in zip(outs, ws)).backward()
    g_fused = [md.weight.grad.clone() for md in mods]
    gx = x.grad.clone()
    for md in mods:
        md.weight.grad = None
    x.grad = None
    ref = [md(x) for md in mods]
    for o, r in zip(outs, ref):
        torch.testing.assert_close(o, r, rtol=0, atol=1e-12)
    sum((r * w).sum() for r, w in zip(ref, ws)).backward()
    for gf, md in zip(g_fused, mods):
        torch.testing.assert_close(gf, md.weight.grad, rtol=0, atol=1e-12)
    torch.testing.assert_close(gx, x.grad, rtol=0, atol=1e-12)


def test_in_place_row_layouts_of_projection_slices():
    """The conv and norm ops read column slices of a fused projection's output in place: the token stride and the
    gate's line layout are derived from the view's strides, and anything they cannot express (a transposed view, a
    stride off the kernels' alignment) falls back to a contiguous copy."""
    from archbench_amd import ops
    B, T, L = 2, 5, 3072
    y = torch.zeros(B, T, L, dtype=torch.bfloat16)
    x, ld = ops._token_rows(y[..., 512:1024])
    assert ld == L and x.data_ptr() == y[..., 512:1024].data_ptr()       # read in place
    x, ld = ops._token_rows(y[..., :512].contiguous())
    assert ld == 512
    x, ld = ops._token_rows(y[..., 2:514])                                # 2 elements in: stride fine, base 4 B off
    assert ld == 512 and x.is_contiguous()
    x, ld = ops._token_rows(y[:1, ::2, :512])                            # every other token of one sequence
    assert ld == 2 * L and not x.is_contiguous()
    x, ld = ops._token_rows(y[:, ::2, :512])                             # ... of two: batch stride != T * ld
    assert ld == 512 and x.is_contiguous()
    x, ld = ops._token_rows(torch.zeros(B, 512, T, dtype=torch.bfloat16).transpose(1, 2))  # channels strided
    assert ld == 512 and x.is_contiguous()
    H, dim = 4, 256
    gate = y[..., 2048:2048 + H * dim].reshape(B, T, H, dim)
    g, ldg, gpl = ops._gate_lines(gate, dim)
    assert (ldg, gpl) == (L, H) and g.data_ptr() == gate.data_ptr()
    g, ldg, gpl = ops._gate_lines(gate.contiguous(), dim)
    assert (ldg, gpl) == (0, 1)
    g, ldg, gpl = ops._gate_lines(gate.transpose(2, 3).contiguous().transpose(2, 3), dim)  # dim not contiguous
    assert (ldg, gpl) == (0, 1) and g.is_contiguous()
