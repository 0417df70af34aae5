"""The C-ABI library loads, exports every symbol include/gdn_mi355x.h declares, and its host-only entry points
(version, support query, workspace sizing, argument validation) behave -- no GPU needed."""

import ctypes
import os
import re

import pytest

from archbench_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "gdn_mi355x.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(gdn_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert {"gdn_chunk_fwd", "gdn_chunk_bwd", "gdn_recurrent_step", "gdn_chunk_fwd_ws_bytes",
            "gdn_chunk_bwd_ws_bytes", "gdn_last_error"} <= set(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert set(names) == set(_lib.SIGNATURES), "binding table out of sync with the header"
    for n in names:
        assert hasattr(lib, n), n


def test_version_and_support_table():
    lib = _lib.load()
    assert lib.gdn_version() >= 100
    assert _lib.supported("chunk", 128, 128, __import__("torch").bfloat16)
    assert _lib.supported("chunk", 64, 64, __import__("torch").float32)
    assert _lib.supported("step", 128, 128, __import__("torch").bfloat16)
    assert not lib.gdn_supported(0, 96, 128, 1)
    assert not lib.gdn_supported(7, 128, 128, 1)


def test_workspace_sizes():
    import torch
    fwd = _lib.ws_bytes("fwd", 8, 4096, 16, 128, 128, torch.bfloat16)
    bwd = _lib.ws_bytes("bwd", 8, 4096, 16, 128, 128, torch.bfloat16)
    BH, NT = 8 * 16, 64
    # the forward's workspace holds the chunk factors: Tm and P (their ten 16x16 blocks on and below the diagonal,
    # packed), G (64 fp32) per chunk
    assert fwd == BH * NT * (2 * 10 * 256 * 2 + 64 * 4)
    # the backward adds the leaving state's gradient (K x V), R and dY (64 x V) per chunk, and the entering state of
    # every second chunk (bf16 at V <= 128: the gradient kernel advances it through the chunk between)
    assert bwd == fwd + BH * NT * (128 * 128 * 2 + 2 * 64 * 128 * 2) + BH * (NT // 2) * 128 * 128 * 2
    # ragged T rounds up to whole chunks
    assert _lib.ws_bytes("bwd", 1, 65, 1, 64, 64, torch.float32) == 2 * _lib.ws_bytes("bwd", 1, 64, 1, 64, 64,
                                                                                        torch.float32)


def test_stash_sizes_split_the_backward_workspace():
    import torch
    for args in [(8, 4096, 16, 128, 128, torch.bfloat16), (1, 65, 3, 64, 64, torch.float32)]:
        stash, grad = _lib.stash_bytes(*args)
        assert stash + grad == _lib.ws_bytes("bwd", *args)
    B, T, H, K, V = 8, 4096, 16, 128, 128
    stash, grad = _lib.stash_bytes(B, T, H, K, V, torch.bfloat16)
    # per chunk: Tm and P (ten 16x16 bf16 blocks each), G (64 fp32), R (64 x V bf16); per pair of chunks: the
    # entering state (K x V bf16)
    assert stash == B * H * 64 * (2 * 10 * 256 * 2 + 64 * 4 + 64 * V * 2) + B * H * 32 * K * V * 2
    # the n-step pair keeps every entering state; so do V = 256 and fp32
    ns_stash, ns_grad = _lib.stash_bytes(B, T, H, K, V, torch.bfloat16, nsgdn=True)
    assert ns_stash == stash + B * H * 32 * K * V * 2 and ns_grad == grad
    s256, _ = _lib.stash_bytes(8, 4096, 16, 128, 256, torch.bfloat16)
    assert s256 == 8 * 16 * 64 * (2 * 10 * 256 * 2 + 64 * 4 + 64 * 256 * 2 + 128 * 256 * 2)
    # odd chunk counts keep the last (unpaired) chunk's state: ceil(NT / 2) states per sequence
    s3, _ = _lib.stash_bytes(1, 130, 1, 64, 64, torch.bfloat16)
    assert s3 == 3 * (2 * 10 * 256 * 2 + 64 * 4 + 64 * 64 * 2) + 2 * 64 * 64 * 2


def test_stashed_backward_rejects_missing_stash():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.gdn_chunk_bwd_stashed(p, p, p, p, p, None, p, None, p, p, p, p, p, None, None, 0, p, 1 << 40,
                                   1, 64, 1, 64, 64, 1.0, 1, None)
    assert rc == _lib.GDN_ERR_WORKSPACE
    assert b"stash" in lib.gdn_last_error()


def test_argument_errors_do_not_touch_the_gpu():
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    assert lib.gdn_chunk_fwd_ws_bytes(1, 64, 1, 64, 64, 5, ctypes.byref(n)) == _lib.GDN_ERR_ARG
    assert b"dtype" in lib.gdn_last_error()
    assert lib.gdn_chunk_fwd_ws_bytes(-1, 64, 1, 64, 64, 1, ctypes.byref(n)) == _lib.GDN_ERR_ARG
    rc = lib.gdn_chunk_fwd(None, None, None, None, None, None, None, None, None, 0, 1, 64, 1, 96, 64, 1.0, 1, None)
    assert rc == _lib.GDN_ERR_SHAPE
    rc = lib.gdn_chunk_fwd(None, None, None, None, None, None, None, None, None, 0, 1, 64, 1, 64, 64, 1.0, 1, None)
    assert rc == _lib.GDN_ERR_ARG  # null pointers rejected before any launch
    with pytest.raises(ValueError):
        _lib.check(_lib.GDN_ERR_SHAPE, "x")


def test_gates_backward_rejects_too_many_heads():
    """The gates backward stages a tile of per-element gradients in LDS (1024 elements): more heads than that
    per token are refused before anything is launched."""
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    assert lib.gdn_gates_bwd_ws_bytes(4, 1024, ctypes.byref(n)) == _lib.GDN_OK
    assert lib.gdn_gates_bwd_ws_bytes(4, 1025, ctypes.byref(n)) == _lib.GDN_ERR_SHAPE
    assert b"1024" in lib.gdn_last_error()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.gdn_gates_bwd(p, p, 0, p, None, None, p, p, p, p, 0, None, None, None, p, 1 << 30, 4, 2000, 1.0,
                           float("-inf"), 1, None)
    assert rc == _lib.GDN_ERR_SHAPE
    # row strides below H are refused
    rc = lib.gdn_gates_fwd(p, p, 3, p, None, None, p, p, 4, 4, 1.0, float("-inf"), 1, None)
    assert rc == _lib.GDN_ERR_ARG and b"lda" in lib.gdn_last_error()


def test_fp32_head_size_error_names_the_bf16_route():
    """fp32 chunk kernels exist for K = 64 only; K = 128 in fp32 is refused with a message pointing to bf16."""
    lib = _lib.load()
    rc = lib.gdn_chunk_fwd(None, None, None, None, None, None, None, None, None, 0, 1, 64, 1, 128, 256, 1.0,
                           _lib.DTYPE_F32, None)
    assert rc == _lib.GDN_ERR_SHAPE
    assert b"bf16" in lib.gdn_last_error() and b"K=64" in lib.gdn_last_error()


def test_strided_input_layouts_are_validated_before_any_launch():
    """The conv's x row stride and the norm's gate line layout are checked on the host: a stride below the row
    width or off a 4-channel (conv) or 16-byte (gate) multiple, or a row count that is not a whole number of gate
    lines, is refused."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = lib.gdn_short_conv_fwd(p, 100, p, None, None, p, None, 1, 8, 128, 4, 0, _lib.DTYPE_BF16, None)
    assert rc == _lib.GDN_ERR_ARG and b"ldx" in lib.gdn_last_error()
    rc = lib.gdn_short_conv_fwd(p, 130, p, None, None, p, None, 1, 8, 128, 4, 0, _lib.DTYPE_BF16, None)
    assert rc == _lib.GDN_ERR_ARG and b"multiple of 4" in lib.gdn_last_error()
    rc = lib.gdn_short_conv_bwd(p, 64, p, None, None, p, p, 0, p, None, None, p, 1 << 20, 1, 8, 128, 4, 0,
                                _lib.DTYPE_BF16, None)
    assert rc == _lib.GDN_ERR_ARG and b"ldx" in lib.gdn_last_error()
    rc = lib.gdn_short_conv_bwd(p, 0, p, None, None, p, p, 126, p, None, None, p, 1 << 20, 1, 8, 128, 4, 0,
                                _lib.DTYPE_BF16, None)
    assert rc == _lib.GDN_ERR_ARG and b"lddx" in lib.gdn_last_error()
    rc = lib.gdn_gated_rmsnorm_fwd(p, p, 3072, 4, None, p, 10, 256, 1e-5, _lib.DTYPE_BF16, None)
    assert rc == _lib.GDN_ERR_ARG and b"gate layout" in lib.gdn_last_error()
    rc = lib.gdn_gated_rmsnorm_fwd(p, p, 512, 4, None, p, 8, 256, 1e-5, _lib.DTYPE_BF16, None)
    assert rc == _lib.GDN_ERR_ARG and b"gate layout" in lib.gdn_last_error()


def test_token_scan_rejects_misaligned_vector_arrays():
    """The token scan reads q, k and u (and the states) as 16-byte vectors: a pointer off a 16-byte boundary (an
    offset view handed straight to the C ABI) is refused before anything is launched, forward and backward."""
    lib = _lib.load()
    ok, off = ctypes.c_void_p(1 << 12), ctypes.c_void_p((1 << 12) + 4)  # never dereferenced: validation fails first
    big = 1 << 40
    for which in range(3):  # q, k, u misaligned in turn
        qku = [ok, ok, ok]
        qku[which] = off
        rc = lib.gdn_token_scan_fwd(*qku, ok, ok, None, ok, ok, ok, big, None, 1, 64, 1, 64, 64, None)
        assert rc == _lib.GDN_ERR_ARG and b"16-byte" in lib.gdn_last_error(), which
        rc = lib.gdn_token_scan_bwd(*qku, ok, ok, ok, big, ok, None, ok, ok, ok, ok, ok, None, ok, big,
                                    1, 64, 1, 64, 64, None)
        assert rc == _lib.GDN_ERR_ARG and b"16-byte" in lib.gdn_last_error(), which
