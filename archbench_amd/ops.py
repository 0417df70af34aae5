"""Gated DeltaNet operator API on the HIP C-ABI library.

Operator level (the reference's own pattern, archbench/layers/nsgdn.py:162-216 and :352-397): functional
``torch.library.custom_op`` ops with ``register_fake`` (so FakeTensor / ``torch.compile(dynamic=False)`` trace
without running kernels) and ``register_autograd``; outputs are allocated here with ``torch.empty``; kernels are
enqueued on the current stream.

    archbench_amd::gdn_chunk_fwd      (q, k, v, g, beta, h0?, scale) -> (o, hT)
    archbench_amd::gdn_chunk_bwd      (q, k, v, g, beta, h0?, do, dhT?, scale) -> (dq, dk, dv, dg, dbeta, dh0)
    archbench_amd::gdn_chunk_fwd_stash  (q, k, v, g, beta, h0?, scale) -> (o, hT, stash)
    archbench_amd::gdn_chunk_bwd_stashed (q, k, v, g, beta, h0?, do, dhT?, stash, scale) -> (dq, ..., dh0)
    archbench_amd::gdn_recurrent_step (q, k, v, g, beta, state!, scale) -> o        (state updated in place)

Training (autograd) uses the stash pair: the forward keeps the per-chunk states, R and chunk factors in a
uint8 ``stash`` tensor saved for the backward, which then skips its recompute sweep (the reference's forward
likewise hands its chunk factor A to the backward, nsgdn.py:352-363, :385-388).  The stash costs
``_lib.stash_bytes(...)[0]`` bytes of device memory per call (about 3.5x the size of v in bf16);
``ARCHBENCH_AMD_GDN_STASH=0`` selects the recompute path (gdn_chunk_fwd + gdn_chunk_bwd) instead.

Python entry points with fla's signatures (the arithmetic behind archbench's ``gdn`` mixer,
archbench/layers/fla.py:36-38):

    chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                           use_qk_l2norm_in_kernel=False) -> (o, final_state | None)
    fused_recurrent_gated_delta_rule(...)  -> (o, final_state | None)      (decode; T = 1 uses the step kernel)
    recurrent_step(q, k, v, g, beta, state, scale=None) -> o               (in-place decode step)

There is no CPU path and no alternative backend: tensors must live on a ROCm GPU and the library must be built.
Shape/dtype problems raise ValueError (as the reference's layer does, nsgdn.py:492-497); a missing library or
a launch failure raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import os
import warnings
from typing import Optional

import torch
from torch import Tensor

from . import _lib

__all__ = ["chunk_gated_delta_rule", "fused_recurrent_gated_delta_rule", "recurrent_step", "chunk_fwd",
           "chunk_bwd", "chunk_fwd_stash", "chunk_bwd_stashed", "nsgdn_scan", "nsgdn_scan_chunk", "short_conv", "mixer_input_stage", "write_direction",
           "gated_rmsnorm", "l2norm", "gdn_gates", "gdn_gates_ab", "cross_entropy_fwd_bwd_"]


def _require_gpu(*ts: Optional[Tensor]) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("the gated DeltaNet op runs only on a ROCm GPU (MI355X); got a tensor on "
                               f"{t.device}. There is no CPU fallback.")


def _arg(t: Optional[Tensor], dtype: Optional[torch.dtype] = None) -> Optional[Tensor]:
    """A kernel argument: ``dtype``, contiguous and 16-byte aligned (the C ABI requires it; an offset view is
    copied)."""
    if t is None:
        return None
    if dtype is not None:
        t = t.to(dtype)
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _token_rows(x: Tensor) -> tuple[Tensor, int]:
    """A [B, T, D] kernel argument as (tensor, ld): read in place when its channels are contiguous and its tokens
    lie ld elements apart with one stride throughout (e.g. a column slice of a fused projection's output, whose
    tokens are the projection's width apart), ld a multiple of 4 and the base 16-byte aligned; otherwise a
    contiguous copy (ld = D)."""
    B, T, D = x.shape
    ld = x.stride(1) if T > 1 else (x.stride(0) if B > 1 else D)
    if (x.stride(2) == 1 and ld >= D and (B <= 1 or x.stride(0) == T * ld) and ld % 4 == 0
            and x.data_ptr() % 16 == 0):
        return x, ld
    return _arg(x), D


def _gate_lines(gate: Tensor, dim: int) -> tuple[Tensor, int, int]:
    """A gate of rows of `dim` channels as (tensor, ldg, gpl): ldg = 0 for contiguous rows; otherwise read in place
    as lines of gpl rows (its second-to-last dimension, gpl * dim contiguous channels) ldg elements apart with one
    stride over the leading dimensions, such as [B, T, H, dim] heads sliced from a fused projection's output."""
    if gate.is_contiguous() and gate.data_ptr() % 16 == 0:
        return gate, 0, 1
    if gate.dim() >= 3 and gate.stride(-1) == 1 and gate.stride(-2) == dim and gate.data_ptr() % 16 == 0:
        gpl, lead = gate.shape[-2], gate.shape[:-2]
        ldg = gate.stride(-3) if lead[-1] > 1 else gpl * dim
        ok, expect = ldg >= gpl * dim and (ldg * gate.element_size()) % 16 == 0, ldg
        for i in range(len(lead) - 1, -1, -1):
            ok = ok and (lead[i] <= 1 or gate.stride(i) == expect)
            expect *= lead[i]
        if ok:
            return gate, ldg, gpl
    return _arg(gate), 0, 1


def _shapes(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, h0: Optional[Tensor]):
    if q.dim() != 4 or k.shape != q.shape:
        raise ValueError(f"q and k must be [B, T, H, K] with equal shapes, got {tuple(q.shape)} and {tuple(k.shape)}")
    B, T, H, K = q.shape
    if v.dim() != 4 or tuple(v.shape[:3]) != (B, T, H):
        raise ValueError(f"v must be [B, T, H, V] matching q's [B, T, H] = {(B, T, H)}, got {tuple(v.shape)}")
    V = v.shape[-1]
    if tuple(g.shape) != (B, T, H) or tuple(beta.shape) != (B, T, H):
        raise ValueError(f"g and beta must be [B, T, H] = {(B, T, H)}, got {tuple(g.shape)} and {tuple(beta.shape)}")
    if h0 is not None and tuple(h0.shape) != (B, H, K, V):
        raise ValueError(f"initial_state must be [B, H, K, V] = {(B, H, K, V)}, got {tuple(h0.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q, k, v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    return B, T, H, K, V


# ------------------------------------------------------------------------------------------------ chunk forward
@torch.library.custom_op("archbench_amd::gdn_chunk_fwd", mutates_args=())
def chunk_fwd(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, h0: Optional[Tensor],
              scale: float) -> tuple[Tensor, Tensor]:
    _require_gpu(q, k, v, g, beta, h0)
    B, T, H, K, V = _shapes(q, k, v, g, beta, h0)
    lib = _lib.load()
    dt = _lib.dtype_code(q.dtype)
    q, k, v = _arg(q), _arg(k), _arg(v)
    g, beta, h0 = _arg(g, torch.float32), _arg(beta, torch.float32), _arg(h0, torch.float32)
    o = torch.empty(B, T, H, V, dtype=q.dtype, device=q.device)
    hT = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    ws = _lib.workspace(q.device, _lib.ws_bytes("fwd", B, T, H, K, V, q.dtype))
    rc = lib.gdn_chunk_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta), _lib.ptr(h0),
                           _lib.ptr(o), _lib.ptr(hT), _lib.ptr(ws), ws.numel(), B, T, H, K, V, float(scale), dt,
                           _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_chunk_fwd")
    return o, hT


@chunk_fwd.register_fake
def _(q, k, v, g, beta, h0, scale):
    B, T, H, K = q.shape
    V = v.shape[-1]
    return q.new_empty(B, T, H, V), q.new_empty(B, H, K, V, dtype=torch.float32)


# ----------------------------------------------------------------------------------------------- chunk backward
@torch.library.custom_op("archbench_amd::gdn_chunk_bwd", mutates_args=())
def chunk_bwd(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, h0: Optional[Tensor], do: Tensor,
              dhT: Optional[Tensor], scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    _require_gpu(q, k, v, g, beta, h0, do, dhT)
    B, T, H, K, V = _shapes(q, k, v, g, beta, h0)
    if tuple(do.shape) != (B, T, H, V):
        raise ValueError(f"dO must be [B, T, H, V] = {(B, T, H, V)}, got {tuple(do.shape)}")
    lib = _lib.load()
    dt = _lib.dtype_code(q.dtype)
    q, k, v, do = _arg(q), _arg(k), _arg(v), _arg(do, q.dtype)
    g, beta, h0 = _arg(g, torch.float32), _arg(beta, torch.float32), _arg(h0, torch.float32)
    dhT = _arg(dhT, torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dg = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
    db = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
    dh0 = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    ws = _lib.workspace(q.device, _lib.ws_bytes("bwd", B, T, H, K, V, q.dtype))
    rc = lib.gdn_chunk_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta), _lib.ptr(h0),
                           _lib.ptr(do), _lib.ptr(dhT), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg),
                           _lib.ptr(db), _lib.ptr(dh0), _lib.ptr(ws), ws.numel(), B, T, H, K, V, float(scale), dt,
                           _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_chunk_bwd")
    return dq, dk, dv, dg, db, dh0


@chunk_bwd.register_fake
def _(q, k, v, g, beta, h0, do, dhT, scale):
    B, T, H, K = q.shape
    V = v.shape[-1]
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), q.new_empty(B, T, H, **f32),
            q.new_empty(B, T, H, **f32), q.new_empty(B, H, K, V, **f32))


def _chunk_setup(ctx, inputs, output):
    q, k, v, g, beta, h0, scale = inputs
    ctx.save_for_backward(q, k, v, g, beta, h0)
    ctx.scale = scale
    ctx.has_h0 = h0 is not None
    ctx.g_dtype, ctx.beta_dtype = g.dtype, beta.dtype
    # an unused final state gets no zero-filled gradient (the kernels take dhT = NULL)
    ctx.set_materialize_grads(False)


def _zero_do(do: Optional[Tensor], q: Tensor, v: Tensor) -> Tensor:
    return do if do is not None else torch.zeros(*q.shape[:3], v.shape[-1], dtype=q.dtype, device=q.device)


def _chunk_backward(ctx, do, dhT):
    q, k, v, g, beta, h0 = ctx.saved_tensors
    dq, dk, dv, dg, db, dh0 = chunk_bwd(q, k, v, g, beta, h0, _zero_do(do, q, v).contiguous(),
                                        None if dhT is None else dhT.contiguous(), ctx.scale)
    return dq, dk, dv, dg.to(ctx.g_dtype), db.to(ctx.beta_dtype), (dh0 if ctx.has_h0 else None), None


chunk_fwd.register_autograd(_chunk_backward, setup_context=_chunk_setup)


# ------------------------------------------------------------------------------------ training (stash) pair
def _prep(q, k, v, g, beta, h0):
    return (_arg(q), _arg(k), _arg(v), _arg(g, torch.float32), _arg(beta, torch.float32),
            _arg(h0, torch.float32))


@torch.library.custom_op("archbench_amd::gdn_chunk_fwd_stash", mutates_args=())
def chunk_fwd_stash(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, h0: Optional[Tensor],
                    scale: float) -> tuple[Tensor, Tensor, Tensor]:
    _require_gpu(q, k, v, g, beta, h0)
    B, T, H, K, V = _shapes(q, k, v, g, beta, h0)
    lib = _lib.load()
    q, k, v, g, beta, h0 = _prep(q, k, v, g, beta, h0)
    o = torch.empty(B, T, H, V, dtype=q.dtype, device=q.device)
    hT = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    stash = torch.empty(_lib.stash_bytes(B, T, H, K, V, q.dtype)[0], dtype=torch.uint8, device=q.device)
    rc = lib.gdn_chunk_fwd_stash(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta), _lib.ptr(h0),
                                 _lib.ptr(o), _lib.ptr(hT), _lib.ptr(stash), stash.numel(), B, T, H, K, V,
                                 float(scale), _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_chunk_fwd_stash")
    return o, hT, stash


@chunk_fwd_stash.register_fake
def _(q, k, v, g, beta, h0, scale):
    B, T, H, K = q.shape
    V = v.shape[-1]
    n = _lib.stash_bytes(B, T, H, K, V, q.dtype)[0]
    return (q.new_empty(B, T, H, V), q.new_empty(B, H, K, V, dtype=torch.float32),
            q.new_empty(n, dtype=torch.uint8))


@torch.library.custom_op("archbench_amd::gdn_chunk_bwd_stashed", mutates_args=())
def chunk_bwd_stashed(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, h0: Optional[Tensor], do: Tensor,
                      dhT: Optional[Tensor], stash: Tensor,
                      scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    _require_gpu(q, k, v, g, beta, h0, do, dhT, stash)
    B, T, H, K, V = _shapes(q, k, v, g, beta, h0)
    if tuple(do.shape) != (B, T, H, V):
        raise ValueError(f"dO must be [B, T, H, V] = {(B, T, H, V)}, got {tuple(do.shape)}")
    lib = _lib.load()
    q, k, v, g, beta, h0 = _prep(q, k, v, g, beta, h0)
    do = _arg(do, q.dtype)
    dhT = _arg(dhT, torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dg = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
    db = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
    dh0 = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    ws = _lib.workspace(q.device, _lib.stash_bytes(B, T, H, K, V, q.dtype)[1])
    rc = lib.gdn_chunk_bwd_stashed(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
                                   _lib.ptr(h0), _lib.ptr(do), _lib.ptr(dhT), _lib.ptr(dq), _lib.ptr(dk),
                                   _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(db), _lib.ptr(dh0), _lib.ptr(stash),
                                   stash.numel(), _lib.ptr(ws), ws.numel(), B, T, H, K, V, float(scale),
                                   _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_chunk_bwd_stashed")
    return dq, dk, dv, dg, db, dh0


@chunk_bwd_stashed.register_fake
def _(q, k, v, g, beta, h0, do, dhT, stash, scale):
    B, T, H, K = q.shape
    V = v.shape[-1]
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), q.new_empty(B, T, H, **f32),
            q.new_empty(B, T, H, **f32), q.new_empty(B, H, K, V, **f32))


def _stash_setup(ctx, inputs, output):
    q, k, v, g, beta, h0, scale = inputs
    ctx.save_for_backward(q, k, v, g, beta, h0, output[2])
    ctx.scale = scale
    ctx.has_h0 = h0 is not None
    ctx.g_dtype, ctx.beta_dtype = g.dtype, beta.dtype
    # no zero-filled gradients for the unused final state or the (integer) stash: the stash of a long sequence
    # is hundreds of MB, and autograd would otherwise fill a zero gradient of it every step
    ctx.set_materialize_grads(False)


def _stash_backward(ctx, do, dhT, _dstash):
    q, k, v, g, beta, h0, stash = ctx.saved_tensors
    dq, dk, dv, dg, db, dh0 = chunk_bwd_stashed(q, k, v, g, beta, h0, _zero_do(do, q, v).contiguous(),
                                                None if dhT is None else dhT.contiguous(), stash, ctx.scale)
    return dq, dk, dv, dg.to(ctx.g_dtype), db.to(ctx.beta_dtype), (dh0 if ctx.has_h0 else None), None


chunk_fwd_stash.register_autograd(_stash_backward, setup_context=_stash_setup)


def _use_stash(*ts: Optional[Tensor]) -> bool:
    if os.environ.get("ARCHBENCH_AMD_GDN_STASH", "1") == "0" or not torch.is_grad_enabled():
        return False
    return any(t is not None and t.requires_grad for t in ts)


# ---------------------------------------------------------------------- separate read / write vectors (nsgdn)
# archbench::nsgdn_chunk_fwd / _bwd (nsgdn.py:352-397): S~ = e^la S, r = v - S~^T k, S = S~ + u r^T, y = S^T q,
# on the same chunk kernels with u as the write key.  The forward fills the stash the backward reads (the
# reference's forward likewise returns its g and A for the backward).  bf16 (the reference casts to bf16).
def _nsgdn_shapes(q, k, u, v, la, h0):
    if u.shape != q.shape:
        raise ValueError(f"u must match q's shape {tuple(q.shape)}, got {tuple(u.shape)}")
    if not (q.dtype == k.dtype == u.dtype == v.dtype == torch.bfloat16):
        raise ValueError("the n-step chunk op takes bfloat16 q, k, u, v (as archbench's nsgdn_scan_chunk)")
    return _shapes(q, k, v, la, la, h0)


@torch.library.custom_op("archbench_amd::nsgdn_chunk_fwd", mutates_args=())
def nsgdn_chunk_fwd(q: Tensor, k: Tensor, u: Tensor, v: Tensor, la: Tensor, h0: Optional[Tensor],
                    scale: float) -> tuple[Tensor, Tensor, Tensor]:
    """(y, hT, stash)."""
    _require_gpu(q, k, u, v, la, h0)
    B, T, H, K, V = _nsgdn_shapes(q, k, u, v, la, h0)
    lib = _lib.load()
    q, k, u, v, la, h0 = _arg(q), _arg(k), _arg(u), _arg(v), _arg(la, torch.float32), _arg(h0, torch.float32)
    y = torch.empty(B, T, H, V, dtype=q.dtype, device=q.device)
    hT = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    stash = torch.empty(_lib.stash_bytes(B, T, H, K, V, q.dtype, nsgdn=True)[0], dtype=torch.uint8, device=q.device)
    rc = lib.gdn_nsgdn_chunk_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(u), _lib.ptr(v), _lib.ptr(la), _lib.ptr(h0),
                                 _lib.ptr(y), _lib.ptr(hT), _lib.ptr(stash), stash.numel(), B, T, H, K, V,
                                 float(scale), _lib.dtype_code(q.dtype), _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_nsgdn_chunk_fwd")
    return y, hT, stash


@nsgdn_chunk_fwd.register_fake
def _(q, k, u, v, la, h0, scale):
    B, T, H, K = q.shape
    V = v.shape[-1]
    n = _lib.stash_bytes(B, T, H, K, V, q.dtype, nsgdn=True)[0]
    return (q.new_empty(B, T, H, V), q.new_empty(B, H, K, V, dtype=torch.float32),
            q.new_empty(n, dtype=torch.uint8))


@torch.library.custom_op("archbench_amd::nsgdn_chunk_bwd", mutates_args=())
def nsgdn_chunk_bwd(q: Tensor, k: Tensor, u: Tensor, v: Tensor, la: Tensor, h0: Optional[Tensor], dy: Tensor,
                    dhT: Optional[Tensor], stash: Tensor,
                    scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dq, dk, du, dv, dla, dh0)."""
    _require_gpu(q, k, u, v, la, h0, dy, dhT, stash)
    B, T, H, K, V = _nsgdn_shapes(q, k, u, v, la, h0)
    lib = _lib.load()
    q, k, u, v, la, h0 = _arg(q), _arg(k), _arg(u), _arg(v), _arg(la, torch.float32), _arg(h0, torch.float32)
    dy, dhT = _arg(dy, q.dtype), _arg(dhT, torch.float32)
    dq, dk, du, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(u), torch.empty_like(v)
    dla = torch.empty(B, T, H, dtype=torch.float32, device=q.device)
    dh0 = torch.empty(B, H, K, V, dtype=torch.float32, device=q.device)
    ws = _lib.workspace(q.device, _lib.stash_bytes(B, T, H, K, V, q.dtype, nsgdn=True)[1])
    rc = lib.gdn_nsgdn_chunk_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(u), _lib.ptr(v), _lib.ptr(la), _lib.ptr(h0),
                                 _lib.ptr(dy), _lib.ptr(dhT), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(du),
                                 _lib.ptr(dv), _lib.ptr(dla), _lib.ptr(dh0), _lib.ptr(stash), stash.numel(),
                                 _lib.ptr(ws), ws.numel(), B, T, H, K, V, float(scale), _lib.dtype_code(q.dtype),
                                 _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_nsgdn_chunk_bwd")
    return dq, dk, du, dv, dla, dh0


@nsgdn_chunk_bwd.register_fake
def _(q, k, u, v, la, h0, dy, dhT, stash, scale):
    B, T, H, K = q.shape
    V = v.shape[-1]
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(u), torch.empty_like(v),
            q.new_empty(B, T, H, **f32), q.new_empty(B, H, K, V, **f32))


def _nsgdn_setup(ctx, inputs, output):
    q, k, u, v, la, h0, scale = inputs
    ctx.save_for_backward(q, k, u, v, la, h0, output[2])
    ctx.scale = scale
    ctx.has_h0 = h0 is not None
    ctx.la_dtype = la.dtype
    ctx.set_materialize_grads(False)  # as for the gated delta rule's stash pair


def _nsgdn_backward(ctx, dy, dhT, _dstash):
    q, k, u, v, la, h0, stash = ctx.saved_tensors
    if dy is None:
        dy = torch.zeros(*q.shape[:3], v.shape[-1], dtype=q.dtype, device=q.device)
    dq, dk, du, dv, dla, dh0 = nsgdn_chunk_bwd(q, k, u, v, la, h0, dy.contiguous(),
                                               None if dhT is None else dhT.contiguous(), stash, ctx.scale)
    return dq, dk, du, dv, dla.to(ctx.la_dtype), (dh0 if ctx.has_h0 else None), None


nsgdn_chunk_fwd.register_autograd(_nsgdn_backward, setup_context=_nsgdn_setup)


# The n-step family's write direction (nsgdn.py:61-75 with the shift of k at :535): u from k (p = the previous
# token's key of the same sequence), beta and the effective lam, one HIP pass each way (gdn_writedir.hip).
@torch.library.custom_op("archbench_amd::write_direction", mutates_args=())
def write_direction(k: Tensor, beta: Tensor, lam: Tensor, n_steps: int) -> Tensor:
    """u [B,T,H,K] in k's dtype: u_1 = beta k, u_{i+1} = u_i - lam beta (p . u_i) (p - (p . k) k), p = k[:, t-1]
    (zero at t = 0).  n_steps <= 1 is u = beta k, as in the reference; any number of steps."""
    _require_gpu(k, beta, lam)
    B, T, H, K = _wd_shapes(k, beta, lam)
    lib = _lib.load()
    k, beta, lam = _arg(k), _arg(beta, torch.float32), _arg(lam, torch.float32)
    u = torch.empty_like(k)
    rc = lib.gdn_write_direction_fwd(_lib.ptr(k), _lib.ptr(beta), _lib.ptr(lam), _lib.ptr(u), B, T, H, K,
                                     max(int(n_steps), 1), _lib.dtype_code(k.dtype), _lib.stream_ptr(k.device))
    _lib.check(rc, "gdn_write_direction_fwd")
    return u


def _wd_shapes(k: Tensor, beta: Tensor, lam: Tensor):
    if k.dim() != 4:
        raise ValueError(f"k must be [B, T, H, K], got {tuple(k.shape)}")
    B, T, H, K = k.shape
    if tuple(beta.shape) != (B, T, H) or tuple(lam.shape) != (H,):
        raise ValueError(f"beta must be [B, T, H] = {(B, T, H)} and lam [H] = [{H}], got {tuple(beta.shape)} and "
                         f"{tuple(lam.shape)}")
    return B, T, H, K


@write_direction.register_fake
def _(k, beta, lam, n_steps):
    return torch.empty_like(k)


@torch.library.custom_op("archbench_amd::write_direction_bwd", mutates_args=())
def write_direction_bwd(k: Tensor, beta: Tensor, lam: Tensor, du: Tensor,
                        n_steps: int) -> tuple[Tensor, Tensor, Tensor]:
    """(dk in k's dtype, dbeta [B,T,H] fp32, dlam [H] fp32)."""
    _require_gpu(k, beta, lam, du)
    B, T, H, K = _wd_shapes(k, beta, lam)
    lib = _lib.load()
    k, beta, lam, du = _arg(k), _arg(beta, torch.float32), _arg(lam, torch.float32), _arg(du, k.dtype)
    dk = torch.empty_like(k)
    dbeta = torch.empty(B, T, H, dtype=torch.float32, device=k.device)
    dlam_rows = torch.empty(B, T, H, dtype=torch.float32, device=k.device)
    rc = lib.gdn_write_direction_bwd(_lib.ptr(k), _lib.ptr(beta), _lib.ptr(lam), _lib.ptr(du), _lib.ptr(dk),
                                     _lib.ptr(dbeta), _lib.ptr(dlam_rows), B, T, H, K, max(int(n_steps), 1),
                                     _lib.dtype_code(k.dtype), _lib.stream_ptr(k.device))
    _lib.check(rc, "gdn_write_direction_bwd")
    return dk, dbeta, dlam_rows.sum((0, 1))


@write_direction_bwd.register_fake
def _(k, beta, lam, du, n_steps):
    B, T, H, K = k.shape
    f32 = dict(dtype=torch.float32)
    return torch.empty_like(k), k.new_empty(B, T, H, **f32), k.new_empty(H, **f32)


def _wd_setup(ctx, inputs, output):
    k, beta, lam, n_steps = inputs
    ctx.save_for_backward(k, beta, lam)
    ctx.n_steps = n_steps
    ctx.dtypes = (beta.dtype, lam.dtype)


def _wd_backward(ctx, du):
    k, beta, lam = ctx.saved_tensors
    dk, dbeta, dlam = write_direction_bwd(k, beta, lam, du.contiguous(), ctx.n_steps)
    return dk, dbeta.to(ctx.dtypes[0]), dlam.to(ctx.dtypes[1]), None


write_direction.register_autograd(_wd_backward, setup_context=_wd_setup)


# The exact fp32 token scan of the n-step family (the reference's "triton" / "ref" scan_impl): archbench::nsgdn_fwd
# and nsgdn_bwd (nsgdn.py:162-216) on gdn_tokenscan.hip.  The forward returns y, the residuals r and the state
# checkpoints, which its backward restarts from; the backward's dq, du, dk and dla come as per-wave-row-block
# partials that are added here in a fixed order.
TOKEN_SCAN_CT = 32  # tokens between the forward's checkpoints (gdn_tokenscan.hip)


def _token_shapes(q: Tensor, k: Tensor, u: Tensor, v: Tensor, la: Tensor):
    if q.dim() != 4 or k.shape != q.shape or u.shape != q.shape:
        raise ValueError(f"q, k, u must be [B, T, H, K] alike, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(u.shape)}")
    B, T, H, K = q.shape
    if v.dim() != 4 or tuple(v.shape[:3]) != (B, T, H) or tuple(la.shape) != (B, T, H):
        raise ValueError(f"v must be [B, T, H, V] and la [B, T, H] with (B, T, H) = {(B, T, H)}, got "
                         f"{tuple(v.shape)}, {tuple(la.shape)}")
    return B, T, H, K, v.shape[-1]


def _token_sizes(lib, B, T, H, K, V):
    st, sc, nb = ctypes.c_size_t(0), ctypes.c_size_t(0), ctypes.c_int(0)
    _lib.check(lib.gdn_token_scan_sizes(B, T, H, K, V, ctypes.byref(st), ctypes.byref(sc), ctypes.byref(nb)),
               "gdn_token_scan_sizes")
    return st.value, sc.value, nb.value


def _state_arg(t: Optional[Tensor], B: int, H: int, K: int, V: int, what: str) -> Optional[Tensor]:
    if t is None:
        return None
    if tuple(t.shape) != (B, H, K, V):
        raise ValueError(f"{what} must be [B, H, K, V] = {(B, H, K, V)}, got {tuple(t.shape)}")
    return _arg(t, torch.float32)


@torch.library.custom_op("archbench_amd::nsgdn_token_fwd", mutates_args=())
def nsgdn_token_fwd(q: Tensor, k: Tensor, u: Tensor, v: Tensor, la: Tensor, h0: Optional[Tensor],
                    output_final_state: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(y, r, st, hT), fp32: the scan's output, its residuals r = v - (e^la S) k, the state checkpoints and the
    final state [B, H, K, V] (empty unless output_final_state).  h0: an initial state [B, H, K, V] or None."""
    _require_gpu(q, k, u, v, la, h0)
    B, T, H, K, V = _token_shapes(q, k, u, v, la)
    lib = _lib.load()
    q, k, u, v, la = (_arg(t, torch.float32) for t in (q, k, u, v, la))
    h0 = _state_arg(h0, B, H, K, V, "h0")
    st_bytes, _, _ = _token_sizes(lib, B, T, H, K, V)
    y, r = torch.empty_like(v), torch.empty_like(v)
    st = torch.empty(st_bytes // 4, dtype=torch.float32, device=q.device)
    hT = torch.empty((B, H, K, V) if output_final_state else (0,), dtype=torch.float32, device=q.device)
    if B * T == 0:  # no token: the final state is the initial one
        if output_final_state:
            hT.copy_(h0) if h0 is not None else hT.zero_()
        return y, r, st, hT
    rc = lib.gdn_token_scan_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(u), _lib.ptr(v), _lib.ptr(la), _lib.ptr(h0),
                                _lib.ptr(y), _lib.ptr(r), _lib.ptr(st), st_bytes,
                                _lib.ptr(hT) if output_final_state else None, B, T, H, K, V,
                                _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_token_scan_fwd")
    return y, r, st, hT


@nsgdn_token_fwd.register_fake
def _(q, k, u, v, la, h0, output_final_state):
    B, T, H, K = q.shape
    V = v.shape[-1]
    nch = -(-T // TOKEN_SCAN_CT)
    f32 = dict(dtype=torch.float32)
    return (v.new_empty(v.shape, **f32), v.new_empty(v.shape, **f32), v.new_empty(B * H * nch * K * V, **f32),
            v.new_empty((B, H, K, V) if output_final_state else (0,), **f32))


@torch.library.custom_op("archbench_amd::nsgdn_token_bwd", mutates_args=())
def nsgdn_token_bwd(q: Tensor, k: Tensor, u: Tensor, la: Tensor, r: Tensor, st: Tensor, dy: Tensor,
                    dhT: Optional[Tensor], need_dh0: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(dq, dk, du, dv, dla, dh0), fp32; dh0 [B, H, K, V] when need_dh0, else empty.  dhT: the final state's
    gradient or None."""
    _require_gpu(q, k, u, la, r, st, dy, dhT)
    B, T, H, K, V = _token_shapes(q, k, u, r, la)
    lib = _lib.load()
    q, k, u, la, r, dy = (_arg(t, torch.float32) for t in (q, k, u, la, r, dy))
    dhT = _state_arg(dhT, B, H, K, V, "dhT")
    st_bytes, sc_bytes, nb = _token_sizes(lib, B, T, H, K, V)
    if st.numel() * 4 < st_bytes:
        raise ValueError("st is not this shape's checkpoint buffer")
    dev = q.device
    parts = [torch.empty(nb, B, T, H, K, dtype=torch.float32, device=dev) for _ in range(3)]
    dla_p = torch.empty(nb, B, T, H, dtype=torch.float32, device=dev)
    dv = torch.empty_like(r)
    dh0 = torch.empty((B, H, K, V) if need_dh0 else (0,), dtype=torch.float32, device=dev)
    if B * T == 0:  # no token: the initial state's gradient is the final state's
        if need_dh0:
            dh0.copy_(dhT) if dhT is not None else dh0.zero_()
        z = torch.zeros(B, T, H, K, dtype=torch.float32, device=dev)
        return z, z.clone(), z.clone(), dv, torch.zeros(B, T, H, dtype=torch.float32, device=dev), dh0
    sc = torch.empty(max(sc_bytes // 4, 1), dtype=torch.float32, device=dev)
    rc = lib.gdn_token_scan_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(u), _lib.ptr(la), _lib.ptr(r), _lib.ptr(st),
                                st.numel() * 4, _lib.ptr(dy), _lib.ptr(dhT), _lib.ptr(dv), _lib.ptr(parts[0]),
                                _lib.ptr(parts[1]), _lib.ptr(parts[2]), _lib.ptr(dla_p),
                                _lib.ptr(dh0) if need_dh0 else None, _lib.ptr(sc), sc.numel() * 4, B, T, H, K, V,
                                _lib.stream_ptr(dev))
    _lib.check(rc, "gdn_token_scan_bwd")
    dq, du, dk = (p[0] if nb == 1 else p.sum(0) for p in parts)
    return dq, dk, du, dv, (dla_p[0] if nb == 1 else dla_p.sum(0)), dh0


@nsgdn_token_bwd.register_fake
def _(q, k, u, la, r, st, dy, dhT, need_dh0):
    B, T, H, K = q.shape
    V = r.shape[-1]
    f32 = dict(dtype=torch.float32)
    return (q.new_empty(q.shape, **f32), q.new_empty(q.shape, **f32), q.new_empty(q.shape, **f32),
            r.new_empty(r.shape, **f32), la.new_empty(la.shape, **f32),
            q.new_empty((B, H, K, V) if need_dh0 else (0,), **f32))


def _token_setup(ctx, inputs, output):
    q, k, u, v, la, h0, output_final_state = inputs
    _, r, st, _ = output
    ctx.save_for_backward(q, k, u, la, r, st)
    ctx.dtypes = tuple(t.dtype for t in (q, k, u, v, la))
    ctx.h0_dtype = None if h0 is None else h0.dtype
    ctx.set_materialize_grads(False)  # r and st take no gradient: no zero-filled buffers for them


def _token_backward(ctx, dy, dr, dst, dhT):
    q, k, u, la, r, st = ctx.saved_tensors
    if dy is None and dhT is None:
        return None, None, None, None, None, None, None
    if dy is None:
        dy = torch.zeros_like(r)
    need_dh0 = ctx.h0_dtype is not None
    dq, dk, du, dv, dla, dh0 = nsgdn_token_bwd(q, k, u, la, r, st, dy.contiguous(),
                                               None if dhT is None else dhT.contiguous(), need_dh0)
    grads = tuple(g.to(dt) for g, dt in zip((dq, dk, du, dv, dla), ctx.dtypes))
    return (*grads, dh0.to(ctx.h0_dtype) if need_dh0 else None, None)


nsgdn_token_fwd.register_autograd(_token_backward, setup_context=_token_setup)


def nsgdn_scan(q: Tensor, k: Tensor, u: Tensor, v: Tensor, la: Tensor) -> Tensor:
    """archbench's nsgdn_scan (nsgdn.py:219-221): y [B, T, H, V] fp32 from the exact fp32 token scan, for q, k, u
    [B, T, H, K] (q already scaled), v [B, T, H, V] and log-retention la [B, T, H].  Differentiable w.r.t. every
    input; K in {64, 128}."""
    return nsgdn_token_fwd(q.float(), k.float(), u.float(), v.float(), la.float(), None, False)[0]


def nsgdn_scan_chunk(q: Tensor, k: Tensor, u: Tensor, v: Tensor, la: Tensor, scale: float = 1.0,
                     initial_state: Tensor | None = None, output_final_state: bool = False):
    """archbench's nsgdn_scan_chunk (nsgdn.py:400-405) on the HIP chunk kernels: returns y [B,T,H,V] in bf16
    (and the fp32 final state with ``output_final_state``).  Differentiable w.r.t. q, k, u, v, la and
    initial_state.  Any T (the reference falls back to its DPLR path when T % 64 != 0, nsgdn.py:402-403)."""
    dt = torch.bfloat16
    y, hT, _ = nsgdn_chunk_fwd(q.to(dt), k.to(dt), u.to(dt), v.to(dt), la.float(), initial_state, float(scale))
    return (y, hT) if output_final_state else y


# ------------------------------------------------------------------------------------ short causal conv + SiLU
# The ShortConv in front of the op (archbench/layers/nsgdn.py:420-470: archbench::causal_conv_silu and its
# backward as custom ops), with fla ShortConvolution's optional bias and decode state, and the per-head L2
# normalisation of q and k (nsgdn.py:527-528) fused in when norm_group > 0.
def _conv_shapes(x: Tensor, w: Tensor, bias: Optional[Tensor], state: Optional[Tensor]):
    if x.dim() != 3:
        raise ValueError(f"x must be [B, T, D], got {tuple(x.shape)}")
    B, T, D = x.shape
    if w.dim() != 2 or w.shape[0] != D:
        raise ValueError(f"w must be [D, W] with D = {D}, got {tuple(w.shape)}")
    W = w.shape[1]
    if bias is not None and tuple(bias.shape) != (D,):
        raise ValueError(f"bias must be [D] = [{D}], got {tuple(bias.shape)}")
    if state is not None and tuple(state.shape) != (B, D, W - 1):
        raise ValueError(f"conv state must be [B, D, W-1] = {(B, D, W - 1)}, got {tuple(state.shape)}")
    return B, T, D, W


@torch.library.custom_op("archbench_amd::short_conv", mutates_args=())
def short_conv(x: Tensor, w: Tensor, bias: Optional[Tensor], state: Optional[Tensor],
               norm_group: int) -> tuple[Tensor, Tensor]:
    """(y [B,T,D], new_state [B,D,W-1]): y = silu(causal depthwise conv(x)) (+ L2 norm per norm_group channels)."""
    _require_gpu(x, w, bias, state)
    B, T, D, W = _conv_shapes(x, w, bias, state)
    lib = _lib.load()
    x, ldx = _token_rows(x)
    w, bias, state = _arg(w, torch.float32), _arg(bias, torch.float32), _arg(state, x.dtype)
    y = x.new_empty(B, T, D)
    new_state = torch.empty(B, D, W - 1, dtype=x.dtype, device=x.device)
    rc = lib.gdn_short_conv_fwd(_lib.ptr(x), ldx, _lib.ptr(w), _lib.ptr(bias), _lib.ptr(state), _lib.ptr(y),
                                _lib.ptr(new_state), B, T, D, W, int(norm_group), _lib.dtype_code(x.dtype),
                                _lib.stream_ptr(x.device))
    _lib.check(rc, "gdn_short_conv_fwd")
    return y, new_state


@short_conv.register_fake
def _(x, w, bias, state, norm_group):
    B, T, D = x.shape
    return x.new_empty(B, T, D), x.new_empty(B, D, w.shape[1] - 1)


@torch.library.custom_op("archbench_amd::short_conv_bwd", mutates_args=())
def short_conv_bwd(x: Tensor, w: Tensor, bias: Optional[Tensor], state: Optional[Tensor], dy: Tensor,
                   norm_group: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dx, dw [D,W] fp32, dbias [D] fp32, dstate [B,D,W-1]); dbias / dstate are zeros-shaped if not needed."""
    _require_gpu(x, w, bias, state, dy)
    B, T, D, W = _conv_shapes(x, w, bias, state)
    dx = x.new_empty(B, T, D)
    dw, db, dstate = _conv_bwd_launch(x, w, bias, state, dy, dx, D, norm_group)
    return dx, dw, db, dstate


def _conv_bwd_launch(x: Tensor, w: Tensor, bias: Optional[Tensor], state: Optional[Tensor], dy: Tensor, dx: Tensor,
                     lddx: int, norm_group: int, dw: Optional[Tensor] = None) -> tuple[Tensor, Tensor, Tensor]:
    """The conv backward into dx, whose tokens lie lddx elements apart (dx may be a column slice of a wider
    gradient), and into dw when given (contiguous fp32 [D, W], e.g. a row slice of a larger weight gradient);
    returns (dw, dbias, dstate)."""
    B, T, D, W = _conv_shapes(x, w, bias, state)
    lib = _lib.load()
    dy = _arg(dy, x.dtype)
    x, ldx = _token_rows(x)
    w, bias, state = _arg(w, torch.float32), _arg(bias, torch.float32), _arg(state, x.dtype)
    if dw is None:
        dw = torch.empty(D, W, dtype=torch.float32, device=x.device)
    elif dw.shape != (D, W) or dw.dtype != torch.float32 or not dw.is_contiguous() or dw.data_ptr() % 16:
        raise ValueError(f"dw must be a contiguous 16-byte aligned fp32 [{D}, {W}] tensor")
    db = torch.empty(D, dtype=torch.float32, device=x.device)
    dstate = torch.empty(B, D, W - 1, dtype=x.dtype, device=x.device)
    ws = _lib.workspace(x.device, _lib.conv_ws_bytes(B, T, D, W))
    rc = lib.gdn_short_conv_bwd(_lib.ptr(x), ldx, _lib.ptr(w), _lib.ptr(bias), _lib.ptr(state), _lib.ptr(dy),
                                _lib.ptr(dx), lddx, _lib.ptr(dw), _lib.ptr(db), _lib.ptr(dstate), _lib.ptr(ws),
                                ws.numel(), B, T, D, W, int(norm_group), _lib.dtype_code(x.dtype),
                                _lib.stream_ptr(x.device))
    _lib.check(rc, "gdn_short_conv_bwd")
    return dw, db, dstate


@short_conv_bwd.register_fake
def _(x, w, bias, state, dy, norm_group):
    B, T, D = x.shape
    W = w.shape[1]
    f32 = dict(dtype=torch.float32)
    return x.new_empty(B, T, D), w.new_empty(D, W, **f32), w.new_empty(D, **f32), x.new_empty(B, D, W - 1)


def _conv_setup(ctx, inputs, output):
    x, w, bias, state, norm_group = inputs
    ctx.save_for_backward(x, w, bias, state)
    ctx.norm_group = norm_group
    ctx.w_dtype = w.dtype
    ctx.has_bias, ctx.has_state = bias is not None, state is not None
    ctx.set_materialize_grads(False)


def _conv_backward(ctx, dy, dstate_out):
    x, w, bias, state = ctx.saved_tensors
    if dy is None:
        dy = torch.zeros_like(x)
    dx, dw, db, dstate = short_conv_bwd(x, w, bias, state, dy.contiguous(), ctx.norm_group)
    if dstate_out is not None:
        # new_state is the last W-1 entries of [state | x^T]: the tail of x, reaching into the old state when
        # T < W-1
        W1, T = dstate_out.shape[-1], x.shape[1]
        if T >= W1:
            dx[:, T - W1:, :] += dstate_out.transpose(1, 2).to(dx.dtype)
        else:
            full = torch.cat([dstate.float(), dx.float().transpose(1, 2)], dim=-1)
            full[..., -W1:] += dstate_out.float()
            dstate, dx = full[..., :W1].to(dstate.dtype), full[..., W1:].transpose(1, 2).to(dx.dtype).contiguous()
    return (dx, dw.to(ctx.w_dtype), (db if ctx.has_bias else None), (dstate if ctx.has_state else None), None)


short_conv.register_autograd(_conv_backward, setup_context=_conv_setup)


# The mixer's input stage in one op: q, k and v convolved straight out of the q/k/v input projection's output y
# [B, T, 2 key_dim + value_dim] (its column groups, read in place), with one weight [2 key_dim + value_dim, W] for
# the three convolutions (q's rows, then k's, then v's).  The backward writes dq, dk, dv's input gradients into the
# column slices of one dy and the three weight gradients into the row slices of one dw, so no gradient of a split
# or of a concatenation costs a pass (the conv backward takes dx's row stride).
def _stage_dims(y: Tensor, w: Tensor, key_dim: int, value_dim: int):
    n = 2 * key_dim + value_dim
    if y.dim() != 3 or y.shape[-1] != n:
        raise ValueError(f"y must be [B, T, 2 key_dim + value_dim = {n}], got {tuple(y.shape)}")
    if w.dim() != 2 or w.shape[0] != n:
        raise ValueError(f"w must be [2 key_dim + value_dim = {n}, W], got {tuple(w.shape)}")
    return (0, key_dim), (key_dim, key_dim), (2 * key_dim, value_dim)


@torch.library.custom_op("archbench_amd::mixer_input_stage", mutates_args=())
def mixer_input_stage(y: Tensor, w: Tensor, key_dim: int, value_dim: int,
                      norm_group: int) -> tuple[Tensor, Tensor, Tensor]:
    """(q, k, v): silu(causal conv(.)) of y's q, k and v columns (q and k L2-normalised per norm_group channels;
    conv weights fp32, used rounded to y's dtype; no bias, no state)."""
    _require_gpu(y, w)
    cols = _stage_dims(y, w, key_dim, value_dim)
    w = _arg(w, torch.float32)
    return tuple(short_conv(y[..., c0:c0 + d], w[c0:c0 + d], None, None, ng)[0]
                 for (c0, d), ng in zip(cols, (norm_group, norm_group, 0)))


@mixer_input_stage.register_fake
def _(y, w, key_dim, value_dim, norm_group):
    B, T, _ = y.shape
    return y.new_empty(B, T, key_dim), y.new_empty(B, T, key_dim), y.new_empty(B, T, value_dim)


@torch.library.custom_op("archbench_amd::mixer_input_stage_bwd", mutates_args=())
def mixer_input_stage_bwd(y: Tensor, w: Tensor, dq: Tensor, dk: Tensor, dv: Tensor, key_dim: int, value_dim: int,
                          norm_group: int) -> tuple[Tensor, Tensor]:
    """(dy, dw): the three conv backwards written into dy's column slices and dw's row slices (dw fp32)."""
    _require_gpu(y, w, dq, dk, dv)
    cols = _stage_dims(y, w, key_dim, value_dim)
    w = _arg(w, torch.float32)
    B, T, L = y.shape
    dy = y.new_empty(B, T, L)
    dw = torch.empty(w.shape, dtype=torch.float32, device=w.device)
    for (c0, d), g, ng in zip(cols, (dq, dk, dv), (norm_group, norm_group, 0)):
        _conv_bwd_launch(y[..., c0:c0 + d], w[c0:c0 + d], None, None, g, dy[..., c0:c0 + d], L, ng, dw[c0:c0 + d])
    return dy, dw


@mixer_input_stage_bwd.register_fake
def _(y, w, dq, dk, dv, key_dim, value_dim, norm_group):
    return torch.empty_like(y), w.new_empty(w.shape, dtype=torch.float32)


def _stage_setup(ctx, inputs, output):
    y, w, key_dim, value_dim, norm_group = inputs
    ctx.save_for_backward(y, w)
    ctx.dims = (key_dim, value_dim, norm_group)


def _stage_backward(ctx, dq, dk, dv):
    y, w = ctx.saved_tensors
    dy, dw = mixer_input_stage_bwd(y, w, dq.contiguous(), dk.contiguous(), dv.contiguous(), *ctx.dims)
    return dy, dw.to(w.dtype), None, None, None


mixer_input_stage.register_autograd(_stage_backward, setup_context=_stage_setup)


# ---------------------------------------------------------------------------------------------- gated RMSNorm
# The output normalisation of the mixer (fla FusedRMSNormGated; nsgdn.py:539-541: self.norm(y) * silu(g)) as one
# pass: y = x * rsqrt(mean(x^2) + eps) * weight * silu(gate) over the last dimension, fp32 arithmetic.
def _norm_rows(x: Tensor, gate: Optional[Tensor], weight: Optional[Tensor]):
    if x.dim() < 1 or x.shape[-1] == 0:
        raise ValueError(f"x must have a non-empty last dimension, got {tuple(x.shape)}")
    dim = x.shape[-1]
    if gate is not None and gate.shape != x.shape:
        raise ValueError(f"gate must match x's shape {tuple(x.shape)}, got {tuple(gate.shape)}")
    if weight is not None and tuple(weight.shape) != (dim,):
        raise ValueError(f"weight must be [{dim}], got {tuple(weight.shape)}")
    return x.numel() // dim, dim


@torch.library.custom_op("archbench_amd::gated_rmsnorm", mutates_args=())
def gated_rmsnorm(x: Tensor, gate: Optional[Tensor], weight: Optional[Tensor], eps: float) -> Tensor:
    _require_gpu(x, gate, weight)
    rows, dim = _norm_rows(x, gate, weight)
    lib = _lib.load()
    x, weight = _arg(x), _arg(weight, torch.float32)
    gate, ldg, gpl = _gate_lines(gate.to(x.dtype), dim) if gate is not None else (None, 0, 1)
    y = torch.empty_like(x)
    rc = lib.gdn_gated_rmsnorm_fwd(_lib.ptr(x), _lib.ptr(gate), ldg, gpl, _lib.ptr(weight), _lib.ptr(y), rows,
                                   dim, float(eps), _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device))
    _lib.check(rc, "gdn_gated_rmsnorm_fwd")
    return y


@gated_rmsnorm.register_fake
def _(x, gate, weight, eps):
    return torch.empty_like(x)


@torch.library.custom_op("archbench_amd::gated_rmsnorm_bwd", mutates_args=())
def gated_rmsnorm_bwd(x: Tensor, gate: Optional[Tensor], weight: Optional[Tensor], dy: Tensor,
                      eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """(dx, dgate (zeros-shaped [0] without a gate), dweight [dim] fp32)."""
    _require_gpu(x, gate, weight, dy)
    rows, dim = _norm_rows(x, gate, weight)
    lib = _lib.load()
    x, weight, dy = _arg(x), _arg(weight, torch.float32), _arg(dy, x.dtype)
    gate, ldg, gpl = _gate_lines(gate.to(x.dtype), dim) if gate is not None else (None, 0, 1)
    dx = torch.empty_like(x)
    dgate = torch.empty_like(x) if gate is not None else x.new_empty(0)
    dw = torch.empty(dim, dtype=torch.float32, device=x.device)
    ws = _lib.workspace(x.device, _lib.norm_ws_bytes(rows, dim))
    rc = lib.gdn_gated_rmsnorm_bwd(_lib.ptr(x), _lib.ptr(gate), ldg, gpl, _lib.ptr(weight), _lib.ptr(dy),
                                   _lib.ptr(dx), _lib.ptr(dgate) if gate is not None else None, _lib.ptr(dw),
                                   _lib.ptr(ws), ws.numel(), rows, dim, float(eps), _lib.dtype_code(x.dtype),
                                   _lib.stream_ptr(x.device))
    _lib.check(rc, "gdn_gated_rmsnorm_bwd")
    return dx, dgate, dw


@gated_rmsnorm_bwd.register_fake
def _(x, gate, weight, dy, eps):
    return (torch.empty_like(x), torch.empty_like(x) if gate is not None else x.new_empty(0),
            x.new_empty(x.shape[-1], dtype=torch.float32))


def _norm_setup(ctx, inputs, output):
    x, gate, weight, eps = inputs
    ctx.save_for_backward(x, gate, weight)
    ctx.eps = eps
    ctx.w_dtype = None if weight is None else weight.dtype


def _norm_backward(ctx, dy):
    x, gate, weight = ctx.saved_tensors
    dx, dgate, dw = gated_rmsnorm_bwd(x, gate, weight, dy, ctx.eps)
    return (dx, (dgate.to(gate.dtype) if gate is not None else None),
            (dw.to(ctx.w_dtype) if weight is not None else None), None)


gated_rmsnorm.register_autograd(_norm_backward, setup_context=_norm_setup)


# ---------------------------------------------------------------------------------------------------- L2 norm
# y = scale * x / max(||x||, eps) over the last dimension: the per-head q / k normalisation (nsgdn.py:527-528,
# F.normalize(.) * DK^-1/2) where it is not fused into the short convolution.
@torch.library.custom_op("archbench_amd::l2norm", mutates_args=())
def l2norm(x: Tensor, eps: float, scale: float) -> Tensor:
    _require_gpu(x)
    rows, dim = _norm_rows(x, None, None)
    lib = _lib.load()
    x = _arg(x)
    y = torch.empty_like(x)
    rc = lib.gdn_l2norm_fwd(_lib.ptr(x), _lib.ptr(y), rows, dim, float(eps), float(scale), _lib.dtype_code(x.dtype),
                            _lib.stream_ptr(x.device))
    _lib.check(rc, "gdn_l2norm_fwd")
    return y


@l2norm.register_fake
def _(x, eps, scale):
    return torch.empty_like(x)


@torch.library.custom_op("archbench_amd::l2norm_bwd", mutates_args=())
def l2norm_bwd(x: Tensor, dy: Tensor, eps: float, scale: float) -> Tensor:
    _require_gpu(x, dy)
    rows, dim = _norm_rows(x, None, None)
    lib = _lib.load()
    x, dy = _arg(x), _arg(dy, x.dtype)
    dx = torch.empty_like(x)
    rc = lib.gdn_l2norm_bwd(_lib.ptr(x), _lib.ptr(dy), _lib.ptr(dx), rows, dim, float(eps), float(scale),
                            _lib.dtype_code(x.dtype), _lib.stream_ptr(x.device))
    _lib.check(rc, "gdn_l2norm_bwd")
    return dx


@l2norm_bwd.register_fake
def _(x, dy, eps, scale):
    return torch.empty_like(x)


def _l2_setup(ctx, inputs, output):
    x, eps, scale = inputs
    ctx.save_for_backward(x)
    ctx.eps, ctx.scale = eps, scale


def _l2_backward(ctx, dy):
    (x,) = ctx.saved_tensors
    return l2norm_bwd(x, dy, ctx.eps, ctx.scale), None, None


l2norm.register_autograd(_l2_backward, setup_context=_l2_setup)


# ------------------------------------------------------------------------------------------------------ gates
# g = max(-exp(A_log) * softplus(a + dt_bias), g_min) and beta = beta_scale * sigmoid(b + b_bias) per token and
# head (nsgdn.py:531-533; fla GatedDeltaNet's g and beta), one pass forward and one backward.
def _gate_shapes(a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Optional[Tensor], b_bias: Optional[Tensor]):
    if a.dim() < 1 or b.shape != a.shape:
        raise ValueError(f"a and b must share a shape [..., H], got {tuple(a.shape)} and {tuple(b.shape)}")
    H = a.shape[-1]
    for n, t in (("A_log", A_log), ("dt_bias", dt_bias), ("b_bias", b_bias)):
        if t is not None and tuple(t.shape) != (H,):
            raise ValueError(f"{n} must be [H] = [{H}], got {tuple(t.shape)}")
    if H == 0:
        raise ValueError("H must be positive")
    return a.numel() // H, H


@torch.library.custom_op("archbench_amd::gdn_gates", mutates_args=())
def gdn_gates(a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Optional[Tensor], b_bias: Optional[Tensor],
              beta_scale: float, g_min: float) -> tuple[Tensor, Tensor]:
    """(g, beta), fp32, shaped like a."""
    _require_gpu(a, b, A_log, dt_bias, b_bias)
    ntok, H = _gate_shapes(a, b, A_log, dt_bias, b_bias)
    lib = _lib.load()
    a, b = _arg(a), _arg(b, a.dtype)
    A_log, dt_bias, b_bias = _arg(A_log, torch.float32), _arg(dt_bias, torch.float32), _arg(b_bias, torch.float32)
    g = torch.empty(a.shape, dtype=torch.float32, device=a.device)
    beta = torch.empty(a.shape, dtype=torch.float32, device=a.device)
    rc = lib.gdn_gates_fwd(_lib.ptr(a), _lib.ptr(b), 0, _lib.ptr(A_log), _lib.ptr(dt_bias), _lib.ptr(b_bias),
                           _lib.ptr(g), _lib.ptr(beta), ntok, H, float(beta_scale), float(g_min),
                           _lib.dtype_code(a.dtype), _lib.stream_ptr(a.device))
    _lib.check(rc, "gdn_gates_fwd")
    return g, beta


@gdn_gates.register_fake
def _(a, b, A_log, dt_bias, b_bias, beta_scale, g_min):
    return a.new_empty(a.shape, dtype=torch.float32), a.new_empty(a.shape, dtype=torch.float32)


@torch.library.custom_op("archbench_amd::gdn_gates_bwd", mutates_args=())
def gdn_gates_bwd(a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Optional[Tensor], b_bias: Optional[Tensor],
                  dg: Tensor, dbeta: Tensor, beta_scale: float,
                  g_min: float) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """(da, db, dA_log, ddt_bias, db_bias); the three [H] gradients fp32."""
    _require_gpu(a, b, A_log, dt_bias, b_bias, dg, dbeta)
    ntok, H = _gate_shapes(a, b, A_log, dt_bias, b_bias)
    lib = _lib.load()
    a, b = _arg(a), _arg(b, a.dtype)
    A_log, dt_bias, b_bias = _arg(A_log, torch.float32), _arg(dt_bias, torch.float32), _arg(b_bias, torch.float32)
    dg, dbeta = _arg(dg, torch.float32), _arg(dbeta, torch.float32)
    da, db = torch.empty_like(a), torch.empty_like(a)
    dA, ddt, dbb = (torch.empty(H, dtype=torch.float32, device=a.device) for _ in range(3))
    ws = _lib.workspace(a.device, _lib.gates_ws_bytes(ntok, H))
    rc = lib.gdn_gates_bwd(_lib.ptr(a), _lib.ptr(b), 0, _lib.ptr(A_log), _lib.ptr(dt_bias), _lib.ptr(b_bias),
                           _lib.ptr(dg), _lib.ptr(dbeta), _lib.ptr(da), _lib.ptr(db), 0, _lib.ptr(dA), _lib.ptr(ddt),
                           _lib.ptr(dbb), _lib.ptr(ws), ws.numel(), ntok, H, float(beta_scale), float(g_min),
                           _lib.dtype_code(a.dtype), _lib.stream_ptr(a.device))
    _lib.check(rc, "gdn_gates_bwd")
    return da, db, dA, ddt, dbb


@gdn_gates_bwd.register_fake
def _(a, b, A_log, dt_bias, b_bias, dg, dbeta, beta_scale, g_min):
    H = a.shape[-1]
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(a), torch.empty_like(a), a.new_empty(H, **f32), a.new_empty(H, **f32),
            a.new_empty(H, **f32))


def _gates_setup(ctx, inputs, output):
    a, b, A_log, dt_bias, b_bias, beta_scale, g_min = inputs
    ctx.save_for_backward(a, b, A_log, dt_bias, b_bias)
    ctx.beta_scale, ctx.g_min = beta_scale, g_min
    ctx.set_materialize_grads(True)


def _gates_backward(ctx, dg, dbeta):
    a, b, A_log, dt_bias, b_bias = ctx.saved_tensors
    da, db, dA, ddt, dbb = gdn_gates_bwd(a, b, A_log, dt_bias, b_bias, dg, dbeta, ctx.beta_scale, ctx.g_min)
    return (da, db.to(b.dtype), dA.to(A_log.dtype), None if dt_bias is None else ddt.to(dt_bias.dtype),
            None if b_bias is None else dbb.to(b_bias.dtype), None, None)


gdn_gates.register_autograd(_gates_backward, setup_context=_gates_setup)


# The same gates from the two halves of one [..., 2H] projection output ab = [a | b] (nsgdn.py:522, :531-534 slice
# ab this way), read in place; the backward writes d(ab) as one tensor, so no gradient of the two slices has to be
# zero-filled and copied back into a full-width one.
def _ab_halves(ab: Tensor):
    if ab.dim() < 1 or ab.shape[-1] % 2 or ab.shape[-1] == 0:
        raise ValueError(f"ab must be [..., 2H], got {tuple(ab.shape)}")
    return ab.shape[-1] // 2


def _half_ptr(t: Tensor, H: int):
    return ctypes.c_void_p(t.data_ptr() + H * t.element_size())


@torch.library.custom_op("archbench_amd::gdn_gates_ab", mutates_args=())
def gdn_gates_ab(ab: Tensor, A_log: Tensor, dt_bias: Optional[Tensor], b_bias: Optional[Tensor], beta_scale: float,
                 g_min: float) -> tuple[Tensor, Tensor]:
    """(g, beta), fp32 [..., H], from ab [..., 2H] = [a | b]."""
    _require_gpu(ab, A_log, dt_bias, b_bias)
    H = _ab_halves(ab)
    ntok, _ = _gate_shapes(ab[..., :H], ab[..., H:], A_log, dt_bias, b_bias)
    lib = _lib.load()
    ab = _arg(ab)
    A_log, dt_bias, b_bias = _arg(A_log, torch.float32), _arg(dt_bias, torch.float32), _arg(b_bias, torch.float32)
    shape = (*ab.shape[:-1], H)
    g = torch.empty(shape, dtype=torch.float32, device=ab.device)
    beta = torch.empty(shape, dtype=torch.float32, device=ab.device)
    rc = lib.gdn_gates_fwd(_lib.ptr(ab), _half_ptr(ab, H), 2 * H, _lib.ptr(A_log), _lib.ptr(dt_bias),
                           _lib.ptr(b_bias), _lib.ptr(g), _lib.ptr(beta), ntok, H, float(beta_scale), float(g_min),
                           _lib.dtype_code(ab.dtype), _lib.stream_ptr(ab.device))
    _lib.check(rc, "gdn_gates_fwd")
    return g, beta


@gdn_gates_ab.register_fake
def _(ab, A_log, dt_bias, b_bias, beta_scale, g_min):
    shape = (*ab.shape[:-1], ab.shape[-1] // 2)
    return ab.new_empty(shape, dtype=torch.float32), ab.new_empty(shape, dtype=torch.float32)


@torch.library.custom_op("archbench_amd::gdn_gates_ab_bwd", mutates_args=())
def gdn_gates_ab_bwd(ab: Tensor, A_log: Tensor, dt_bias: Optional[Tensor], b_bias: Optional[Tensor], dg: Tensor,
                     dbeta: Tensor, beta_scale: float, g_min: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(d ab [..., 2H] in ab's dtype, dA_log, ddt_bias, db_bias fp32)."""
    _require_gpu(ab, A_log, dt_bias, b_bias, dg, dbeta)
    H = _ab_halves(ab)
    ntok, _ = _gate_shapes(ab[..., :H], ab[..., H:], A_log, dt_bias, b_bias)
    lib = _lib.load()
    ab = _arg(ab)
    A_log, dt_bias, b_bias = _arg(A_log, torch.float32), _arg(dt_bias, torch.float32), _arg(b_bias, torch.float32)
    dg, dbeta = _arg(dg, torch.float32), _arg(dbeta, torch.float32)
    dab = torch.empty_like(ab)
    dA, ddt, dbb = (torch.empty(H, dtype=torch.float32, device=ab.device) for _ in range(3))
    ws = _lib.workspace(ab.device, _lib.gates_ws_bytes(ntok, H))
    rc = lib.gdn_gates_bwd(_lib.ptr(ab), _half_ptr(ab, H), 2 * H, _lib.ptr(A_log), _lib.ptr(dt_bias),
                           _lib.ptr(b_bias), _lib.ptr(dg), _lib.ptr(dbeta), _lib.ptr(dab), _half_ptr(dab, H), 2 * H,
                           _lib.ptr(dA), _lib.ptr(ddt), _lib.ptr(dbb), _lib.ptr(ws), ws.numel(), ntok, H,
                           float(beta_scale), float(g_min), _lib.dtype_code(ab.dtype), _lib.stream_ptr(ab.device))
    _lib.check(rc, "gdn_gates_bwd")
    return dab, dA, ddt, dbb


@gdn_gates_ab_bwd.register_fake
def _(ab, A_log, dt_bias, b_bias, dg, dbeta, beta_scale, g_min):
    H = ab.shape[-1] // 2
    f32 = dict(dtype=torch.float32)
    return torch.empty_like(ab), ab.new_empty(H, **f32), ab.new_empty(H, **f32), ab.new_empty(H, **f32)


def _gates_ab_setup(ctx, inputs, output):
    ab, A_log, dt_bias, b_bias, beta_scale, g_min = inputs
    ctx.save_for_backward(ab, A_log, dt_bias, b_bias)
    ctx.beta_scale, ctx.g_min = beta_scale, g_min
    ctx.set_materialize_grads(True)


def _gates_ab_backward(ctx, dg, dbeta):
    ab, A_log, dt_bias, b_bias = ctx.saved_tensors
    dab, dA, ddt, dbb = gdn_gates_ab_bwd(ab, A_log, dt_bias, b_bias, dg, dbeta, ctx.beta_scale, ctx.g_min)
    return (dab, dA.to(A_log.dtype), None if dt_bias is None else ddt.to(dt_bias.dtype),
            None if b_bias is None else dbb.to(b_bias.dtype), None, None)


gdn_gates_ab.register_autograd(_gates_ab_backward, setup_context=_gates_ab_setup)


# ------------------------------------------------------------------------------------------- cross entropy
# Forward + backward of the cross-entropy in one pass, in place on a logits chunk (fla's cross_entropy_fwd +
# cross_entropy_bwd(inplace_backward=True) in archbench/fused_ce.py:33-45).
@torch.library.custom_op("archbench_amd::cross_entropy_fwd_bwd_", mutates_args=("logits",))
def cross_entropy_fwd_bwd_(logits: Tensor, target: Tensor, dloss: Optional[Tensor],
                           ignore_index: int) -> tuple[Tensor, Tensor]:
    """(loss per row fp32, lse per row fp32); logits [N, V] become dloss * (softmax - onehot)."""
    _require_gpu(logits, target, dloss)
    if logits.dim() != 2 or target.shape != logits.shape[:1]:
        raise ValueError(f"logits must be [N, V] and target [N], got {tuple(logits.shape)}, {tuple(target.shape)}")
    if logits.stride(1) != 1 or logits.data_ptr() % 16:
        raise ValueError("logits rows must be contiguous and 16-byte aligned (updated in place)")
    N, V = logits.shape
    lib = _lib.load()
    target = _arg(target, torch.int64)
    dloss = _arg(dloss, torch.float32)
    loss = torch.empty(N, dtype=torch.float32, device=logits.device)
    lse = torch.empty(N, dtype=torch.float32, device=logits.device)
    rc = lib.gdn_cross_entropy_fwd_bwd(_lib.ptr(logits), _lib.ptr(target), _lib.ptr(loss), _lib.ptr(lse),
                                       _lib.ptr(dloss), N, V, logits.stride(0), int(ignore_index),
                                       _lib.dtype_code(logits.dtype), _lib.stream_ptr(logits.device))
    _lib.check(rc, "gdn_cross_entropy_fwd_bwd")
    return loss, lse


@cross_entropy_fwd_bwd_.register_fake
def _(logits, target, dloss, ignore_index):
    N = logits.shape[0]
    return logits.new_empty(N, dtype=torch.float32), logits.new_empty(N, dtype=torch.float32)


# ------------------------------------------------------------------------------------------------- decode step
@torch.library.custom_op("archbench_amd::gdn_recurrent_step", mutates_args=("state",))
def _recurrent_step(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state: Tensor,
                    scale: float) -> Tensor:
    _require_gpu(q, k, v, g, beta, state)
    if q.dim() != 3 or k.shape != q.shape or v.dim() != 3 or tuple(v.shape[:2]) != tuple(q.shape[:2]):
        raise ValueError(f"decode step takes q, k [B, H, K] and v [B, H, V], got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, H, K = q.shape
    V = v.shape[-1]
    if tuple(g.shape) != (B, H) or tuple(beta.shape) != (B, H):
        raise ValueError(f"g and beta must be [B, H] = {(B, H)}")
    if tuple(state.shape) != (B, H, K, V) or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError(f"state must be a contiguous fp32 [B, H, K, V] = {(B, H, K, V)} tensor")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    lib = _lib.load()
    q, k, v = _arg(q), _arg(k), _arg(v)
    g, beta = _arg(g, torch.float32), _arg(beta, torch.float32)
    o = torch.empty(B, H, V, dtype=q.dtype, device=q.device)
    rc = lib.gdn_recurrent_step(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
                                _lib.ptr(state), _lib.ptr(o), B, H, K, V, float(scale), _lib.dtype_code(q.dtype),
                                _lib.stream_ptr(q.device))
    _lib.check(rc, "gdn_recurrent_step")
    return o


@_recurrent_step.register_fake
def _(q, k, v, g, beta, state, scale):
    B, H, _ = q.shape
    return q.new_empty(B, H, v.shape[-1])


# ----------------------------------------------------------------------------------------------- public API
def _l2norm(x: Tensor) -> Tensor:
    """F.normalize over the last dimension (eps 1e-12) on the HIP row-norm kernel."""
    return l2norm(x, 1e-12, 1.0)


def chunk_gated_delta_rule(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, scale: float | None = None,
                           initial_state: Tensor | None = None, output_final_state: bool = False,
                           use_qk_l2norm_in_kernel: bool = False, cu_seqlens: Tensor | None = None,
                           head_first: bool = False):
    """fla-compatible chunkwise gated delta rule: returns (o [B,T,H,V], final_state [B,H,K,V] fp32 or None).

    q, k [B,T,H,K]; v [B,T,H,V] (bf16 or fp32, shared dtype); g (natural-log decay) and beta [B,T,H];
    scale defaults to K**-0.5 (fla's default); differentiable w.r.t. q, k, v, g, beta and initial_state.
    """
    if head_first:
        raise ValueError("head_first=True layouts are not supported; pass [B, T, H, *] tensors")
    if cu_seqlens is not None:
        raise ValueError("variable-length packing (cu_seqlens) is not supported")
    if use_qk_l2norm_in_kernel:
        q, k = _l2norm(q), _l2norm(k)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    if _fp32_token_route(q, v):
        return _gdn_token_scan(q, k, v, g, beta, float(scale), initial_state, output_final_state)
    if _use_stash(q, k, v, g, beta, initial_state):
        o, hT, _ = chunk_fwd_stash(q, k, v, g, beta, initial_state, float(scale))
    else:
        o, hT = chunk_fwd(q, k, v, g, beta, initial_state, float(scale))
    return o, (hT if output_final_state else None)


_TOKEN_ROUTE_WARNED = [False]


def _fp32_token_route(q: Tensor, v: Tensor) -> bool:
    """fp32 inputs at a head size the fp32 chunk kernels are not compiled for, which the exact token scan covers."""
    if q.dtype != torch.float32 or not q.is_cuda or q.dim() != 4 or v.dim() != 4:
        return False
    K, V = q.shape[-1], v.shape[-1]
    return not _lib.supported("chunk", K, V, torch.float32) and K in (64, 128)


def _gdn_token_scan(q, k, v, g, beta, scale, initial_state, output_final_state):
    """The gated delta rule in fp32 where no fp32 chunk kernel is compiled: the exact token scan with write vector
    u = beta k and log-decay g (S <- e^g S + beta (v - e^g S k) k^T is the scan's recurrence at that u); exact to
    fp32 rounding and much slower than the bf16 chunk kernels, which the trainer's bf16 autocast selects."""
    if not _TOKEN_ROUTE_WARNED[0]:
        _TOKEN_ROUTE_WARNED[0] = True
        warnings.warn(f"chunk_gated_delta_rule: fp32 q/k/v at K={q.shape[-1]}, V={v.shape[-1]} run the exact fp32 "
                      "token scan (no fp32 chunk kernels at this size); bf16 inputs (e.g. under "
                      "torch.autocast(dtype=torch.bfloat16)) run the chunk kernels, many times faster",
                      UserWarning, stacklevel=3)
    u = beta.float()[..., None] * k
    y, _, _, hT = nsgdn_token_fwd(q * scale, k, u, v, g.float(), initial_state, bool(output_final_state))
    return y, (hT if output_final_state else None)


def recurrent_step(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor, state: Tensor,
                   scale: float | None = None) -> Tensor:
    """One decode step on [B,H,*] inputs; ``state`` (fp32 [B,H,K,V]) is updated in place; returns o [B,H,V]."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    return _recurrent_step(q, k, v, g, beta, state, float(scale))


def _owns_state(state: Tensor | None, B: int, H: int, K: int, V: int) -> bool:
    """True if ``state`` can be advanced in place: a contiguous fp32 [B, H, K, V] tensor outside autograd."""
    return (state is not None and state.dtype == torch.float32 and state.is_contiguous()
            and tuple(state.shape) == (B, H, K, V) and not state.requires_grad)


def fused_recurrent_gated_delta_rule(q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor,
                                     scale: float | None = None, initial_state: Tensor | None = None,
                                     output_final_state: bool = False, use_qk_l2norm_in_kernel: bool = False,
                                     inplace_final_state: bool = False):
    """fla-compatible recurrent entry point.  T = 1 without grad (decode) runs the single-token step kernel
    where it is compiled for (K, V) and the chunk kernels elsewhere; longer inputs run the chunk kernels, which
    compute the same recurrence.

    With ``inplace_final_state`` and an ``initial_state`` that is a contiguous fp32 [B, H, K, V] tensor, that
    tensor is advanced in place and returned as the final state (one read and one write of the state per step;
    fla's fused recurrent kernel offers the same flag).  Otherwise the initial state is left untouched and the
    final state is a new tensor."""
    if use_qk_l2norm_in_kernel:
        q, k = _l2norm(q), _l2norm(k)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    B, T, H, K = q.shape
    V = v.shape[-1]
    inplace = inplace_final_state and _owns_state(initial_state, B, H, K, V)
    if T == 1 and not torch.is_grad_enabled() and _lib.supported("step", K, V, q.dtype):
        if inplace:
            state = initial_state
        elif initial_state is None:
            state = torch.zeros(B, H, K, V, dtype=torch.float32, device=q.device)
        else:
            state = initial_state.float().clone().contiguous()
        o = _recurrent_step(q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0], state, float(scale))
        return o[:, None], (state if output_final_state or inplace else None)
    o, hT = chunk_gated_delta_rule(q, k, v, g, beta, scale, initial_state, output_final_state or inplace)
    if inplace:
        with torch.no_grad():
            initial_state.copy_(hT)
        hT = initial_state
    return o, hT
