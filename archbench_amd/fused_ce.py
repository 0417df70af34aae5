"""Chunked linear + cross-entropy that never materialises the full (N, V) logits, on MI355X.

Same interface and arithmetic as archbench/fused_ce.py:20-57 (``fused_linear_cross_entropy(x, target, weight,
num_chunks=8, ignore_index=-100)`` -> mean token cross-entropy; the forward computes every gradient and the
backward only scales them).  Per chunk of rows: logits = x W^T and the two gradient products dx = dlogits W,
dW += dlogits^T x (fp32 accumulation) are plain library GEMMs (hipBLASLt through torch.mm / addmm); between them
one HIP kernel (``ops.cross_entropy_fwd_bwd_``) computes each row's loss and overwrites the logits with
dloss * (softmax - onehot), reading and writing the chunk once.  With 288 GB of HBM a chunk of 2048 rows x 50304
classes (206 MB in bf16) is cheap to hold, so the logits are kept rather than recomputed -- and even one chunk
for 32768 tokens (3.3 GB): with ``num_chunks=1`` the weight gradient comes straight out of one bf16-output GEMM
instead of fp32 accumulation across chunks, the fastest configuration on MI355X.
"""

from __future__ import annotations

import torch

from . import _lib, ops


def fused_ce_available() -> bool:
    """True when the HIP library is built (the kernel path has no fallback)."""
    try:
        _lib.load()
    except _lib.GDNLibraryError:
        return False
    return True


class _FusedLinearCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, target, weight, num_chunks: int, ignore_index: int):
        N, _ = x.shape
        C = -(-N // num_chunks)
        total = target.ne(ignore_index).sum().clamp_min(1)
        dloss = total.float().reciprocal().reshape(1)  # device scalar: no host sync
        loss_rows = torch.empty(N, device=x.device, dtype=torch.float32)
        dx = torch.empty_like(x)
        if C >= N:
            # one chunk: dW needs no accumulation across chunks, so the GEMM writes it in the weight's dtype
            # directly (fp32 accumulation inside, one rounding -- where the chunked path rounds at the end)
            logits = x @ weight.t()
            loss_rows = ops.cross_entropy_fwd_bwd_(logits, target, dloss, ignore_index)[0]
            dx = logits @ weight
            dw = logits.t() @ x
        else:
            dw = torch.zeros(weight.shape, device=x.device, dtype=torch.float32)
            for s in range(0, N, C):
                e = min(s + C, N)
                c_x = x[s:e]
                logits = c_x @ weight.t()
                loss_rows[s:e] = ops.cross_entropy_fwd_bwd_(logits, target[s:e], dloss, ignore_index)[0]
                dx[s:e] = logits @ weight
                dw = torch.addmm(dw, logits.t(), c_x, out_dtype=torch.float32)
        ctx.save_for_backward(dx, dw.to(weight.dtype))
        return loss_rows.sum() / total

    @staticmethod
    def backward(ctx, dout):
        dx, dw = ctx.saved_tensors
        return dx * dout, None, dw * dout, None, None


def fused_linear_cross_entropy(x, target, weight, num_chunks: int = 8, ignore_index: int = -100):
    """x (B, T, H), target (B, T), weight (V, H) -> mean token cross-entropy (fused_ce.py:55-57)."""
    return _FusedLinearCE.apply(x.reshape(-1, x.shape[-1]), target.reshape(-1), weight, num_chunks, ignore_index)
