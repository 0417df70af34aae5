"""ctypes binding of the C-ABI library libgdn_mi355x.so (declared in include/gdn_mi355x.h).

The library is the only compute path: if it is missing, every op raises instead of falling back to anything.
"""

from __future__ import annotations

import ctypes
import functools
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime the library binds to by soname)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgdn_mi355x.so")

GDN_OK, GDN_ERR_ARG, GDN_ERR_SHAPE, GDN_ERR_WORKSPACE, GDN_ERR_LAUNCH = 0, 1, 2, 3, 4
DTYPE_F32, DTYPE_BF16 = 0, 1

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_i64 = ctypes.c_int64

# name -> (restype, argtypes); must list every function include/gdn_mi355x.h declares
SIGNATURES = {
    "gdn_version": (_i, []),
    "gdn_last_error": (ctypes.c_char_p, []),
    "gdn_supported": (_i, [_i, _i, _i, _i]),
    "gdn_chunk_fwd_ws_bytes": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "gdn_chunk_bwd_ws_bytes": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "gdn_chunk_fwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _i, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_chunk_bwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz,
                           _i, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_chunk_fwd_noalloc": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_chunk_stash_bytes": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "gdn_nsgdn_stash_bytes": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "gdn_chunk_fwd_stash": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _i, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_chunk_bwd_stashed": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p, _sz,
                                   _i, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_nsgdn_chunk_fwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _i, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_nsgdn_chunk_bwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p, _sz,
                                 _i, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_recurrent_step": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _i, _p]),
    "gdn_short_conv_fwd": (_i, [_p, _i64, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "gdn_short_conv_bwd_ws_bytes": (_i, [_i, _i, _i, _i, ctypes.POINTER(_sz)]),
    "gdn_short_conv_bwd": (_i, [_p, _i64, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _sz, _i, _i, _i, _i, _i, _i,
                                _p]),
    "gdn_gated_rmsnorm_fwd": (_i, [_p, _p, _i64, _i, _p, _p, _i64, _i, _f, _i, _p]),
    "gdn_gated_rmsnorm_bwd_ws_bytes": (_i, [_i64, _i, ctypes.POINTER(_sz)]),
    "gdn_gated_rmsnorm_bwd": (_i, [_p, _p, _i64, _i, _p, _p, _p, _p, _p, _p, _sz, _i64, _i, _f, _i, _p]),
    "gdn_l2norm_fwd": (_i, [_p, _p, _i64, _i, _f, _f, _i, _p]),
    "gdn_l2norm_bwd": (_i, [_p, _p, _p, _i64, _i, _f, _f, _i, _p]),
    "gdn_gates_fwd": (_i, [_p, _p, _i64, _p, _p, _p, _p, _p, _i64, _i, _f, _f, _i, _p]),
    "gdn_gates_bwd_ws_bytes": (_i, [_i64, _i, ctypes.POINTER(_sz)]),
    "gdn_gates_bwd": (_i, [_p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _sz, _i64, _i, _f, _f,
                           _i, _p]),
    "gdn_cross_entropy_fwd_bwd": (_i, [_p, _p, _p, _p, _p, _i64, _i, _i64, _i64, _i, _p]),
    "gdn_write_direction_fwd": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "gdn_write_direction_bwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p]),
    "gdn_token_scan_sizes": (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(_sz), ctypes.POINTER(_sz), ctypes.POINTER(_i)]),
    "gdn_token_scan_fwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p, _i, _i, _i, _i, _i, _p]),
    "gdn_token_scan_bwd": (_i, [_p, _p, _p, _p, _p, _p, _sz, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _i, _i, _i,
                                _i, _i, _p]),
    "gdn_profile_enable": (_i, [_i]),
    "gdn_profile_read": (_i, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i), _i]),
    "gdn_profile_stage_name": (ctypes.c_char_p, [_i]),
}
PROFILE_STAGES = 23

_lock = threading.Lock()
_lib = None


class GDNLibraryError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise GDNLibraryError(
                    f"{LIB_PATH} is missing: build it with `python -m archbench_amd.build` (hipcc, gfx950). "
                    "The gated DeltaNet op has no other implementation.")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc == GDN_OK:
        return
    msg = load().gdn_last_error().decode(errors="replace")
    if rc in (GDN_ERR_ARG, GDN_ERR_SHAPE):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise ValueError(f"gated DeltaNet kernels take bfloat16 or float32 q/k/v, got {dt}")


def ptr(t: torch.Tensor | None):
    # the argtypes are c_void_p: ctypes converts the integer address (and None -> NULL) itself
    return None if t is None else t.data_ptr()


def stream_ptr(device: torch.device):
    return torch.cuda.current_stream(device).cuda_stream


# Workspaces (scratch that lives only for one call's kernels) are kept per (device, stream) and reused while large
# enough, instead of a torch.empty per call: the library's kernels on one stream run in order, so a later call on
# the same stream cannot overlap an earlier one's use.  A buffer that is too small is replaced (the caching
# allocator reuses the old block on that stream only after the work queued there).  Under CUDA / HIP graph capture
# every call allocates its own workspace from the graph's pool as before, so a captured graph never holds the
# address of a cached buffer that a later call could replace.  The cache holds, per stream, the largest workspace
# requested so far until the process ends (or release_workspaces()).
_ws_cache: dict = {}
_ws_lock = threading.Lock()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A uint8 device buffer of at least nbytes for one call's kernels on the current stream of `device`."""
    stream = torch.cuda.current_stream(device)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    key = (stream.device_index, stream.cuda_stream)
    with _ws_lock:
        buf = _ws_cache.get(key)
        if buf is None or buf.numel() < nbytes:
            _ws_cache.pop(key, None)
            buf = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
            _ws_cache[key] = buf
        return buf


def release_workspaces() -> None:
    """Drop the cached workspaces (their memory returns to PyTorch's caching allocator)."""
    with _ws_lock:
        _ws_cache.clear()


def supported(op: str, K: int, V: int, dtype: torch.dtype) -> bool:
    return bool(load().gdn_supported({"chunk": 0, "step": 1}[op], K, V, dtype_code(dtype)))


# The size queries are pure functions of the shape and the device (the C side reads its CU count), so their results
# are cached per device.
@functools.lru_cache(maxsize=1024)
def _ws_bytes(kind: str, B: int, T: int, H: int, K: int, V: int, dtype: torch.dtype, dev: int) -> int:
    out = _sz(0)
    fn = load().gdn_chunk_fwd_ws_bytes if kind == "fwd" else load().gdn_chunk_bwd_ws_bytes
    check(fn(B, T, H, K, V, dtype_code(dtype), ctypes.byref(out)), f"gdn_chunk_{kind}_ws_bytes")
    return out.value


def ws_bytes(kind: str, B: int, T: int, H: int, K: int, V: int, dtype: torch.dtype) -> int:
    return _ws_bytes(kind, B, T, H, K, V, dtype, _device_index())


def _device_index() -> int:
    return torch.cuda.current_device() if torch.cuda.is_available() else -1


def stash_bytes(B: int, T: int, H: int, K: int, V: int, dtype: torch.dtype, nsgdn: bool = False) -> tuple[int, int]:
    """(stash bytes for gdn_chunk_fwd_stash, workspace bytes for gdn_chunk_bwd_stashed); with nsgdn, the sizes of
    the separate-write-key pair gdn_nsgdn_chunk_fwd / _bwd."""
    return _stash_bytes(B, T, H, K, V, dtype, nsgdn, _device_index())


@functools.lru_cache(maxsize=1024)
def _stash_bytes(B: int, T: int, H: int, K: int, V: int, dtype: torch.dtype, nsgdn: bool,
                 dev: int) -> tuple[int, int]:
    st, ws = _sz(0), _sz(0)
    fn = load().gdn_nsgdn_stash_bytes if nsgdn else load().gdn_chunk_stash_bytes
    check(fn(B, T, H, K, V, dtype_code(dtype), ctypes.byref(st), ctypes.byref(ws)),
          "gdn_nsgdn_stash_bytes" if nsgdn else "gdn_chunk_stash_bytes")
    return st.value, ws.value


def conv_ws_bytes(B: int, T: int, D: int, W: int) -> int:
    out = _sz(0)
    check(load().gdn_short_conv_bwd_ws_bytes(B, T, D, W, ctypes.byref(out)), "gdn_short_conv_bwd_ws_bytes")
    return out.value


def norm_ws_bytes(rows: int, dim: int) -> int:
    out = _sz(0)
    check(load().gdn_gated_rmsnorm_bwd_ws_bytes(rows, dim, ctypes.byref(out)), "gdn_gated_rmsnorm_bwd_ws_bytes")
    return out.value


def gates_ws_bytes(ntok: int, H: int) -> int:
    out = _sz(0)
    check(load().gdn_gates_bwd_ws_bytes(ntok, H, ctypes.byref(out)), "gdn_gates_bwd_ws_bytes")
    return out.value


class StageTimer:
    """Per-kernel-stage timing with events recorded by the library on the launch stream.

        with StageTimer() as st:
            ...  # gdn calls
        st.result  # {stage_name: (total_ms, launches)}
    """

    def __enter__(self):
        load().gdn_profile_enable(1)
        return self

    def __exit__(self, *exc):
        lib = load()
        ms = (ctypes.c_double * PROFILE_STAGES)()
        n = (_i * PROFILE_STAGES)()
        rc = lib.gdn_profile_read(ms, n, PROFILE_STAGES)
        lib.gdn_profile_enable(0)
        check(rc, "gdn_profile_read")
        self.result = {lib.gdn_profile_stage_name(i).decode(): (ms[i], n[i]) for i in range(PROFILE_STAGES) if n[i]}
        return False
