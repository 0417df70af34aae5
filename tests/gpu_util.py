"""Helpers shared by the GPU parity tests: seeded inputs on the device and error metrics."""

import sys

import torch

from archbench_amd.synthetic import make_inputs


def banner(msg: str) -> None:
    """Name the case before a GPU step, flushed, so a failing run says what it was doing."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def device_inputs(B, T, H, K, V, dtype, seed=0, g_shift=4.0, h0_std=None, with_do=False):
    """Returns (host fp32 inputs rounded through ``dtype``, device inputs).  The oracle runs on the rounded
    values, so the comparison measures the kernels, not the input cast."""
    x = make_inputs(B, T, H, K, V, seed=seed, g_shift=g_shift, h0_std=h0_std, with_do=with_do)
    r = lambda t: None if t is None else t.to(dtype).float()
    host = type(x)(r(x.q), r(x.k), r(x.v), x.g, x.beta, x.h0, r(x.do))
    dev = x.to("cuda", dtype)
    return host, dev


def assert_fp32_close(what: str, names, got, ref, tol: float) -> None:
    """fp32 bar: absolute max-abs error <= tol for every tensor; the achieved errors (and each reference's
    largest magnitude, for scale) are printed before the check."""
    errs = {n: (max_abs(a, b), b.abs().max().item()) for n, a, b in zip(names, got, ref) if b is not None}
    print(f"[fp32 max-abs] {what}: " + ", ".join(f"{n} {e:.2e} (|ref| {m:.3g})" for n, (e, m) in errs.items()),
          flush=True)
    bad = {n: e for n, (e, _) in errs.items() if not e <= tol}
    assert not bad, f"{what}: max-abs above {tol}: {bad}"
