#!/usr/bin/env python3
"""Gated DeltaNet benchmark on one MI355X.

Headline (one JSON line on stdout): chunk forward + backward of the GDN op at B=8, T=4096, H=16, K=V=128, bf16
inputs with fp32 state/accumulation, synthetic seeded data resident in HBM.  One step = one training forward
call (gdn_chunk_fwd_stash: o and hT, keeping the per-chunk states for the backward, as autograd does) and one
backward call (gdn_chunk_bwd_stashed: every gradient, dq, dk, dv, dg, dbeta).  tokens/s = B*T / step time.
The recompute path (gdn_chunk_fwd + gdn_chunk_bwd, no stash) is timed beside it as recompute_ms_per_step.

Also reported in the same line:
  roofline      the training step (its four kernels: chunk factors, forward sweep, reverse sweep, gradient kernel)
                on the workload's own algorithmic basis: 3 * F_fwd FLOPs and 2,840 bytes per token-head (q, k, v, g,
                beta read and o written by the forward; q, k, v, dO, g, beta read and dq, dk, dv, dg, dbeta written by
                the backward, at K = V = 128 bf16).  Its intensity (190 FLOP/B) is below the ridge (2.5 PFLOP/s /
                8 TB/s = 312), so HBM bounds it: achieved = algorithmic bytes / step time (HIP events on the launch
                stream over the timed loop), against 8 TB/s; mfma_frac and the MFMA ceiling that bound allows
                (190 FLOP/B x 8 TB/s / 2.5 PFLOP/s) are given beside it.  traffic = the HBM bytes the step's kernels
                actually move (rocprofv3 FETCH_SIZE / WRITE_SIZE per kernel, profiles/hbm_traffic.json), and
                traffic_ratio = traffic / algorithmic bytes (the bytes the design moves beyond the minimum);
  kernels       each kernel of the step: time per launch (HIP events around each launch, a separate loop),
                its design bytes (every input and workspace buffer read once, every output written once) and
                design FLOPs (the dense MFMA products it performs), measured traffic, and, where the profile holds
                them, rocprofv3's MfmaUtil (MFMA busy cycles / (active cycles x SIMDs)) and executed bf16 MFMA FLOPs;
  mfma_frac     the whole step at the workload's algorithmic count 3 * F_fwd per token-head,
                F_fwd = 2C(3K + 2V) + 6KV (C = 64);
  fwd_only      forward alone at B=8, T=2048, H=8, K=V=128 (% of the bf16 MFMA peak);
  long_context  forward + backward at B=1, T=16384, H=16, K=128, V=256, nonzero initial state, slow decay
                (g = logsigmoid(N(0,1) + 6)), the training pair with dh0; tokens/s and % of the bf16 MFMA peak at
                3 * F_fwd(128, 256) per token-head;
  nsgdn         the separate-write-key training pair (nsgdn_chunk_fwd + nsgdn_chunk_bwd: u != beta k, the n-step
                family's write vectors) at archbench's nsgdn layer shape (head_dim 128, expand_v 2, 4 heads,
                seq_len 1024: K=128, V=256, H=4, T=1024) with B=64; tokens/s and % of the bf16 MFMA peak at
                3 * F_fwd(128, 256) per token-head;
  gdn_layer     the drop-in `gdn` mixer as archbench's model builds it for configs/65m/gdn.yaml (d_model 512,
                4 heads, head_dim 128, expand_v 2, gate, short conv 4), fed fp32 hidden states under bf16 autocast as
                the trainer runs Block.forward, at B=64, T=1024: forward + backward of the whole layer (projections
                on hipBLASLt, conv, gates, the op, gated RMSNorm, output projection; gradients unset before each
                step, as after zero_grad(set_to_none=True)), tokens/s by the host clock and the step's GPU span by
                events, with the library's kernels' share of that span (the rest: PyTorch's kernels, mostly the
                projection GEMMs, and any time the GPU waits for the host);
  nsgdn_layer   the same for archbench's `nsgdn` mixer (configs/65m/nsgdn.yaml: n_steps 2, lam 1, the same
                projections, conv and norm around the separate-write-key chunk kernels, plus the write direction);
  token_scan    the exact fp32 token scan of the n-step family (the reference's scan_impl "triton" / "ref") at
                B=16, T=1024, H=4, K=128, V=256: the forward + backward op pair by the host clock (tokens/s), and
                its two scan kernels by events (an exactness path, not a fast one: the chunk pair does the same
                tokens in a fraction of the time);
  decode_step   one recurrent decode step at B=256, H=16, K=V=128 with the fp32 state updated in place
                (HBM GB/s against 8 TB/s);
  short_conv    the causal depthwise conv (kernel 4) + SiLU in front of the op at the layer's shape, B=8, T=4096,
                D = H*K = 2048 channels, bf16: with the per-head (128-channel) L2 normalisation of q and k, and
                without (v); forward and backward kernel times, HBM GB/s against 8 TB/s on the algorithmic bytes
                (forward: x read, y written; backward: x and dy read, dx written);
  gated_rmsnorm the output norm(o) * silu(gate) over B*T*H = 524288 rows of DV = 128, bf16, forward and backward
                (HBM GB/s: forward reads x and gate, writes y; backward reads x, gate, dy, writes dx, dgate);
  gates         g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) over B*T = 32768 tokens x H = 16;
  fused_linear_ce  archbench's chunked linear + cross-entropy (fused_ce.py) at N = 8*4096 tokens, d_model 1024,
                vocabulary 50304, bf16, one chunk: the GEMMs are hipBLASLt, the per-row loss + in-place gradient is
                the HIP kernel (HBM GB/s on one read and one write of the logits);
  cpu_baseline  the CPU oracle (fp32 token recurrence + exact reverse-time backward) timed on this host's
                cores on the full headline shape (about 20 s of CPU work at ~2e3 tokens/s on 16 threads).
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

MFMA_BF16_PEAK = 2.5e15  # MI355X dense bf16 MFMA, FLOP/s
HBM_PEAK = 8.0e12        # MI355X HBM3E, B/s
C = 64
METRIC = "gated-DeltaNet fwd+bwd tokens/s (H16,d128,T4096) + % bf16 MFMA peak"


def f_fwd(K: int, V: int) -> int:
    """Algorithmic dense FLOPs per token-head of the chunk forward (the workload's counting convention)."""
    return 2 * C * (3 * K + 2 * V) + 6 * K * V


def stage_flops(stage: str, K: int, V: int) -> int:
    """Dense MFMA FLOPs per token-head that each kernel performs (C = 64 tokens per chunk; the 64 x 64 inverse
    of the chunk factors is not counted).  A product an (M x N) = (M x L)(L x N) counts 2 M N L, divided by the
    C tokens of its chunk."""
    return {
        "factors": 4 * C * K,                                # K K^T, Q K^T
        "fwd": 6 * K * V + 4 * C * V,                        # K S, Q S, K^T R; Tm Y, P R
        "fwd_stash": 6 * K * V + 4 * C * V,                  # the same, states and R also written
        "bwd_recompute": 4 * K * V + 2 * C * V,              # K S, K^T R; Tm Y
        "bwd_state": 6 * K * V + 4 * C * V,                  # K dS, Q^T dO, K^T Z; P^T dO, Tm^T dR
        "bwd_intra": 6 * K * V + 4 * C * V + 12 * C * K,     # dO S0^T, R dSC^T, dY S0^T; dO R^T, dY R^T;
                                                             # K K^T, Q K^T, dPm K, dPm^T Q, D K, D^T K
    }.get(stage, 0)


def stage_bytes(stage: str, K: int, V: int, es: int = 2, hstride: int = 2) -> int:
    """Design HBM bytes per token-head of each kernel: every input and workspace buffer read once, every output
    written once (q, k: es*K; v, o, dO, dv, R, dY: es*V; g, beta, G, dg, dbeta: 4; Tm, P: es*40 per token, their
    ten 16 x 16 blocks on and below the diagonal per 64 tokens; a
    chunk's state or state gradient: es*K*V/C per token, the stash keeping the state entering every hstride-th
    chunk: every second one in bf16 at V <= 128).  The second V-block workgroup's reads of q, k, Tm and P in the
    sweeps, which hit L2, count once."""
    qk, vv, st, tm = es * K, es * V, es * K * V // C, es * 10 * 256 // C
    sh = st // hstride
    return {
        "factors": 2 * qk + 8 + 2 * tm + 4,                  # q k g beta -> Tm P G
        "fwd": 2 * qk + vv + 8 + 2 * tm + vv,                # q k v beta G Tm P -> o
        "fwd_stash": 2 * qk + vv + 8 + 2 * tm + vv + sh + vv,  # ... -> o, states, R
        "bwd_recompute": qk + vv + 8 + tm + sh + vv,         # k v beta G Tm -> states, R
        "bwd_state": 2 * qk + vv + 8 + 2 * tm + st + vv,     # q k dO beta G Tm P -> dstates, dY
        "bwd_intra": 2 * qk + 2 * vv + 8 + sh + st + 2 * vv + 2 * qk + vv + 8,  # q k v dO beta G S0 dSC R dY ->
                                                                               # dq dk dv dg dbeta
    }.get(stage, 0)


def algo_bytes_step(K: int, V: int, es: int = 2) -> int:
    """Minimum HBM bytes per token-head of one training step (forward + backward) at the op boundary: the
    forward reads q, k, v, g, beta and writes o; the backward reads q, k, v, dO, g, beta and writes dq, dk, dv,
    dg, dbeta (2,840 bytes at K = V = 128 bf16)."""
    fwd = es * (2 * K + V) + 8 + es * V
    bwd = es * (2 * K + 2 * V) + 8 + es * (2 * K + V) + 8
    return fwd + bwd


def _profile_json(name: str) -> dict:
    """A profiles/ summary, if it was measured on these kernel sources (its "sources" digest equals this tree's);
    otherwise empty, so that no figure measured on other kernels is reported as this build's."""
    from archbench_amd.build import source_digest

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", name)
    try:
        with open(path) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        return {}
    if doc.get("sources") != source_digest():
        log(f"profiles/{name} was measured on other kernel sources ({doc.get('sources')}); not used")
        return {}
    return doc


def measured_traffic() -> dict:
    """HBM bytes per launch by stage, from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarised in
    profiles/hbm_traffic.json (calibrated on a copy of known size); empty if that file is absent."""
    return _profile_json("hbm_traffic.json").get("per_launch", {})


def measured_mfma() -> dict:
    """MfmaUtil and executed bf16 MFMA FLOPs per launch by stage, from the rocprofv3 counter run summarised in
    profiles/mfma_counters.json; empty if that file is absent."""
    return _profile_json("mfma_counters.json").get("per_launch", {})


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def timed_loop(fn, steps: int, warmup: int, torch, events: bool = False, collect: bool = True,
               settle_ms: float = 40.0):
    """Seconds per call of fn over `steps` calls after `warmup` untimed ones, by the host clock between two
    synchronisations; with events, also the GPU time between HIP events recorded on the current stream (the
    stream the library launches on) around the same calls: (host_s, event_s).

    Python's garbage collector is run before the warmup and kept off through the warmup and the timed region, as
    timeit does: a full collection late in this process takes about 80 ms (measured), and one falling among 20
    steps of a 2.6 ms layer step read as 6.3 ms per step.  Collecting before the warmup rather than between it and
    the timed steps also keeps the GPU from idling there: after some tens of milliseconds idle its clocks start
    from their idle state again, and the first 25 ms or so of a heavy load then run up to 30% slower.  With
    collect false the caller has already collected and disabled the collector (loops timed back to back).

    Before the warmup, fn is run untimed for about settle_ms of GPU time (0: not at all), so that a short step's
    timed calls fall after that transient rather than inside it."""
    if collect:
        gc.collect()
        gc.disable()
    try:
        if settle_ms > 0:
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            one = max(time.perf_counter() - t0, 1e-5)
            for _ in range(min(int(settle_ms * 1e-3 / one), 20000)):
                fn()
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        host = (time.perf_counter() - t0) / steps
    finally:
        if collect:
            gc.enable()
    return (host, e0.elapsed_time(e1) * 1e-3 / steps) if events else host


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(T: int) -> dict:
    """The oracle on this host's cores (kind 'port'): bounded sample of the headline shape."""
    import torch

    from archbench_amd.synthetic import make_inputs
    from oracle import gdn_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    B, H, K, V = 8, 16, 128, 128
    x = make_inputs(B, T, H, K, V, seed=0, with_do=True)
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < 10.0:  # whole passes, at least 10 s of CPU work
        O.recurrent_fwd(x.q, x.k, x.v, x.g, x.beta, 1.0, None, dtype=torch.float32)
        O.recurrent_bwd(x.q, x.k, x.v, x.g, x.beta, x.do, 1.0, None, None, ckpt=64, dtype=torch.float32)
        reps += 1
    dt = time.perf_counter() - t0
    return {"value": round(reps * B * T / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"B={B} T={T} H={H} K=V={K} fp32: token-recurrence forward + exact reverse-time backward "
                      f"(checkpoint every 64 tokens), {reps} pass(es) in {dt:.1f} s on {threads} threads of "
                      f"'{cpu_model()}'"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-sample-T", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default="all",
                    help="comma-separated workloads to run (all, train, fwd, long, decode, conv, norm, ce), for "
                         "profiling runs; the JSON line needs 'all' or 'train'")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="end with two device copies of 256 MiB (the known-size dispatch that calibrates rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    only = set(args.only.split(","))
    known = {"all", "train", "fwd", "long", "nsgdn", "layer", "nsgdn_layer", "token_scan", "decode", "conv", "norm",
             "ce"}
    if not only <= known:
        ap.error(f"--only: unknown workload(s) {sorted(only - known)}; choose from {sorted(known)}")
    want = lambda w: "all" in only or w in only
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures a single GPU: the gated DeltaNet op shards over batch and heads with no "
              "communication, and this build has no multi-GPU path. Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from archbench_amd import _lib, ops
    from archbench_amd.synthetic import make_inputs, make_step_inputs

    _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    out: dict = {}

    if want("train"):
        B, T, H, K, V = 8, 4096, 16, 128, 128
        log(f"headline fwd+bwd B={B} T={T} H={H} K={K} V={V} bf16: generating inputs")
        x = make_inputs(B, T, H, K, V, seed=0, with_do=True).to(dev, torch.bfloat16)

        def step():
            _, _, stash = ops.chunk_fwd_stash(x.q, x.k, x.v, x.g, x.beta, None, 1.0)
            ops.chunk_bwd_stashed(x.q, x.k, x.v, x.g, x.beta, None, x.do, None, stash, 1.0)

        def step_recompute():
            ops.chunk_fwd(x.q, x.k, x.v, x.g, x.beta, None, 1.0)
            ops.chunk_bwd(x.q, x.k, x.v, x.g, x.beta, None, x.do, None, 1.0)

        # The recompute path is timed first (same step counts) and the headline right after it, with no idle time in
        # between: the inputs are generated on the host, during which the GPU idles, and for about 25-30 ms after it
        # goes from idle to this load its clocks dip (per step 0.88 -> 1.09 -> 0.83 ms over the first 40 steps, by
        # HIP events), so the headline's timed steps would otherwise measure that transient rather than the
        # sustained rate.
        log(f"timing {args.steps} steps after {args.warmup} warmup (recompute path first)")
        # Collected once, before all three loops (the per-kernel stage timing follows at once too): a collection
        # between them would leave the GPU idle.
        gc.collect()
        gc.disable()
        try:
            sec_rc = timed_loop(step_recompute, args.steps, args.warmup, torch, collect=False, settle_ms=0)
            sec, sec_ev = timed_loop(step, args.steps, args.warmup, torch, events=True, collect=False, settle_ms=0)
            with _lib.StageTimer() as st:
                for _ in range(max(3, min(args.steps, 10))):
                    step()
        finally:
            gc.enable()
        tokens = B * T
        stages = {k: (ms / n, n) for k, (ms, n) in st.result.items()}
        call_flops = 3 * f_fwd(K, V) * B * T * H
        algo_bytes = algo_bytes_step(K, V) * B * T * H
        traffic_by_stage, mfma_by_stage = measured_traffic(), measured_mfma()
        step_stages = ("factors", "fwd_stash", "bwd_state", "bwd_intra")
        traffic = (sum(traffic_by_stage[k]["bytes"] for k in step_stages)
                   if all(k in traffic_by_stage for k in step_stages) else None)
        roof = {"kernel": "training step: chunk_factors + fwd_sweep<stash> + bwd_state + bwd_intra",
                "bound": "hbm", "achieved": round(algo_bytes / sec_ev / 1e9, 1), "peak": HBM_PEAK / 1e9,
                "unit": "GB/s", "frac": round(algo_bytes / sec_ev / HBM_PEAK, 4), "traffic": traffic,
                "algorithmic_bytes": algo_bytes,
                "traffic_ratio": None if traffic is None else round(traffic / algo_bytes, 3),
                "flops": call_flops, "intensity_flop_per_byte": round(call_flops / algo_bytes, 1),
                "step_ms_events": round(sec_ev * 1e3, 4),
                "mfma_frac": round(call_flops / sec_ev / MFMA_BF16_PEAK, 4),
                "mfma_ceiling_frac": round(call_flops / algo_bytes * HBM_PEAK / MFMA_BF16_PEAK, 4)}
        kernels = {}
        for k in step_stages:
            if k not in stages:
                continue
            ms = stages[k][0]
            fl, by = stage_flops(k, K, V) * B * T * H, stage_bytes(k, K, V) * B * T * H
            ent = {"ms": round(ms, 4), "design_flops": fl, "design_bytes": by,
                   "design_GB_per_s": round(by / (ms * 1e-3) / 1e9, 1),
                   "mfma_frac": round(fl / (ms * 1e-3) / MFMA_BF16_PEAK, 4)}
            if k in traffic_by_stage:
                tb = traffic_by_stage[k]["bytes"]
                ent.update({"traffic": tb, "traffic_GB_per_s": round(tb / (ms * 1e-3) / 1e9, 1),
                            "hbm_frac": round(tb / (ms * 1e-3) / HBM_PEAK, 4)})
            if k in mfma_by_stage:
                ent.update({kk: mfma_by_stage[k][kk] for kk in ("mfma_util", "executed_bf16_flops")
                            if kk in mfma_by_stage[k]})
            kernels[k] = ent
        out.update({
            "metric": METRIC, "value": round(tokens / sec, 1), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic",
            "config": {"workload": "gdn_chunk_fwd_bwd", "B": B, "T": T, "H": H, "K": K, "V": V, "chunk": C,
                       "scale": 1.0, "state": "fp32", "g_shift": 4.0},
            "mfma_frac": round(call_flops / sec / MFMA_BF16_PEAK, 4),
            "roofline": roof,
            "kernels": kernels,
            "stages_ms": {k: round(v[0], 4) for k, v in stages.items()},
            "recompute_ms_per_step": round(sec_rc * 1e3, 4),
        })
        log(f"fwd+bwd {sec * 1e3:.3f} ms/step, {tokens / sec:.3e} tokens/s; stages {out['stages_ms']}; "
            f"recompute path {sec_rc * 1e3:.3f} ms/step")
        del x
        torch.cuda.empty_cache()

    if want("fwd"):
        B, T, H, K, V = 8, 2048, 8, 128, 128
        log(f"forward only B={B} T={T} H={H} K={K} V={V} bf16")
        x = make_inputs(B, T, H, K, V, seed=0).to(dev, torch.bfloat16)
        sec, sec_ev = timed_loop(lambda: ops.chunk_fwd(x.q, x.k, x.v, x.g, x.beta, None, 1.0), args.steps,
                                 args.warmup, torch, events=True)
        out["fwd_only"] = {"workload": "gdn_chunk_fwd", "B": B, "T": T, "H": H, "K": K, "V": V,
                           "ms": round(sec * 1e3, 4), "ms_events": round(sec_ev * 1e3, 4),
                           "tokens_per_s": round(B * T / sec, 1),
                           "mfma_frac": round(f_fwd(K, V) * B * T * H / sec_ev / MFMA_BF16_PEAK, 4)}
        log(f"fwd {sec * 1e3:.3f} ms by the host clock, {sec_ev * 1e3:.3f} ms by events")
        del x
        torch.cuda.empty_cache()

    if want("long"):
        B, T, H, K, V = 1, 16384, 16, 128, 256
        log(f"long context fwd+bwd B={B} T={T} H={H} K={K} V={V} bf16, h0 ~ N(0, 0.1^2), g_shift 6")
        x = make_inputs(B, T, H, K, V, seed=0, g_shift=6.0, h0_std=0.1, with_do=True).to(dev, torch.bfloat16)
        dhT = torch.zeros(B, H, K, V, device=dev)

        def long_step():
            _, _, stash = ops.chunk_fwd_stash(x.q, x.k, x.v, x.g, x.beta, x.h0, 1.0)
            ops.chunk_bwd_stashed(x.q, x.k, x.v, x.g, x.beta, x.h0, x.do, dhT, stash, 1.0)

        n = max(5, min(args.steps, 20))
        sec, sec_ev = timed_loop(long_step, n, 2, torch, events=True)
        with _lib.StageTimer() as st:
            for _ in range(3):
                long_step()
        fl = 3 * f_fwd(K, V) * B * T * H
        out["long_context"] = {"workload": "gdn_chunk_fwd_bwd", "B": B, "T": T, "H": H, "K": K, "V": V,
                               "h0": "N(0, 0.1^2)", "g_shift": 6.0, "steps": n, "ms_per_step": round(sec * 1e3, 4),
                               "tokens_per_s": round(B * T / sec, 1),
                               "mfma_frac": round(fl / sec_ev / MFMA_BF16_PEAK, 4),
                               "stages_ms": {k: round(v[0] / v[1], 4) for k, v in st.result.items()}}
        log(f"long context {sec * 1e3:.3f} ms/step, {B * T / sec:.3e} tokens/s, "
            f"{out['long_context']['mfma_frac'] * 100:.1f}% of bf16 MFMA peak; "
            f"stages {out['long_context']['stages_ms']}")
        del x
        torch.cuda.empty_cache()

    if want("nsgdn"):
        B, T, H, K, V = 64, 1024, 4, 128, 256
        log(f"nsgdn training pair B={B} T={T} H={H} K={K} V={V} bf16 (separate write keys)")
        x = make_inputs(B, T, H, K, V, seed=0, with_do=True)
        gen = torch.Generator().manual_seed(1)
        u = (x.beta[..., None] * x.k + 0.05 * torch.randn(B, T, H, K, generator=gen)).to(dev, torch.bfloat16)
        q, k, v, dy = (t.to(dev, torch.bfloat16) for t in (x.q, x.k, x.v, x.do))
        la = x.g.to(dev)
        sc = K ** -0.5

        def nsgdn_step():
            _, _, stash = ops.nsgdn_chunk_fwd(q, k, u, v, la, None, sc)
            ops.nsgdn_chunk_bwd(q, k, u, v, la, None, dy, None, stash, sc)

        n = max(5, min(args.steps, 20))
        sec, sec_ev = timed_loop(nsgdn_step, n, 2, torch, events=True)
        with _lib.StageTimer() as st:
            for _ in range(3):
                nsgdn_step()
        fl = 3 * f_fwd(K, V) * B * T * H
        out["nsgdn"] = {"workload": "nsgdn_chunk_fwd_bwd", "B": B, "T": T, "H": H, "K": K, "V": V, "steps": n,
                        "ms_per_step": round(sec * 1e3, 4), "tokens_per_s": round(B * T / sec, 1),
                        "mfma_frac": round(fl / sec_ev / MFMA_BF16_PEAK, 4),
                        "stages_ms": {k_: round(v_[0] / v_[1], 4) for k_, v_ in st.result.items()}}
        log(f"nsgdn {sec * 1e3:.3f} ms/step, {B * T / sec:.3e} tokens/s, "
            f"{out['nsgdn']['mfma_frac'] * 100:.1f}% of bf16 MFMA peak; stages {out['nsgdn']['stages_ms']}")
        del x, q, k, u, v, dy, la
        torch.cuda.empty_cache()

    if want("layer") or want("nsgdn_layer"):
        from archbench_amd import layers

        B, T, D, nh = 64, 1024, 512, 4
        mixers = []
        if want("layer"):
            mixers.append(("gdn", "gdn_layer", dict(use_gate=True, use_short_conv=True, conv_size=4)))
        if want("nsgdn_layer"):
            mixers.append(("nsgdn", "nsgdn_layer",
                           dict(n_steps=2, lam=1.0, use_gate=True, use_short_conv=True, conv_size=4)))
        for arch, key, cfg in mixers:
            log(f"{arch} layer (configs/65m/{arch}.yaml: d_model {D}, {nh} heads, K=128, V=256) B={B} T={T}, fp32 "
                f"input under bf16 autocast, forward + backward")
            torch.manual_seed(0)
            m = layers.build_mixer(arch, D, 0, 10, num_heads=nh, head_dim=128, expand_v=2.0, **cfg).to(dev)
            xin = torch.randn(B, T, D, device=dev, generator=torch.Generator(dev).manual_seed(1)).requires_grad_()
            gy = torch.randn(B, T, D, device=dev, generator=torch.Generator(dev).manual_seed(2))

            params = list(m.parameters())

            def layer_step():
                # gradients start unset, as after the trainer's zero_grad(set_to_none=True); the input's stands
                # for the gradient the block passes on, which the model does not accumulate across steps
                xin.grad = None
                for p_ in params:
                    p_.grad = None
                with torch.autocast("cuda", dtype=torch.bfloat16):
                    y = m(xin)
                y.backward(gy)

            n = max(5, min(args.steps, 20))
            # warmup >= 5: the first steps of a mixer pay one-time costs (hipBLASLt's first calls at each GEMM
            # shape, the caching allocator's growth) that are not the step's
            sec, sec_ev = timed_loop(layer_step, n, max(5, args.warmup), torch, events=True)
            with _lib.StageTimer() as st:
                for _ in range(3):
                    layer_step()
            lib_ms = sum(v_[0] for v_ in st.result.values()) / 3
            ev_ms = sec_ev * 1e3
            out[key] = {"workload": f"{arch} mixer fwd+bwd (configs/65m/{arch}.yaml)", "B": B, "T": T,
                        "d_model": D, "heads": nh, "K": 128, "V": 256, "steps": n,
                        "ms_per_step": round(sec * 1e3, 4), "ms_per_step_events": round(ev_ms, 4),
                        "tokens_per_s": round(B * T / sec, 1),
                        "library_kernels_ms": round(lib_ms, 4),
                        # the GPU span of a step less this library's kernels: PyTorch's kernels (the projection
                        # GEMMs on hipBLASLt, casts, gradient sums) and any time the GPU waits for the host
                        "other_ms": round(ev_ms - lib_ms, 4),
                        "library_share": round(lib_ms / ev_ms, 4),
                        "stages_ms": {k_: round(v_[0] / 3, 4) for k_, v_ in st.result.items()}}
            log(f"{arch} layer {sec * 1e3:.3f} ms/step by the host clock, {ev_ms:.3f} ms by events, "
                f"{B * T / sec:.3e} tokens/s; library kernels {lib_ms:.3f} ms per step {out[key]['stages_ms']}")
            del m, xin, gy
            torch.cuda.empty_cache()

    if want("token_scan"):
        B, T, H, K, V = 16, 1024, 4, 128, 256
        log(f"exact fp32 token scan B={B} T={T} H={H} K={K} V={V}")
        gen = torch.Generator(device=dev).manual_seed(0)
        qt = torch.nn.functional.normalize(torch.randn(B, T, H, K, device=dev, generator=gen), dim=-1) * K ** -0.5
        kt = torch.nn.functional.normalize(torch.randn(B, T, H, K, device=dev, generator=gen), dim=-1)
        ut, vt = kt * 0.5, torch.randn(B, T, H, V, device=dev, generator=gen)
        lat = -torch.nn.functional.softplus(torch.randn(B, T, H, device=dev, generator=gen))
        dyt = torch.randn(B, T, H, V, device=dev, generator=gen)
        def scan_pair():
            _, r1, st1, _ = ops.nsgdn_token_fwd(qt, kt, ut, vt, lat, None, False)
            ops.nsgdn_token_bwd(qt, kt, ut, lat, r1, st1, dyt, None, False)

        # the op pair as called (the backward's host side also sums the per-block partial rows of dq, du, dk
        # and dla): host clock over whole calls; the two scan kernels by events beside it
        sec = timed_loop(scan_pair, 5, 1, torch)
        with _lib.StageTimer() as st:
            for _ in range(2):
                scan_pair()
        f_ms = st.result["token_scan_fwd"][0] / 2
        b_ms = st.result["token_scan_bwd"][0] / 2
        out["token_scan"] = {"workload": "nsgdn exact fp32 token scan (scan_impl triton/ref)", "B": B, "T": T, "H": H,
                             "K": K, "V": V, "ms_per_step": round(sec * 1e3, 3), "fwd_kernel_ms": round(f_ms, 3),
                             "bwd_kernel_ms": round(b_ms, 3), "tokens_per_s": round(B * T / sec, 1)}
        log(f"token scan fwd+bwd {sec * 1e3:.3f} ms per call pair; kernels fwd {f_ms:.3f} ms, bwd {b_ms:.3f} ms")
        del qt, kt, ut, vt, lat, dyt
        torch.cuda.empty_cache()

    if want("decode"):
        B, H, K, V = 256, 16, 128, 128
        log(f"decode step B={B} H={H} K={K} V={V} (fp32 state in place)")
        q, k, v, g, b, S = make_step_inputs(B, H, K, V)
        q, k, v = (t.to(dev, torch.bfloat16) for t in (q, k, v))
        g, b, S = g.to(dev), b.to(dev), S.to(dev)
        n_steps = max(args.steps, 50)
        sec = timed_loop(lambda: ops.recurrent_step(q, k, v, g, b, S, 1.0), n_steps, args.warmup, torch)
        with _lib.StageTimer() as st:
            for _ in range(20):
                ops.recurrent_step(q, k, v, g, b, S, 1.0)
        kern_ms = st.result["step"][0] / st.result["step"][1]
        nbytes = 2 * B * H * K * V * 4 + B * H * (2 * K + 2 * V) * 2 + B * H * 2 * 4
        out["decode_step"] = {"workload": "gdn_recurrent_step", "B": B, "H": H, "K": K, "V": V,
                              "traffic": measured_traffic().get("step", {}).get("bytes"),
                              "us_per_step": round(sec * 1e6, 2), "kernel_us": round(kern_ms * 1e3, 2),
                              "bytes_per_step": nbytes, "GB_per_s": round(nbytes / (kern_ms * 1e-3) / 1e9, 1),
                              "hbm_frac": round(nbytes / (kern_ms * 1e-3) / HBM_PEAK, 4),
                              "tokens_per_s": round(B / sec, 1)}
        log(f"decode kernel {kern_ms * 1e3:.2f} us, {out['decode_step']['GB_per_s']} GB/s")

    if want("conv"):
        B, T, D = 8, 4096, 2048
        log(f"short conv B={B} T={T} D={D} kernel 4 bf16")
        gen = torch.Generator(device=dev).manual_seed(0)
        xc = torch.randn(B, T, D, device=dev, generator=gen).to(torch.bfloat16)
        dyc = torch.randn(B, T, D, device=dev, generator=gen).to(torch.bfloat16)
        wc = torch.randn(D, 4, device=dev, generator=gen) * 0.5
        res = {}
        for name, ng in (("qk_norm128", 128), ("v_plain", 0)):
            def conv_step():
                ops.short_conv(xc, wc, None, None, ng)
                ops.short_conv_bwd(xc, wc, None, None, dyc, ng)
            timed_loop(conv_step, 3, 2, torch)
            with _lib.StageTimer() as st:
                for _ in range(max(10, min(args.steps, 30))):
                    conv_step()
            f_ms = st.result["conv_fwd"][0] / st.result["conv_fwd"][1]
            b_ms = st.result["conv_bwd"][0] / st.result["conv_bwd"][1]
            fb, bb = 2 * B * T * D * 2, 3 * B * T * D * 2
            res[name] = {"norm_group": ng, "fwd_us": round(f_ms * 1e3, 2), "bwd_us": round(b_ms * 1e3, 2),
                         "fwd_GB_per_s": round(fb / (f_ms * 1e-3) / 1e9, 1),
                         "bwd_GB_per_s": round(bb / (b_ms * 1e-3) / 1e9, 1),
                         "fwd_hbm_frac": round(fb / (f_ms * 1e-3) / HBM_PEAK, 4),
                         "bwd_hbm_frac": round(bb / (b_ms * 1e-3) / HBM_PEAK, 4)}
            log(f"short conv {name}: fwd {f_ms * 1e3:.1f} us ({res[name]['fwd_GB_per_s']} GB/s), "
                f"bwd {b_ms * 1e3:.1f} us ({res[name]['bwd_GB_per_s']} GB/s)")
        out["short_conv"] = {"workload": "gdn_short_conv", "B": B, "T": T, "D": D, "W": 4, **res}
        del xc, dyc
        torch.cuda.empty_cache()

    if want("norm"):
        rows, dim, ntok, H = 8 * 4096 * 16, 128, 8 * 4096, 16
        log(f"gated RMSNorm rows={rows} dim={dim} and gates ntok={ntok} H={H}, bf16")
        gen = torch.Generator(device=dev).manual_seed(1)
        xn, gn, dyn = (torch.randn(rows, dim, device=dev, generator=gen).to(torch.bfloat16) for _ in range(3))
        wn = torch.rand(dim, device=dev, generator=gen) + 0.5
        ga, gb = (torch.randn(ntok, H, device=dev, generator=gen).to(torch.bfloat16) for _ in range(2))
        gA, gdt = torch.rand(H, device=dev, generator=gen), torch.randn(H, device=dev, generator=gen)
        gdg, gdb = (torch.randn(ntok, H, device=dev, generator=gen) for _ in range(2))

        def norm_step():
            ops.gated_rmsnorm(xn, gn, wn, 1e-5)
            ops.gated_rmsnorm_bwd(xn, gn, wn, dyn, 1e-5)
            ops.gdn_gates(ga, gb, gA, gdt, None, 1.0, float("-inf"))
            ops.gdn_gates_bwd(ga, gb, gA, gdt, None, gdg, gdb, 1.0, float("-inf"))

        timed_loop(norm_step, 3, 2, torch)
        with _lib.StageTimer() as st:
            for _ in range(max(10, min(args.steps, 30))):
                norm_step()
        us = {k: st.result[k][0] / st.result[k][1] * 1e3 for k in ("norm_fwd", "norm_bwd", "gates_fwd", "gates_bwd")}
        E = rows * dim * 2
        out["gated_rmsnorm"] = {"workload": "gdn_gated_rmsnorm", "rows": rows, "dim": dim,
                                "fwd_us": round(us["norm_fwd"], 2), "bwd_us": round(us["norm_bwd"], 2),
                                "fwd_GB_per_s": round(3 * E / us["norm_fwd"] / 1e3, 1),
                                "bwd_GB_per_s": round(5 * E / us["norm_bwd"] / 1e3, 1),
                                "fwd_hbm_frac": round(3 * E / (us["norm_fwd"] * 1e-6) / HBM_PEAK, 4),
                                "bwd_hbm_frac": round(5 * E / (us["norm_bwd"] * 1e-6) / HBM_PEAK, 4)}
        out["gates"] = {"workload": "gdn_gates", "ntok": ntok, "H": H, "fwd_us": round(us["gates_fwd"], 2),
                        "bwd_us": round(us["gates_bwd"], 2)}
        log(f"gated RMSNorm fwd {us['norm_fwd']:.1f} us ({out['gated_rmsnorm']['fwd_GB_per_s']} GB/s), bwd "
            f"{us['norm_bwd']:.1f} us ({out['gated_rmsnorm']['bwd_GB_per_s']} GB/s); gates fwd "
            f"{us['gates_fwd']:.1f} us, bwd {us['gates_bwd']:.1f} us")
        del xn, gn, dyn
        torch.cuda.empty_cache()

    if want("ce"):
        from archbench_amd import fused_ce

        N, Hd, Vv, nch = 8 * 4096, 1024, 50304, 1
        log(f"fused linear cross-entropy N={N} d_model={Hd} vocab={Vv} bf16, {nch} chunks")
        gen = torch.Generator(device=dev).manual_seed(2)
        xc = torch.randn(N, Hd, device=dev, generator=gen).to(torch.bfloat16).requires_grad_()
        wc = (torch.randn(Vv, Hd, device=dev, generator=gen) * 0.02).to(torch.bfloat16).requires_grad_()
        tc = torch.randint(0, Vv, (N,), device=dev, generator=gen)

        def ce_step():
            fused_ce.fused_linear_cross_entropy(xc, tc, wc, num_chunks=nch).backward()
            xc.grad = wc.grad = None

        sec = timed_loop(ce_step, max(3, min(args.steps, 10)), 2, torch)
        with _lib.StageTimer() as st:
            ce_step()
        ce_ms = st.result["cross_entropy"][0]
        flops = 3 * 2 * N * Vv * Hd
        ce_bytes = 2 * N * Vv * 2
        out["fused_linear_ce"] = {"workload": "fused_linear_cross_entropy", "N": N, "d_model": Hd, "vocab": Vv,
                                  "chunks": nch, "ms": round(sec * 1e3, 3), "tokens_per_s": round(N / sec, 1),
                                  "gemm_mfma_frac": round(flops / (sec - ce_ms * 1e-3) / MFMA_BF16_PEAK, 4),
                                  "ce_kernel_ms": round(ce_ms, 4),
                                  "ce_GB_per_s": round(ce_bytes / (ce_ms * 1e-3) / 1e9, 1),
                                  "ce_hbm_frac": round(ce_bytes / (ce_ms * 1e-3) / HBM_PEAK, 4)}
        log(f"fused linear CE {sec * 1e3:.2f} ms ({N / sec:.3e} tokens/s); CE kernels {ce_ms:.3f} ms "
            f"({out['fused_linear_ce']['ce_GB_per_s']} GB/s); GEMMs at "
            f"{out['fused_linear_ce']['gemm_mfma_frac'] * 100:.1f}% of bf16 peak")
        del xc, wc
        torch.cuda.empty_cache()

    if args.calibration_copy:
        a = torch.ones(256 * 2 ** 20, dtype=torch.uint8, device=dev)
        c = torch.empty_like(a)
        for _ in range(2):
            c.copy_(a)
        torch.cuda.synchronize()
        del a, c

    if want("train") and not args.no_cpu_baseline:
        log(f"cpu baseline (oracle, T={args.cpu_sample_T})")
        out["cpu_baseline"] = cpu_baseline(args.cpu_sample_T)
        log(f"cpu {out['cpu_baseline']['value']} tokens/s")

    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
