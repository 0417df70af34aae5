#!/usr/bin/env python3
"""Gated DeltaNet benchmark on one MI355X.

Headline (one JSON line on stdout): chunk forward + backward of the GDN op at B=8, T=4096, H=16, K=V=128, bf16
inputs with fp32 state/accumulation, synthetic seeded data resident in HBM.  One step = one training forward
call (gdn_chunk_fwd_stash: o and hT, keeping the per-chunk states for the backward, as autograd does) and one
backward call (gdn_chunk_bwd_stashed: every gradient, dq, dk, dv, dg, dbeta).  tokens/s = B*T / step time.
The recompute path (gdn_chunk_fwd + gdn_chunk_bwd, no stash) is timed beside it as recompute_ms_per_step.

Also reported in the same line:
  roofline      the dominant kernel of the step against the roofline that bounds it: its algorithmic intensity
                (stage_flops / stage_bytes) decides between HBM (below the ridge, 2.5 PFLOP/s / 8 TB/s) and
                MFMA; achieved = algorithmic bytes (or FLOPs) per launch over the launch's average duration
                (HIP events on the launch stream); traffic = measured HBM bytes per launch;
  mfma_frac     the whole step at the workload's algorithmic count 3 * F_fwd per token-head,
                F_fwd = 2C(3K + 2V) + 6KV (C = 64);
  fwd_only      forward alone at B=8, T=2048, H=8, K=V=128 (% of the bf16 MFMA peak);
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
    """Algorithmic dense MFMA FLOPs per token-head of each kernel stage (C = 64 tokens per chunk).  Work a
    stage repeats for every 64-wide V block (the chunk factors) is counted once."""
    return {
        "fwd": 6 * C * K + 4 * C * V + 6 * K * V,            # KK^T, QK^T, W; U, PR; WS, QS, K^T R
        "fwd_stash": 6 * C * K + 4 * C * V + 6 * K * V,      # the forward's products (states also written)
        "bwd_recompute": 4 * C * K + 2 * C * V + 4 * K * V,  # KK^T, W; U; WS, K^T R
        "bwd_state": 6 * C * K + 2 * C * V + 6 * K * V,      # KK^T, QK^T, W; P^T dO; K dS, Qg^T dO, W^T dR
        "bwd_intra": 4 * C * V + 6 * K * V + 12 * C * K,     # dO R^T, dY R^T; dO S0^T, R dSC^T, dY S0^T; KK^T, QK^T, dq, dk
    }.get(stage, 0)


def stage_bytes(stage: str, K: int, V: int, es: int = 2) -> int:
    """Algorithmic HBM bytes per token-head of each kernel stage: every input read once and every output
    written once (q, k: es*K; v, o, dO: es*V; g, beta, G: 4; per-chunk workspace: state es*K*V/C, R es*V,
    Tm es*C).  Intermediates the design keeps on-chip count nothing."""
    qk, vv, st, r, tm = es * K, es * V, es * K * V // C, es * V, es * C
    return {
        "fwd": 2 * qk + vv + 8 + vv,                           # q k v g beta -> o
        "fwd_stash": 2 * qk + vv + 8 + vv + st + r + tm + 4,   # ... -> o, states, R, Tm, G
        "bwd_recompute": qk + vv + 8 + st + r + tm + 4,        # k v g beta -> states, R, Tm, G
        "bwd_state": 2 * qk + vv + 8 + st + r,                 # q k dO g beta -> dstates, dY
        "bwd_intra": 2 * qk + 2 * vv + 8 + 2 * st + 2 * r + 2 * qk + vv + 8,  # ... G, S0, dSC, R, dY -> dq dk dv dg db
    }.get(stage, 0)


def measured_traffic() -> dict:
    """HBM bytes per launch by stage, from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarised in
    profiles/hbm_traffic.json (calibrated on a copy of known size); empty if that file is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("per_launch", {})
    except (OSError, ValueError):
        return {}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def timed_loop(fn, steps: int, warmup: int, torch) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


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
    ap.add_argument("--only", choices=["all", "train", "fwd", "decode", "conv", "norm", "ce"], default="all",
                    help="run one workload only (profiling runs); the JSON line needs 'all' or 'train'")
    args = ap.parse_args()
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

    if args.only in ("all", "train"):
        B, T, H, K, V = 8, 4096, 16, 128, 128
        log(f"headline fwd+bwd B={B} T={T} H={H} K={K} V={V} bf16: generating inputs")
        x = make_inputs(B, T, H, K, V, seed=0, with_do=True).to(dev, torch.bfloat16)

        def step():
            _, _, stash = ops.chunk_fwd_stash(x.q, x.k, x.v, x.g, x.beta, None, 1.0)
            ops.chunk_bwd_stashed(x.q, x.k, x.v, x.g, x.beta, None, x.do, None, stash, 1.0)

        def step_recompute():
            ops.chunk_fwd(x.q, x.k, x.v, x.g, x.beta, None, 1.0)
            ops.chunk_bwd(x.q, x.k, x.v, x.g, x.beta, None, x.do, None, 1.0)

        log(f"timing {args.steps} steps after {args.warmup} warmup")
        sec = timed_loop(step, args.steps, args.warmup, torch)
        sec_rc = timed_loop(step_recompute, max(3, args.steps // 2), 1, torch)
        tokens = B * T
        with _lib.StageTimer() as st:
            for _ in range(max(3, min(args.steps, 10))):
                step()
        stages = {k: (ms / n, n) for k, (ms, n) in st.result.items()}
        dom = max(stages, key=lambda s: stages[s][0])
        dom_ms = stages[dom][0]
        dom_flops = stage_flops(dom, K, V) * B * T * H
        dom_bytes = stage_bytes(dom, K, V) * B * T * H
        hbm_bound = dom_flops / dom_bytes < MFMA_BF16_PEAK / HBM_PEAK
        if hbm_bound:
            roof = {"kernel": dom, "bound": "hbm", "achieved": round(dom_bytes / (dom_ms * 1e-3) / 1e9, 1),
                    "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(dom_bytes / (dom_ms * 1e-3) / HBM_PEAK, 4)}
        else:
            roof = {"kernel": dom, "bound": "mfma", "achieved": round(dom_flops / (dom_ms * 1e-3) / 1e12, 2),
                    "peak": MFMA_BF16_PEAK / 1e12, "unit": "TFLOP/s",
                    "frac": round(dom_flops / (dom_ms * 1e-3) / MFMA_BF16_PEAK, 4)}
        roof.update({"traffic": measured_traffic().get(dom, {}).get("bytes"), "algorithmic_bytes": dom_bytes,
                     "flops_per_launch": dom_flops,
                     "mfma_frac": round(dom_flops / (dom_ms * 1e-3) / MFMA_BF16_PEAK, 4),
                     "avg_ms": round(dom_ms, 4)})
        call_flops = 3 * f_fwd(K, V) * B * T * H
        out.update({
            "metric": METRIC, "value": round(tokens / sec, 1), "unit": "tokens/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic",
            "config": {"workload": "gdn_chunk_fwd_bwd", "B": B, "T": T, "H": H, "K": K, "V": V, "chunk": C,
                       "scale": 1.0, "state": "fp32", "g_shift": 4.0},
            "mfma_frac": round(call_flops / sec / MFMA_BF16_PEAK, 4),
            "roofline": roof,
            "stages_ms": {k: round(v[0], 4) for k, v in stages.items()},
            "recompute_ms_per_step": round(sec_rc * 1e3, 4),
        })
        log(f"fwd+bwd {sec * 1e3:.3f} ms/step, {tokens / sec:.3e} tokens/s; stages {out['stages_ms']}; "
            f"recompute path {sec_rc * 1e3:.3f} ms/step")
        del x
        torch.cuda.empty_cache()

    if args.only in ("all", "fwd"):
        B, T, H, K, V = 8, 2048, 8, 128, 128
        log(f"forward only B={B} T={T} H={H} K={K} V={V} bf16")
        x = make_inputs(B, T, H, K, V, seed=0).to(dev, torch.bfloat16)
        sec = timed_loop(lambda: ops.chunk_fwd(x.q, x.k, x.v, x.g, x.beta, None, 1.0), args.steps, args.warmup,
                         torch)
        out["fwd_only"] = {"workload": "gdn_chunk_fwd", "B": B, "T": T, "H": H, "K": K, "V": V,
                           "ms": round(sec * 1e3, 4), "tokens_per_s": round(B * T / sec, 1),
                           "mfma_frac": round(f_fwd(K, V) * B * T * H / sec / MFMA_BF16_PEAK, 4)}
        log(f"fwd {sec * 1e3:.3f} ms")
        del x
        torch.cuda.empty_cache()

    if args.only in ("all", "decode"):
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

    if args.only in ("all", "conv"):
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

    if args.only in ("all", "norm"):
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

    if args.only in ("all", "ce"):
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

    if args.only in ("all", "train") and not args.no_cpu_baseline:
        log(f"cpu baseline (oracle, T={args.cpu_sample_T})")
        out["cpu_baseline"] = cpu_baseline(args.cpu_sample_T)
        log(f"cpu {out['cpu_baseline']['value']} tokens/s")

    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
