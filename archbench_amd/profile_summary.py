"""Summaries of rocprofv3 runs of bench.py, written to profiles/ (the files bench.py reads back).

    # kernel durations (rocprofv3 --kernel-trace --output-format csv -d DIR -o run -- python3 bench.py ...)
    python -m archbench_amd.profile_summary trace DIR --title "..." --command "..." -o profiles/X.md
    # HBM traffic per launch, from a FETCH_SIZE run and a WRITE_SIZE run of a command that ends with
    # bench.py's --calibration-copy (two device copies of 256 MiB calibrate the counters)
    python -m archbench_amd.profile_summary traffic FETCH_DIR WRITE_DIR --workload "..." --command "..." \
        -o profiles/hbm_traffic.json --md profiles/X.md
    # MFMA utilisation per launch, from a run with --pmc MfmaUtil MfmaFlopsBF16 (plus any SQ_* counters)
    python -m archbench_amd.profile_summary counters DIR --workload "..." --command "..." \
        -o profiles/mfma_counters.json --md profiles/X.md

Kernels are grouped into the stage names the library's own event timer uses (factors, fwd, fwd_stash,
bwd_recompute, prefix, seg_scan, bwd_local, bwd_state, bwd_intra, step, conv_fwd, conv_bwd, norm_fwd, norm_bwd,
...), so the numbers line up with bench.py's per-kernel table; a stage that ran at several grid sizes is split into
stage@grid (threads).
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import statistics
import sys
from collections import defaultdict

COPY_BYTES = 256 * 2 ** 20  # bench.py --calibration-copy: two copies of this many bytes


def _digest() -> str:
    """The kernel-source digest of this tree (bench.py reads a profile only if it matches its own sources)."""
    from archbench_amd.build import source_digest

    return source_digest()


def stage_of(name: str) -> str:
    """Stage name of a kernel (the library's mangled template names carry the forward sweep's mode)."""
    if "chunk_factors_kernel" in name:
        return "factors"
    if "fwd_sweep_kernel" in name:
        args = re.findall(r"Li(\d+)E", name)  # K, BV, MODE
        mode = int(args[2]) if len(args) >= 3 else -1
        return {0: "fwd", 1: "bwd_recompute", 2: "fwd_stash", 3: "prefix"}.get(mode, "fwd_sweep")
    if "bwd_state_kernel" in name:
        flags = re.findall(r"Lb(\d)E", name)  # SEPU, STORE (STORE = 0: the local pass of a segmented sweep)
        return "bwd_local" if len(flags) >= 2 and flags[1] == "0" else "bwd_state"
    for key, stage in (("seg_scan_kernel", "seg_scan"), ("bwd_intra_kernel", "bwd_intra"),
                       ("step_kernel", "step"), ("conv_silu_fwd", "conv_fwd"), ("conv_silu_bwd", "conv_bwd"),
                       ("row_norm_fwd", "norm_fwd"), ("row_norm_bwd", "norm_bwd"), ("gates_fwd", "gates_fwd"),
                       ("gates_bwd", "gates_bwd"), ("ce_fwd_bwd", "cross_entropy"), ("column_sum", "column_sum"),
                       ("write_dir_fwd", "write_dir_fwd"), ("write_dir_bwd", "write_dir_bwd"),
                       ("token_scan_fwd", "token_scan_fwd"), ("token_scan_bwd", "token_scan_bwd"),
                       ("copyBuffer", "copy"), ("copy_kernel", "copy")):
        if key in name:
            return stage
    return "other:" + name[:60]


def _csv(dir_: str, suffix: str) -> list[dict]:
    files = sorted(glob.glob(os.path.join(dir_, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {dir_}")
    rows = []
    for f in files:
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    return rows


def trace(args) -> None:
    rows = _csv(args.dir, "kernel_trace.csv")
    by = defaultdict(list)
    for r in rows:
        by[r["Kernel_Name"]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in by.values())
    lines = [f"# rocprofv3 kernel trace: {args.title}", "", "Command (repo root, one MI355X):", "", "```",
             args.command, "```", "", "Durations from the kernel trace, microseconds; stage = the library's stage "
             "name.", "", "| stage | kernel | calls | total (us) | average (us) | median (us) | min (us) | max (us) | % |",
             "|---|---|---|---|---|---|---|---|---|"]
    for name, d in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        short = name if len(name) <= 110 else name[:107] + "..."
        lines.append(f"| {stage_of(name)} | `{short}` | {len(d)} | {sum(d):.1f} | {statistics.mean(d):.2f} | "
                     f"{statistics.median(d):.2f} | {min(d):.2f} | {max(d):.2f} | {100 * sum(d) / total:.1f} |")
    open(args.out, "w").write("\n".join(lines) + "\n")
    print(f"wrote {args.out}")


def _per_dispatch(rows: list[dict]) -> dict:
    """{dispatch id: (group key, {counter: value})}; the key is the stage name and the dispatch's grid size in
    threads, so that launches of one kernel at different shapes are averaged apart."""
    out: dict = {}
    for r in rows:
        d = out.setdefault(r["Dispatch_Id"], ((stage_of(r["Kernel_Name"]), int(r.get("Grid_Size", 0) or 0)), {}))
        d[1][r["Counter_Name"]] = d[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return out


def _keys(groups) -> dict:
    """(stage, grid) -> the name used in the summaries: the stage alone when it ran at one grid size only,
    otherwise stage@grid (threads)."""
    grids = defaultdict(set)
    for st, g in groups:
        grids[st].add(g)
    return {(st, g): (st if len(grids[st]) == 1 else f"{st}@{g}") for st, g in groups}


def traffic(args) -> None:
    fetch, write = _per_dispatch(_csv(args.fetch_dir, "counter_collection.csv")), _per_dispatch(
        _csv(args.write_dir, "counter_collection.csv"))
    sums = {}
    for tag, disp, ctr in (("fetch", fetch, "FETCH_SIZE"), ("write", write, "WRITE_SIZE")):
        per = defaultdict(list)
        for key, vals in disp.values():
            if ctr in vals:
                per[key].append(vals[ctr])
        sums[tag] = per
    names = _keys(set(sums["fetch"]) | set(sums["write"]))
    sums = {tag: {names[k]: v for k, v in per.items()} for tag, per in sums.items()}
    copy_f = sum(sum(v) for k, v in sums["fetch"].items() if k.split("@")[0] == "copy")
    copy_w = sum(sum(v) for k, v in sums["write"].items() if k.split("@")[0] == "copy")
    if not copy_f or not copy_w:
        raise SystemExit("no calibration copy in the runs (run bench.py with --calibration-copy)")
    # KiB read / written by the two 256 MiB copies -> bytes per counter unit
    ff, fw = 2 * COPY_BYTES / copy_f, 2 * COPY_BYTES / copy_w
    per_launch, table = {}, []
    for st in sorted(set(sums["fetch"]) & set(sums["write"])):
        if st.split("@")[0] == "copy" or st.startswith("other:"):
            continue
        rf, rw = statistics.mean(sums["fetch"][st]), statistics.mean(sums["write"][st])
        per_launch[st] = {"read_bytes": round(rf * ff), "write_bytes": round(rw * fw), "bytes": round(rf * ff + rw * fw),
                          "launches": len(sums["fetch"][st])}
        table.append(f"| {st} | {len(sums['fetch'][st])} | {rf:.0f} | {rw:.0f} | {rf * ff / 1e6:.1f} | "
                     f"{rw * fw / 1e6:.1f} | {(rf * ff + rw * fw) / 1e6:.1f} |")
    doc = {"workload": args.workload, "command": args.command, "sources": _digest(),
           "calibration": {"fetch_bytes_per_unit": round(ff, 4), "write_bytes_per_unit": round(fw, 4),
                           "copy": "two device copies of 256 MiB (bench.py --calibration-copy)"},
           "per_launch": per_launch}
    json.dump(doc, open(args.out, "w"), indent=1)
    print(f"wrote {args.out}")
    if args.md:
        lines = [f"# HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE): {args.workload}", "",
                 "Commands (repo root, one MI355X), one counter per run:", "", "```", args.command, "```", "",
                 f"Calibration: the two 256 MiB copies read {copy_f:.0f} FETCH_SIZE units and write {copy_w:.0f} "
                 f"WRITE_SIZE units, so bytes = FETCH_SIZE x {ff:.4f} and WRITE_SIZE x {fw:.4f}.", "",
                 "| stage | launches | FETCH_SIZE (avg) | WRITE_SIZE (avg) | read (MB) | written (MB) | total (MB) |",
                 "|---|---|---|---|---|---|---|", *table]
        open(args.md, "w").write("\n".join(lines) + "\n")
        print(f"wrote {args.md}")


def counters(args) -> None:
    disp = _per_dispatch(_csv(args.dir, "counter_collection.csv"))
    names_of = _keys({key for key, _ in disp.values()})
    per = defaultdict(lambda: defaultdict(list))
    for key, vals in disp.values():
        st = names_of[key]
        for c, v in vals.items():
            per[st][c].append(v)
    names = sorted({c for st in per.values() for c in st})
    # with SQ_WAVE_CYCLES present, every other SQ_ counter is also shown as a fraction of it (the share of the
    # waves' cycles spent in that state; the SQ cycle counters share its unit)
    frac_names = [c for c in names if c.startswith("SQ_") and c != "SQ_WAVE_CYCLES"] if "SQ_WAVE_CYCLES" in names \
        else []
    per_launch, table = {}, []
    for st in sorted(per):
        if st.split("@")[0] == "copy" or st.startswith("other:"):
            continue
        avg = {c: statistics.mean(per[st][c]) for c in per[st]}
        ent = {"launches": len(next(iter(per[st].values())))}
        if "MfmaUtil" in avg:
            ent["mfma_util"] = round(avg["MfmaUtil"] / 100.0, 4)
        if "MfmaFlopsBF16" in avg:
            ent["executed_bf16_flops"] = round(avg["MfmaFlopsBF16"])
        ent.update({c: round(v, 1) for c, v in avg.items() if c not in ("MfmaUtil", "MfmaFlopsBF16")})
        fr = [avg.get(c, float("nan")) / avg["SQ_WAVE_CYCLES"] for c in frac_names] if frac_names else []
        if frac_names:
            ent["per_wave_cycle"] = {c: round(f, 4) for c, f in zip(frac_names, fr)}
        per_launch[st] = ent
        table.append(f"| {st} | {ent['launches']} | " + " | ".join(f"{avg.get(c, float('nan')):.4g}" for c in names)
                     + "".join(f" | {f:.3f}" for f in fr) + " |")
    json.dump({"workload": args.workload, "command": args.command, "sources": _digest(), "per_launch": per_launch},
              open(args.out, "w"),
              indent=1)
    print(f"wrote {args.out}")
    if args.md:
        lines = [f"# rocprofv3 counters per launch: {args.workload}", "", "Command (repo root, one MI355X):", "",
                 "```", args.command, "```", "", "Averages over the launches of each stage" +
                 ("; the last columns are the SQ counters over SQ_WAVE_CYCLES." if frac_names else "."), "",
                 "| stage | launches | " + " | ".join(names) + "".join(f" | {c} / WAVE_CYCLES" for c in frac_names)
                 + " |", "|---|---|" + "---|" * (len(names) + len(frac_names)), *table]
        open(args.md, "w").write("\n".join(lines) + "\n")
        print(f"wrote {args.md}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--title", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("-o", "--out", required=True)
    t.set_defaults(fn=trace)
    f = sub.add_parser("traffic")
    f.add_argument("fetch_dir")
    f.add_argument("write_dir")
    f.add_argument("--workload", required=True)
    f.add_argument("--command", required=True)
    f.add_argument("-o", "--out", required=True)
    f.add_argument("--md")
    f.set_defaults(fn=traffic)
    c = sub.add_parser("counters")
    c.add_argument("dir")
    c.add_argument("--workload", required=True)
    c.add_argument("--command", required=True)
    c.add_argument("-o", "--out", required=True)
    c.add_argument("--md")
    c.set_defaults(fn=counters)
    args = ap.parse_args(argv)
    args.fn(args)
    return 0


if __name__ == "__main__":
    sys.exit(main())
