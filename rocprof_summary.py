"""Reduce rocprofv3 CSV output to the short summaries kept under profiles/.

  python rocprof_summary.py trace DIR --out FILE.md --command "..."
      kernel-trace + stats: per-kernel durations of the ppk kernels, and the
      decode-step period and inter-kernel gaps measured from the dispatch trace.
  python rocprof_summary.py counters DIR [DIR ...] --kernel-regex RX --out FILE.md
         --title T --command "..."
      any --pmc runs: the median per-dispatch value of every counter for each kernel
      matching RX, plus the L2 hit rate when TCC_HIT_sum and TCC_MISS_sum were read.
  python rocprof_summary.py traffic FETCH_DIR WRITE_DIR --kernel NAME
         --calib-regex REGEX --calib-bytes N --algorithmic-bytes N --workload W --split S
         --out-md FILE.md --out-json FILE.json --command "..."
      --pmc FETCH_SIZE / WRITE_SIZE: HBM KiB per dispatch of one kernel, scaled by
      the same counters read on a plain copy kernel of known size.

Standalone (no torch / GPU import): runs on the profiling host right after rocprofv3.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import shlex
import statistics
import sys


def _rows(path: str) -> list[dict]:
    with open(path, newline="") as f:
        return [{k.strip().lower(): v for k, v in r.items()} for r in csv.DictReader(f)]


def _one(dirpath: str, suffix: str) -> str:
    hits = glob.glob(os.path.join(dirpath, "**", f"*{suffix}"), recursive=True)
    if not hits:
        raise SystemExit(f"no *{suffix} under {dirpath}")
    return sorted(hits)[0]


def trace(args) -> None:
    stats = _rows(_one(args.dir, "kernel_stats.csv"))
    disp = _rows(_one(args.dir, "kernel_trace.csv"))
    lines = [f"# rocprofv3 kernel trace: {args.title}", "", "Command (from the repository root):", "",
             f"    {args.command}", "", "Summarised with:", "", f"    {_self_command()}", "",
             f"## Per-kernel durations (kernels matching `{args.kernel_regex}`, all dispatches)", "",
             "| kernel | calls | avg µs | min µs | max µs | total ms |", "|---|---|---|---|---|---|"]
    for r in sorted(stats, key=lambda r: -float(r.get("totaldurationns", 0))):
        name = r.get("name", "")
        if not re.search(args.kernel_regex, name):
            continue
        lines.append(f"| {name} | {r['calls']} | {float(r['averagens']) / 1e3:.2f} | {float(r['minns']) / 1e3:.2f} | "
                     f"{float(r['maxns']) / 1e3:.2f} | {float(r['totaldurationns']) / 1e6:.3f} |")
    # Step period and gaps: consecutive dispatches of the step's kernels, last N steps.
    seq = sorted((int(r["start_timestamp"]), int(r["end_timestamp"]), r["kernel_name"]) for r in disp
                 if r["kernel_name"].startswith("ppk_"))
    anchor = [s for s in seq if s[2].startswith(args.anchor)]
    tail = anchor[-args.steps:] if len(anchor) > args.steps else anchor
    if len(tail) >= 2:
        periods = [(b[0] - a[0]) / 1e3 for a, b in zip(tail, tail[1:])]
        lines += ["", f"## Decode-step period from the dispatch trace (last {len(tail)} {args.anchor} starts)", "",
                  f"- mean {statistics.mean(periods):.2f} µs, median {statistics.median(periods):.2f} µs, "
                  f"min {min(periods):.2f} µs"]
        t0 = tail[0][0]
        window = [s for s in seq if s[0] >= t0]
        gaps = {}
        for a, b in zip(window, window[1:]):
            gaps.setdefault(f"{a[2]} -> {b[2]}", []).append((b[0] - a[1]) / 1e3)
        lines += ["", "| transition | count | mean gap µs (end of first -> start of next) |", "|---|---|---|"]
        for k, v in sorted(gaps.items()):
            lines.append(f"| {k} | {len(v)} | {statistics.mean(v):.2f} |")
    _write(args.out, "\n".join(lines) + "\n")


def _per_dispatch(path: str, counter: str) -> dict[int, tuple[str, float]]:
    out: dict[int, tuple[str, float]] = {}
    for r in _rows(path):
        if r.get("counter_name", "").strip() != counter:
            continue
        did = int(r["dispatch_id"])
        name = r["kernel_name"]
        prev = out.get(did, (name, 0.0))[1]
        out[did] = (name, prev + float(r["counter_value"]))
    return out


def traffic(args) -> None:
    fetch = _per_dispatch(_one(args.fetch_dir, "counter_collection.csv"), "FETCH_SIZE")
    write = _per_dispatch(_one(args.write_dir, "counter_collection.csv"), "WRITE_SIZE")
    kre, cre = re.compile(args.kernel), re.compile(args.calib_regex)

    def pick(d, rx):
        return [v for _, (n, v) in sorted(d.items()) if rx.search(n)]

    kf, kw, cf, cw = pick(fetch, kre), pick(write, kre), pick(fetch, cre), pick(write, cre)
    if not (kf and kw and cf and cw):
        raise SystemExit(f"missing dispatches: kernel fetch/write {len(kf)}/{len(kw)}, calib {len(cf)}/{len(cw)}")
    # The calibration kernel is the largest dispatch matching its regex.
    cf, cw = [max(cf)], [max(cw)]
    calib_kib = args.calib_bytes / 1024.0
    f_factor = statistics.median(cf) / calib_kib  # counter KiB per true KiB read
    w_factor = statistics.median(cw) / calib_kib
    fetch_bytes = statistics.median(kf) / f_factor * 1024.0
    write_bytes = statistics.median(kw) / w_factor * 1024.0
    total = fetch_bytes + write_bytes
    res = {"workload": args.workload, "split": args.split, "kernel": args.kernel,
           "hbm_bytes_per_launch": round(total), "fetch_bytes_per_launch": round(fetch_bytes),
           "write_bytes_per_launch": round(write_bytes), "algorithmic_bytes_per_launch": args.algorithmic_bytes,
           "traffic_over_algorithmic": round(total / args.algorithmic_bytes, 4),
           "fetch_kib_raw_median": statistics.median(kf), "write_kib_raw_median": statistics.median(kw),
           "calibration": {"kernel_regex": args.calib_regex, "bytes_each_way": args.calib_bytes,
                           "fetch_kib_raw": statistics.median(cf), "write_kib_raw": statistics.median(cw),
                           "fetch_factor": round(f_factor, 4), "write_factor": round(w_factor, 4)},
           "dispatches": {"kernel_fetch": len(kf), "kernel_write": len(kw)}}
    _write(args.out_json, json.dumps(res, indent=1) + "\n")
    md = [f"# HBM traffic per launch: {args.kernel}, {args.workload}", "", "Commands (from the repository root):", "",
          f"    {args.command}", "", "Summarised with:", "", f"    {_self_command()}", "",
          f"- FETCH_SIZE median {res['fetch_kib_raw_median']:.0f} KiB/dispatch over {len(kf)} dispatches; "
          f"WRITE_SIZE median {res['write_kib_raw_median']:.0f} KiB over {len(kw)}",
          f"- calibration: one {args.calib_bytes} B-in / {args.calib_bytes} B-out elementwise kernel "
          f"(`{args.calib_regex}`) read FETCH {res['calibration']['fetch_kib_raw']:.0f} KiB and WRITE "
          f"{res['calibration']['write_kib_raw']:.0f} KiB: factors {f_factor:.4f} / {w_factor:.4f}",
          f"- scaled HBM bytes per launch: fetch {fetch_bytes:.4g} + write {write_bytes:.4g} = {total:.4g}",
          f"- algorithmic bytes per launch: {args.algorithmic_bytes} -> traffic / algorithmic = "
          f"{res['traffic_over_algorithmic']:.4f}"]
    _write(args.out_md, "\n".join(md) + "\n")


def counters(args) -> None:
    kre = re.compile(args.kernel_regex)
    per: dict[str, dict[str, list[float]]] = {}
    for d in args.dirs:
        path = _one(d, "counter_collection.csv")
        by_dispatch: dict[tuple[int, str], tuple[str, float]] = {}
        for r in _rows(path):
            name = r["kernel_name"]
            if not kre.search(name):
                continue
            key = (int(r["dispatch_id"]), r["counter_name"].strip())
            prev = by_dispatch.get(key, (name, 0.0))[1]
            by_dispatch[key] = (name, prev + float(r["counter_value"]))
        for (_, counter), (name, value) in by_dispatch.items():
            per.setdefault(name, {}).setdefault(counter, []).append(value)
    if not per:
        raise SystemExit(f"no dispatches of kernels matching {args.kernel_regex!r}")
    lines = [f"# rocprofv3 counters: {args.title}", "", "Commands (from the repository root):", "",
             f"    {args.command}", "", "Summarised with:", "", f"    {_self_command()}", "",
             "| kernel | counter | dispatches | median per dispatch |", "|---|---|---|---|"]
    for name in sorted(per):
        for counter in sorted(per[name]):
            vals = per[name][counter]
            lines.append(f"| {name} | {counter} | {len(vals)} | {statistics.median(vals):.6g} |")
        hit, miss = per[name].get("TCC_HIT_sum"), per[name].get("TCC_MISS_sum")
        if hit and miss:
            h, m = statistics.median(hit), statistics.median(miss)
            lines.append(f"| {name} | L2 hit rate = TCC_HIT / (TCC_HIT + TCC_MISS) | {len(hit)} | "
                         f"{100.0 * h / max(h + m, 1.0):.2f} % |")
    _write(args.out, "\n".join(lines) + "\n")


def _self_command() -> str:
    return "python3 rocprof_summary.py " + shlex.join(sys.argv[1:])


def _write(path: str, text: str) -> None:
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        f.write(text)
    print(text)


def main(argv=None) -> int:
    p = argparse.ArgumentParser()
    sub = p.add_subparsers(dest="mode", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--out", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--title", default="decode step")
    t.add_argument("--anchor", default="ppk_decode")
    t.add_argument("--kernel-regex", default="^ppk_", help="kernels listed in the duration table")
    t.add_argument("--steps", type=int, default=100)
    f = sub.add_parser("traffic")
    f.add_argument("fetch_dir")
    f.add_argument("write_dir")
    f.add_argument("--kernel", required=True)
    f.add_argument("--calib-regex", required=True)
    f.add_argument("--calib-bytes", type=int, required=True)
    f.add_argument("--algorithmic-bytes", type=int, required=True)
    f.add_argument("--workload", required=True)
    f.add_argument("--split", type=int, required=True)
    f.add_argument("--out-md", required=True)
    f.add_argument("--out-json", required=True)
    f.add_argument("--command", required=True)
    c = sub.add_parser("counters")
    c.add_argument("dirs", nargs="+")
    c.add_argument("--kernel-regex", required=True)
    c.add_argument("--out", required=True)
    c.add_argument("--title", required=True)
    c.add_argument("--command", required=True)
    a = p.parse_args(argv)
    {"trace": trace, "traffic": traffic, "counters": counters}[a.mode](a)
    return 0


if __name__ == "__main__":
    sys.exit(main())
