"""Decode-step benchmark of the MI355X int8 KV path.

One step = quantize-and-append of the new K/V token of every (sequence, head)
+ decode attention over the 8192-token int8 history and the current token
(ppk_decode_step), on one GPU with all inputs resident in HBM. Prints one
JSON line.

  python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pop2-bezier_amd"))

METRIC = "decode-attention µs/step + achieved HBM GB/s (% of peak), B=32 ctx=8192 int8 KV"
HBM_PEAK_GBPS = 8000.0
SEED = 20261011


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=300)
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--heads", type=int, default=16)
    p.add_argument("--head-dim", type=int, default=128)
    p.add_argument("--context", type=int, default=8192)
    p.add_argument("--split", type=int, default=0, help="tokens per split (0 = library policy)")
    p.add_argument("--config", type=int, choices=(1, 2, 3, 4, 5), default=5,
                   help="BASELINE config: 5 (default) is the headline workload; 1, 3, 4 are the latency-bound "
                        "decode shapes and 2 the append-only shape, timed warm and cold (HBM) with the same "
                        "fields")
    p.add_argument("--kv", choices=("int8", "bf16", "f32"), default="int8",
                   help="int8 (default, the headline workload) or the float-KV decode path over a bf16/f32 store")
    p.add_argument("--sampler", action="store_true",
                   help="time the CFG + Renyi sampler instead (batch = --batch, --choices, --guidance)")
    p.add_argument("--arena", action="store_true",
                   help="time the KV arena manager: joining prefilled caches into batch arenas, then decode rounds "
                        "of one-token appends over --layers layers with a shared write plan")
    p.add_argument("--dequantize", choices=("bf16", "f32", "f16"), default=None,
                   help="time ppk_dequantize (int8 -> DTYPE) over one tensor of the headline history "
                        "(B*H rows x --context tokens x D)")
    p.add_argument("--quantize", choices=("bf16", "f32", "f16"), default=None,
                   help="time ppk_quantize (DTYPE -> int8 codes + scales) over one tensor of the headline "
                        "history (B*H rows x --context tokens x D)")
    p.add_argument("--layers", type=int, default=24)
    p.add_argument("--prefill", type=int, default=1000)
    p.add_argument("--choices", type=int, default=2048)
    p.add_argument("--guidance", type=int, default=2)
    p.add_argument("--device-lengths", action="store_true",
                   help="configs 1, 3, 4 and --lengths: pass the lengths on the device only (no host copy), i.e. "
                        "the per-row plan")
    p.add_argument("--plan", choices=("auto", "per-row", "balanced"), default="auto",
                   help="configs 1, 3, 4 and --lengths with host lengths: the launch plan (auto = the library's "
                        "choice; per-row or balanced fix it, PPK_ATTN_PLAN_PER_ROW / PPK_ATTN_PLAN_BALANCED)")
    p.add_argument("--step", action="store_true",
                   help="with --kv bf16/f32: time the fused float decode step (ppk_float_decode_step: write the "
                        "current token at slot lengths[b] - 1, attend lengths[b] tokens) beside the reference's "
                        "order (the token written by torch indexing, then the attention call)")
    p.add_argument("--lengths", default=None,
                   help="with --kv bf16/f32 or --config 4: comma-separated per-sequence lengths of a ragged batch "
                        "(NxL repeats L N times; uniform:B:LO:HI:SEED draws B lengths from numpy's "
                        "default_rng(SEED).integers(LO, HI + 1)); the batch is their count and the store holds the "
                        "longest")
    p.add_argument("--bf16-history", action="store_true",
                   help="int8 decode: round every dequantised history element to bf16 before the fp32 dot "
                        "(PPK_ATTN_BF16_HISTORY, the reference kernel's pp_i8_load arithmetic; kernels "
                        "ppk_decode_bf16h_d*) instead of the default fp32 dequantisation")
    p.add_argument("--no-append", action="store_true",
                   help="int8 config 5: time ppk_decode_attention alone (the uncommitted partial query: the current "
                        "token attended from its copy, nothing written to the arenas) instead of the fused step")
    p.add_argument("--wave-clock", default=None, metavar="OUT.md",
                   help="int8 configs 1, 3, 4, 5: after the timed runs, run up to 10 steps again on a context "
                        "created from the wave-clock code object (ppk_kernels_clock.hsaco) and write the per-phase "
                        "breakdown of every decode and merge launch to OUT.md (summary also in the JSON line; "
                        "PPK_WAVE_CLOCK_RAW=FILE.npy also saves the raw records)")
    p.add_argument("--probe", action="store_true",
                   help="int8 config 5 / --head-dim, or --kv bf16|f32 (uniform lengths): after the timed runs, "
                        "time the streaming-read probe "
                        "(ppk/libppk_probe.so) at the decode launch's geometry (its waves, waves per block, blocks "
                        "per CU and 1 KiB tiles, 4 per batch) for 2, 3, 4 and 6 batches in flight, and add the "
                        "rates and the decode's fraction of the probe at its own ring depth to the JSON line")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-rows", type=int, default=0,
                   help="head rows timed for the CPU baseline (0 = every row of the step)")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--calibrate-copy", action="store_true",
                   help="run one plain 1 GiB elementwise copy (torch.neg, f32) first: the known-size kernel that "
                        "scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings")
    p.add_argument("--traffic", default=None,
                   help="JSON with measured HBM bytes per partial launch (rocprofv3 --pmc), if present")
    return p.parse_args()


def committed_traffic(tpath: str, **match) -> tuple[int | None, str | None]:
    """HBM bytes per launch from a committed rocprofv3 traffic summary (profiles/*_traffic.json), if it was
    measured on this exact workload (every `match` key equal). The figure comes from a separate profiled run
    (FETCH_SIZE and WRITE_SIZE, scaled by a copy kernel of known size), not from this process: the returned
    source string says so, and the bench line carries it beside the number."""
    if not os.path.exists(tpath):
        return None, None
    try:
        with open(tpath) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, None
    if any(t.get(k) != v for k, v in match.items()):
        return None, None
    return t.get("hbm_bytes_per_launch"), (os.path.relpath(tpath, ROOT) + ": rocprofv3 FETCH_SIZE + WRITE_SIZE of "
                                          "a separate profiled run of this workload, scaled by a copy kernel")


WAVE_CLOCK_HZ = 100e6  # the real-time clock the wave-clock build reads (s_memrealtime)
DECODE_POINTS = ("entry", "loads issued", "past[b] here", "first K data here", "stream done", "block joined",
                 "output stored")


def wave_clock_run(steps_fn, calls, steps: int, dev, raw: str | None = None) -> tuple[dict, str]:
    """Run `steps_fn` `steps` times with every prepared call in `calls` on a context made from the wave-clock
    code object, read the records (layout in pop2-bezier_amd/csrc/ppk_kernel_args.h) and summarise them:
    per decode launch the intervals between a wave's clock points and the launch's dispatch spread and span,
    per merge launch entry -> records combined -> stored, and the gaps between consecutive launches."""
    import ctypes
    import statistics

    import torch
    from ppk import _abi

    lib = _abi.lib()
    path = os.path.join(ROOT, "pop2-bezier_amd", "ppk", "ppk_kernels_clock.hsaco")
    ctx = ctypes.c_void_p()
    _abi.check(lib.ppk_context_create(dev.index or 0, path.encode(), ctypes.byref(ctx)), "ppk_context_create")
    # Slots per launch and kernel kind: the most waves of any decode launch, or rows of a merge launch.
    per = max(max(c.plan_info["blocks"] * c.plan_info["waves_per_block"],
                  c.args.attn.rows if hasattr(c.args, "attn") else c.args.rows) for c in calls)
    nrec = per * 2 * len(calls) * steps
    buf = torch.zeros(16 * (nrec + 1), dtype=torch.int64, device=dev)
    buf[0], buf[1] = per, nrec
    saved = [c.ctx for c in calls]
    try:
        for c in calls:
            c.ctx = ctx
        for _ in range(3):  # warm: code object, caches (no clock yet)
            steps_fn()
        torch.cuda.synchronize()
        _abi.check(lib.ppk_context_set_wave_clock(ctx, ctypes.c_void_p(buf.data_ptr()), buf.numel() * 8),
                   "ppk_context_set_wave_clock")
        for _ in range(steps):
            steps_fn()
        torch.cuda.synchronize()
        rec = buf[16:].view(-1, 16).cpu().numpy().view("uint64")
        rec = rec[rec[:, 0] != 0]  # slots never written (fewer waves than the slot count)
        if raw:
            import numpy as np
            np.save(raw, rec)
        _abi.check(lib.ppk_context_set_wave_clock(ctx, None, 0), "ppk_context_set_wave_clock")
    finally:
        for c, old in zip(calls, saved):
            c.ctx = old
        torch.cuda.synchronize()
        lib.ppk_context_release(ctx)
    return summarize_wave_clock(rec)


def summarize_wave_clock(rec) -> tuple[dict, str]:
    """Summary dict and markdown tables of wave-clock records (uint64 [n, 16], the written slots only; layout
    in pop2-bezier_amd/csrc/ppk_kernel_args.h)."""
    import statistics

    us = 1e6 / WAVE_CLOCK_HZ
    kind = (rec[:, 0] >> 56).astype(int)
    seq = ((rec[:, 0] >> 32) & 0xFFFFFF).astype(int)
    wave = (rec[:, 0] & 0xFF).astype(int)
    t = rec[:, 2:10].astype("int64")
    launches = {}
    for i in range(len(rec)):
        launches.setdefault((int(seq[i]), int(kind[i])), []).append(i)

    def med(xs):
        return round(statistics.median(xs), 2) if xs else None

    def p90(xs):
        return round(sorted(xs)[int(0.9 * (len(xs) - 1))], 2) if xs else None

    iv = {k: [] for k in ("entry -> loads issued", "entry -> past[b] here", "entry -> first K data here",
                          "first K data -> stream done", "stream done -> block joined",
                          "block joined -> output stored (wave 0)")}
    d_spread, d_span, m_span, m_comb, m_store, gap_dm, gap_md, layer = [], [], [], [], [], [], [], []
    xcc = ((rec[:, 1] >> 32) & 0xF).astype(int)  # the XCD the wave ran on
    by_xcd = {}  # XCD -> stream durations, wave ends after the launch's first entry, per-launch last ends
    seqs = sorted({s_ for s_, k_ in launches})
    for s_ in seqs:
        d = launches.get((s_, 1), [])
        m = launches.get((s_, 2), [])
        if not d:
            continue
        te = t[d, 0]
        ends = [int(t[i, 6] if wave[i] == 0 else t[i, 5]) for i in d]
        d_spread.append((te.max() - te.min()) * us)
        d_span.append((max(ends) - te.min()) * us)
        last = {}
        for i, e in zip(d, ends):
            x = by_xcd.setdefault(int(xcc[i]), {"stream": [], "end": [], "last": []})
            if t[i, 3]:
                x["stream"].append((t[i, 4] - t[i, 3]) * us)
            x["end"].append((e - te.min()) * us)
            last[int(xcc[i])] = max(last.get(int(xcc[i]), 0), e)
        for k_, e in last.items():
            by_xcd[k_]["last"].append((e - te.min()) * us)
        for i in d:
            iv["entry -> loads issued"].append((t[i, 1] - t[i, 0]) * us)
            iv["entry -> past[b] here"].append((t[i, 2] - t[i, 0]) * us)
            if t[i, 3]:
                iv["entry -> first K data here"].append((t[i, 3] - t[i, 0]) * us)
                iv["first K data -> stream done"].append((t[i, 4] - t[i, 3]) * us)
            iv["stream done -> block joined"].append((t[i, 5] - t[i, 4]) * us)
            if wave[i] == 0:
                iv["block joined -> output stored (wave 0)"].append((t[i, 6] - t[i, 5]) * us)
        end = max(ends)
        if m:
            me = t[m, 0]
            m_span.append((t[m, 2].max() - me.min()) * us)
            m_comb += [(t[i, 1] - t[i, 0]) * us for i in m]
            m_store += [(t[i, 2] - t[i, 1]) * us for i in m]
            gap_dm.append((me.min() - end) * us)
            end = int(t[m, 2].max())
        layer.append((end - te.min()) * us)
        nxt = launches.get((s_ + 1, 1), [])
        if nxt:
            gap_md.append((t[nxt, 0].min() - end) * us)
    summary = {
        "launches": len(d_span), "records": int(len(rec)), "clock_hz": WAVE_CLOCK_HZ,
        "decode_wave_intervals_us_median": {k: med(v) for k, v in iv.items()},
        "decode_wave_intervals_us_p90": {k: p90(v) for k, v in iv.items()},
        "decode_dispatch_spread_us": med(d_spread), "decode_span_us": med(d_span),
        "merge_span_us": med(m_span), "merge_entry_to_combined_us": med(m_comb),
        "merge_combined_to_stored_us": med(m_store),
        "gap_decode_end_to_merge_start_us": med(gap_dm), "gap_merge_end_to_next_decode_start_us": med(gap_md),
        "layer_first_entry_to_last_store_us": med(layer),
        "decode_by_xcd": {str(k_): {"waves": len(v["end"]), "stream_us_median": med(v["stream"]),
                                    "wave_end_us_median": med(v["end"]), "last_end_us_median": med(v["last"])}
                          for k_, v in sorted(by_xcd.items())},
    }
    md = ["| decode wave (every wave of every launch) | median µs | p90 µs |", "|---|---|---|"]
    md += [f"| {k} | {summary['decode_wave_intervals_us_median'][k]} | {summary['decode_wave_intervals_us_p90'][k]} |"
           for k in iv]
    md += ["", "| per launch (median over launches) | µs |", "|---|---|",
           f"| decode: first wave entry -> last wave entry (dispatch spread) | {summary['decode_dispatch_spread_us']} |",
           f"| decode: first wave entry -> last wave's store (span seen by the waves) | {summary['decode_span_us']} |",
           f"| gap: decode's last store -> merge's first wave entry | {summary['gap_decode_end_to_merge_start_us']} |",
           f"| merge: entry -> records combined (per wave) | {summary['merge_entry_to_combined_us']} |",
           f"| merge: records combined -> output stored (per wave) | {summary['merge_combined_to_stored_us']} |",
           f"| merge: first wave entry -> last store | {summary['merge_span_us']} |",
           f"| gap: layer's last store (the merge's when one runs) -> next decode's first wave entry | "
           f"{summary['gap_merge_end_to_next_decode_start_us']} |",
           f"| layer: decode's first wave entry -> last store (the merge's when one runs) | "
           f"{summary['layer_first_entry_to_last_store_us']} |"]
    md += ["", "| decode waves by XCD (XCC id) | waves | stream median µs | wave end median µs | XCD's last end µs "
           "(median over launches) |", "|---|---|---|---|---|"]
    md += [f"| {k_} | {v['waves']} | {v['stream_us_median']} | {v['wave_end_us_median']} | {v['last_end_us_median']} |"
           for k_, v in summary["decode_by_xcd"].items()]
    md += ["", "Wave ends and last ends are measured from the launch's first wave entry; a wave's end is its "
           "block-joined point (wave 0: its store)."]
    return summary, "\n".join(md)


def read_probe(kc, vc, waves_per_row: int, waves_per_block: int, blocks_per_cu: int, split: int, steps: int,
               dev, packed: bool = True) -> dict:
    """Time the streaming-read probe (pop2-bezier_amd/csrc/ppk_read_probe.hip) on torch's current stream at a
    decode launch's geometry: one wave per (row, split-token range), each reading its range of K codes then of V
    codes in 1 KiB tiles, 4 tiles per batch, for 2, 3, 4 and 6 batches in flight. Placement "arena" reads the
    arenas `kc`/`vc` themselves at the decode's addresses (row stride = capacity * D); placement "packed" reads
    buffers of the same size whose ranges all start a power of two apart (skipped when `packed` is false). Per
    placement and ring depth: the
    average launch time over `steps` back-to-back launches (HIP events around them, after 10 warm launches) and
    the read rate."""
    import ctypes

    import torch
    from ppk.int8_kv_ops import current_stream_handle

    lib = ctypes.CDLL(os.path.join(ROOT, "pop2-bezier_amd", "ppk", "libppk_probe.so"))
    lib.ppk_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    rows, cap, D = kc.shape
    assert kc.is_contiguous() and vc.is_contiguous() and (split * D) % 4096 == 0 and cap * D % 16 == 0
    tiles = split * D // 1024
    waves = rows * waves_per_row
    assert (waves_per_row - 1) * split + split <= cap  # every range inside its row
    nbytes = waves * tiles * 1024
    out = torch.empty(waves * 64, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    placements = {"arena": (kc, vc, cap * D // 16, split * D // 16)}
    buf = None
    if packed:
        buf = torch.randint(0, 256, (2, nbytes), dtype=torch.uint8, device=dev)
        placements["packed"] = (buf[0], buf[1], waves_per_row * tiles * 64, tiles * 64)
    res = {}
    for name, (k, v, row_stride, wave_stride) in placements.items():
        res[name] = {}
        for ring in (2, 3, 4, 6):
            def launch():
                rc = lib.ppk_read_probe(ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(v.data_ptr()), tiles,
                                        waves, waves_per_block, blocks_per_cu, ring, waves_per_row, row_stride,
                                        wave_stride, ctypes.c_void_p(out.data_ptr()), current_stream_handle(dev))
                if rc != 0:
                    raise RuntimeError(f"ppk_read_probe failed ({rc})")
            for _ in range(10):
                launch()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            t0.record(stream)
            for _ in range(steps):
                launch()
            t1.record(stream)
            torch.cuda.synchronize()
            us = t0.elapsed_time(t1) / steps * 1e3
            res[name][str(ring)] = {"avg_launch_us": round(us, 2), "gbps": round(2 * nbytes / (us * 1e-6) / 1e9, 1)}
    del buf, out
    return {"kernel": "read_probe<ring> (pop2-bezier_amd/csrc/ppk_read_probe.hip, ppk/libppk_probe.so)",
            "waves": waves, "waves_per_block": waves_per_block, "blocks_per_cu": blocks_per_cu,
            "waves_per_cu": waves_per_block * blocks_per_cu, "tokens_per_wave": split, "tiles_per_range": tiles,
            "bytes_per_launch": 2 * nbytes, "launches": steps, "by_placement": res}


def _host_cpus() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _time_cpu(fn, seconds: float, max_reps: int = 1000) -> tuple[int, float]:
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= max_reps:
            return reps, el


def cpu_baseline(q, kc, vc, ks, vs, kn, vn, past, heads, args, *, threads: int | None = None,
                 rows: int | None = None, seconds: float | None = None, context: int | None = None,
                 repeat: int = 1, what: str = "") -> dict:
    """The reference's Candle CPU decode (restated in C, oracle/cpu_baseline.c) over the step's head rows.

    By default every row of the step; a smaller `rows` (or --cpu-rows) times the first rows (whole
    sequences) and scales by total/sampled rows. `repeat` scales by identical layers of one step."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # noqa: E402  (CPU baseline leg only)

    rows_total = q.shape[0]
    want = args.cpu_rows if rows is None else rows
    n = min(want, rows_total) if want else rows_total
    n -= n % heads
    n = max(n, heads)
    L = args.context if context is None else context
    q_h = q[:n].float().reshape(n, -1).cpu().numpy()
    k_h = kc[:n, :L].cpu().numpy()
    v_h = vc[:n, :L].cpu().numpy()
    ks_h = ks[:n, :L].cpu().numpy()
    vs_h = vs[:n, :L].cpu().numpy()
    sk_h = kn.float().reshape(rows_total, -1)[:n].cpu().numpy()
    sv_h = vn.float().reshape(rows_total, -1)[:n].cpu().numpy()
    past_h = past[: n // heads].cpu().numpy().astype(np.uint32)
    # Dense host copies made once, outside the timed calls (the history views skip the arena's spare slots).
    q_h, k_h, v_h, ks_h, vs_h, sk_h, sv_h = (np.ascontiguousarray(x) for x in (q_h, k_h, v_h, ks_h, vs_h, sk_h, sv_h))
    if threads is None:
        threads = _host_cpus()  # every usable core, as Candle's Rayon pool
    reps, el = _time_cpu(lambda: oracle.cpu_baseline(q_h, k_h, v_h, ks_h, vs_h, sk_h, sv_h, past_h, heads, threads),
                         args.cpu_seconds if seconds is None else seconds)
    scale = rows_total / n * repeat
    us_per_step = el / reps * 1e6 * scale
    scaled = f", scaled x{scale:g}" if scale != 1 else ""
    return {"value": round(us_per_step, 1), "unit": "us/step", "cores": threads, "kind": "port",
            "sample": f"{n} of {rows_total} head rows{what} (Candle CPU path restated in C, "
                      f"oracle/cpu_baseline.c cpu_baseline_decode, {oracle.cpu_baseline_isa()}), "
                      f"{reps} reps in {el:.1f} s{scaled}",
            "cpu_model": _cpu_model(), "host_cpus": _host_cpus()}


def bench_float(args) -> int:
    """The float-KV decode path (ppk_float_decode_attention) on a B x H x ctx bf16/f32 store that already
    holds the current token; one step = one attention call over every row's ctx tokens."""
    import numpy as np
    import torch
    import ppk

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    H, D = args.heads, args.head_dim
    if args.lengths:
        seq = parse_lengths(args.lengths)
        B, L = len(seq), max(seq)
    else:
        B, L = args.batch, args.context
        seq = [L] * B
    rows = B * H
    kv_dtype = torch.bfloat16 if args.kv == "bf16" else torch.float32
    eb = 2 if args.kv == "bf16" else 4
    print(f"# bench: float KV {args.kv} B={B} H={H} D={D} ctx={L} building store", file=sys.stderr, flush=True)
    g = torch.Generator(device=dev).manual_seed(SEED)
    k = torch.randn((rows, L, D), generator=g, device=dev, dtype=kv_dtype)
    v = torch.randn((rows, L, D), generator=g, device=dev, dtype=kv_dtype)
    q = torch.randn((rows, 1, D), generator=g, device=dev, dtype=torch.float32)
    lengths = torch.tensor(seq, dtype=torch.int32, device=dev)
    host = seq if args.lengths and not args.device_lengths else None
    two_call = None
    if args.step:
        # Each row holds lengths - 1 tokens; the step writes the current one and attends all of them.
        stored = torch.tensor([n - 1 for n in seq], dtype=torch.int32, device=dev)
        k_new = torch.randn((rows, D), generator=g, device=dev, dtype=torch.float32)
        v_new = torch.randn((rows, D), generator=g, device=dev, dtype=torch.float32)
        call = ppk.FloatDecodeStep(q, k, v, stored, H, k_new, v_new, args.split, max_length=L,
                                   lengths_host=[n - 1 for n in seq] if host else None, plan=args.plan)
        plan_args = call.args.attn
        attend = ppk.FloatDecodeAttention(q, k, v, lengths, H, args.split, max_length=L, lengths_host=host,
                                          plan=args.plan)
        row_idx = torch.arange(rows, device=dev)
        slot = stored.repeat_interleave(H).long()
        k_cast, v_cast = k_new.to(kv_dtype), v_new.to(kv_dtype)

        def two_call():
            k[row_idx, slot] = k_cast
            v[row_idx, slot] = v_cast
            attend()
    else:
        call = ppk.FloatDecodeAttention(q, k, v, lengths, H, args.split, max_length=L, lengths_host=host,
                                        plan=args.plan)
        plan_args = call.args
    # The library reports the plan it takes (ppk_float_attention_plan_info).
    flat = ppk.fused_attention.plan_info(plan_args, call.ctx)["kind"] == "balanced"
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    torch.cuda.synchronize()
    print("# bench: warmup", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        call()
    stream = torch.cuda.current_stream(dev)
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for _ in range(args.steps):
        call()
    t_end.record(stream)
    torch.cuda.synchronize()
    step_ms = t_start.elapsed_time(t_end) / args.steps
    two_call_ms = None
    if two_call is not None:
        for _ in range(args.warmup):
            two_call()
        torch.cuda.synchronize()
        t_start.record(stream)
        for _ in range(args.steps):
            two_call()
        t_end.record(stream)
        torch.cuda.synchronize()
        two_call_ms = t_start.elapsed_time(t_end) / args.steps

    ppk.kernel_stats(ppk.PPK_KERNEL_FLOAT_ATTENTION, reset=True)
    ppk.set_profiling(True)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_FLOAT_ATTENTION, reset=True)
    kernel_avg_ms = kernel_ms / max(launches, 1)

    # Algorithmic bytes: every row's K and V (its live tokens x D x element size), the f32 query and output.
    kv_bytes = sum(seq) * H * 2 * D * eb
    step_bytes = kv_bytes + rows * D * 4 + rows * D * 4
    if flat:  # the balanced decode launch; its records (a small share here) are not counted
        kernel_bytes = step_bytes
    else:
        kernel_bytes = step_bytes if call.ngroups == 1 else kv_bytes + rows * D * 4 + rows * call.ngroups * (D + 2) * 4
    achieved = kernel_bytes / (kernel_avg_ms * 1e-3) / 1e9
    step_gbps = step_bytes / (step_ms * 1e-3) / 1e9
    kname = f"ppk_{'fstep' if args.step else 'fdecode'}_{'flat_' if flat else ''}{args.kv}_d{D}"
    if args.lengths:
        skew = args.lengths.replace(",", "_")
        tpath = os.path.join(ROOT, "profiles", f"{kname}_h{H}_skew{skew}_traffic.json")
        workload = f"H{H}D{D}skew{skew}{args.kv}"
    else:
        tpath = os.path.join(ROOT, "profiles", f"ppk_fdecode_{args.kv}_d{D}_b{B}_h{H}_ctx{L}_traffic.json")
        workload = f"B{B}H{H}D{D}L{L}{args.kv}"
    traffic, traffic_source = committed_traffic(tpath, split=call.split_tokens, workload=workload, kernel=kname)
    result = {
        "metric": f"float-KV decode-{'step' if args.step else 'attention'} µs/step + achieved HBM GB/s (% of peak), "
                  f"B={B} ctx={L} {args.kv} KV" + (f", ragged lengths {args.lengths}" if args.lengths else ""),
        "value": round(step_ms * 1e3, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": args.kv,
        "data": f"synthetic (seeded torch.randn {args.kv} K/V and f32 q on the device)",
        "config": {"workload": "float-KV decode attention (ppk_float_decode_attention, the reference's "
                               "fused_attention::decode_attention)", "batch": B, "heads": H, "head_dim": D,
                   "context": L, "kv": args.kv, "query": "f32", "tokens_per_wave": call.split_tokens,
                   "blocks_per_row": call.ngroups, "launches_per_step": 1 if call.ngroups == 1 else 2,
                   "lengths": args.lengths, "plan": "balanced" if flat else "per-row",
                   "fused_step": bool(args.step)},
        "step_hbm_gbps": round(step_gbps, 1), "step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": kernel_bytes, "avg_launch_us": round(kernel_avg_ms * 1e3, 2),
                     "launches": launches},
    }
    if args.step:
        result["config"]["workload"] = ("float-KV fused decode step (ppk_float_decode_step: the graph-decode "
                                        "session's scatter_set pair + fused_attention::decode_attention)")
        result["write_then_attend_us"] = round(two_call_ms * 1e3, 2)
        result["write_then_attend_note"] = ("the reference's order on the same buffers: the current token "
                                            "written by torch indexing (two kernels), then "
                                            "ppk_float_decode_attention over lengths tokens")
    if not args.no_cpu_baseline:
        print("# bench: cpu baseline", file=sys.stderr, flush=True)
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # noqa: E402  (CPU baseline leg only)

        n = max(1, min(args.cpu_rows, rows)) if args.cpu_rows else rows
        n = max(H, n - n % H)

        def host_bits(t):
            return t.view(torch.int16).cpu().numpy().view(np.uint16) if eb == 2 else t.cpu().numpy()

        # One call per sequence over its live tokens (dense host copies made once, outside the timed calls).
        parts = [(np.ascontiguousarray(q[b * H:(b + 1) * H].cpu().numpy()),
                  np.ascontiguousarray(host_bits(k[b * H:(b + 1) * H, :seq[b]])),
                  np.ascontiguousarray(host_bits(v[b * H:(b + 1) * H, :seq[b]]))) for b in range(n // H) if seq[b]]
        threads = _host_cpus()
        reps, t0 = 0, time.perf_counter()
        while True:
            for q_h, k_h, v_h in parts:
                oracle.cpu_baseline_float(q_h, k_h, v_h, threads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds or reps >= 1000:
                break
        scale = sum(seq) / max(sum(seq[: n // H]), 1)
        result["cpu_baseline"] = {
            "value": round(el / reps * 1e6 * scale, 1), "unit": "us/step", "cores": threads, "kind": "port",
            "sample": f"{n} of {rows} head rows over their live tokens (Candle's ordinary CPU attention restated "
                      f"in C, oracle/cpu_baseline.c cpu_baseline_float_decode, {oracle.cpu_baseline_isa()}), "
                      f"{reps} reps in {el:.1f} s" + (f", scaled x{scale:g} by live tokens" if n != rows else ""),
            "cpu_model": _cpu_model(), "host_cpus": _host_cpus()}
    else:
        result["cpu_baseline"] = None
    if args.probe:
        # The float decode's own geometry (per-row plan, one block per row): the probe reads the K and V stores
        # as bytes, D * element size per token, with the decode's two batches in flight.
        info = ppk.fused_attention.plan_info(plan_args, call.ctx)
        wpb = info["waves_per_block"]
        assert not flat and call.ngroups == 1 and not args.lengths, "the probe mirrors the one-block-per-row plan"
        print("# bench: read probe", file=sys.stderr, flush=True)
        kb, vb = (t.view(torch.uint8).reshape(rows, L, D * eb) for t in (k, v))
        probe = read_probe(kb, vb, wpb, wpb, max(2, (16 if wpb > 8 else 8) // wpb), call.split_tokens, args.steps,
                           dev, packed=False)
        probe["decode_ring"] = 2
        probe["decode_frac_of_probe"] = round(achieved / probe["by_placement"]["arena"]["2"]["gbps"], 4)
        result["read_probe"] = probe
    print(json.dumps(result), flush=True)
    return 0


def bench_sampler(args) -> int:
    """The CFG + Renyi sampler (ppk_renyi_sample): one step = one call over `batch` logical rows of
    guidance x choices fp32 logits, every row's whole head legal."""
    import numpy as np
    import torch
    import ppk

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, G, C = args.batch, args.guidance, args.choices
    cfg = 2.0 if G == 2 else 1.0
    rng = np.random.default_rng(SEED)
    raw_h = (rng.standard_normal((B * G, C)) * 3).astype(np.float32)
    u_h = rng.uniform(0, 1, B).astype(np.float32)
    bounds_h = np.tile(np.array([0, C], np.uint32), (B, 1))
    raw = torch.from_numpy(raw_h).to(dev)
    u = torch.from_numpy(u_h.reshape(B, 1)).to(dev)
    bounds = torch.from_numpy(bounds_h.view(np.int32)).to(dev)
    call = ppk.RenyiSampler(raw, u, bounds, 4.0, cfg, G, 0)
    for _ in range(args.warmup):
        call()
    stream = torch.cuda.current_stream(dev)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(args.steps):
        call()
    t1.record(stream)
    torch.cuda.synchronize()
    step_ms = t0.elapsed_time(t1) / args.steps
    ppk.kernel_stats(ppk.PPK_KERNEL_RENYI_SAMPLE, reset=True)
    ppk.set_profiling(True)
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_RENYI_SAMPLE, reset=True)
    kernel_avg_ms = kernel_ms / max(launches, 1)
    kernel_bytes = B * G * C * 4 + B * 4 + B * 8 + 3 * B * 4
    achieved = kernel_bytes / (kernel_avg_ms * 1e-3) / 1e9
    result = {
        "metric": f"CFG + Renyi sampler µs/call, batch={B} guidance={G} choices={C}", "value": round(step_ms * 1e3, 2),
        "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_ms, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0, 9) logits, uniforms U[0,1), whole head legal; alpha 4)",
        "config": {"workload": "CFG + Renyi sampler (ppk_renyi_sample, the reference's hip_sampling::sample)",
                   "batch": B, "guidance": G, "choices": C, "alpha": 4.0, "cfg": cfg},
        "roofline": {"bound": "latency (hbm bytes shown)", "kernel": "ppk_renyi_sample", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 5),
                     "traffic": None, "algorithmic_bytes_per_launch": kernel_bytes,
                     "avg_launch_us": round(kernel_avg_ms * 1e3, 2), "launches": launches},
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # noqa: E402  (CPU baseline leg only)

        reps, t_start = 0, time.perf_counter()
        while True:
            oracle.renyi_sample(raw_h, u_h, bounds_h, 4.0, cfg, G, 0, cfg_fma=False)
            reps += 1
            el = time.perf_counter() - t_start
            if el >= args.cpu_seconds or reps >= 100000:
                break
        result["cpu_baseline"] = {"value": round(el / reps * 1e6, 1), "unit": "us/step", "cores": 1, "kind": "port",
                                  "sample": f"the whole batch ({B} rows), oracle_renyi_sample (the reference's host "
                                            f"oracle restated in C), {reps} reps in {el:.1f} s",
                                  "cpu_model": _cpu_model(), "host_cpus": _host_cpus()}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def bench_arena(args) -> int:
    """KV arena manager (ppk_kv_query_batch): B sequences x `layers` int8 caches prefilled with `prefill`
    tokens each (single-sequence arenas), one joining round that moves every layer's caches into a batch
    arena (committed prefixes copied once), then `steps` decode rounds of one-token appends per layer with
    one shared write plan per round."""
    import numpy as np
    import torch
    import ppk
    from ppk.kv_arena import LayerCache, WritePlan

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, D, Lyr, T0 = args.batch, args.heads, args.head_dim, args.layers, args.prefill
    print(f"# bench: arena B={B} H={H} D={D} layers={Lyr} prefill={T0}", file=sys.stderr, flush=True)
    g = torch.Generator(device=dev).manual_seed(SEED)
    prefill = torch.randn((H, T0, D), generator=g, device=dev, dtype=torch.bfloat16)
    layers = []
    # Prefill: one multi-token commit per cache (quantize-and-append of H x T0 tokens of K and V).
    ppk.kernel_stats(ppk.PPK_KERNEL_APPEND, reset=True)
    ppk.set_profiling(True)
    p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    p0.record()
    for _ in range(Lyr):
        caches = [LayerCache("int8", H, D, max_context=8192) for _ in range(B)]
        for c in caches:
            c.query(prefill, prefill, 0, True)
        layers.append(caches)
    p1.record()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    pre_launches, pre_ms = ppk.kernel_stats(ppk.PPK_KERNEL_APPEND, reset=True)
    pre_us = pre_ms / max(pre_launches, 1) * 1e3
    pre_bytes = 2 * H * T0 * D * prefill.element_size() + 2 * H * T0 * (D + 4)
    kv = torch.randn((B, H, 1, D), generator=g, device=dev, dtype=torch.bfloat16)

    # Joining round: every layer's caches move into a new batch arena.
    ppk.kernel_stats(ppk.PPK_KERNEL_COPY, reset=True)
    ppk.set_profiling(True)
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    past = [T0] * B
    plan = WritePlan(past, H, D)
    for caches in layers:
        LayerCache.query_batch(caches, kv, kv, past, True, plan)
    e1.record()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    copy_launches, copy_ms = ppk.kernel_stats(ppk.PPK_KERNEL_COPY, reset=True)
    past = [p + 1 for p in past]
    join_ms = e0.elapsed_time(e1)
    join_host_ms = (time.perf_counter() - t0) * 1e3
    # Copied bytes: committed K/V codes + scales of every row, read once and written once.
    join_bytes = 2 * Lyr * B * H * T0 * (2 * D + 8)

    # Steady decode rounds (warmup, then timed): per round one write plan and
    # one ppk_kv_query_batch per layer, called through the C-ABI with argument
    # blocks built once (the per-layer cost a native caller pays).
    import ctypes
    from ppk import _abi

    lib = _abi.lib()
    ctx = ppk.context(dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    handles = [(ctypes.c_void_p * B)(*[c.handle.value for c in caches]) for caches in layers]
    write = _abi.PpkKvWrite(struct_size=ctypes.sizeof(_abi.PpkKvWrite), src_dtype=_abi.PPK_BF16, tokens=1,
                            commit=1, k=kv.data_ptr(), v=kv.data_ptr())
    view = _abi.PpkKvView(struct_size=ctypes.sizeof(_abi.PpkKvView))
    fn = lib.ppk_kv_query_batch

    def round_():
        nonlocal past
        lens = (ctypes.c_uint32 * B)(*past)
        plan = ctypes.c_void_p()
        _abi.check(lib.ppk_write_plan_create(ctx, stream, lens, B, H, D, ctypes.byref(plan)), "plan")
        for h in handles:
            st = fn(ctx, stream, h, B, lens, ctypes.byref(write), plan, ctypes.byref(view))
            if st:
                _abi.check(st, "ppk_kv_query_batch")
        lib.ppk_write_plan_release(plan)
        past = [p + 1 for p in past]

    for _ in range(args.warmup):
        round_()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        round_()
    e1.record()
    torch.cuda.synchronize()
    round_ms = e0.elapsed_time(e1) / args.steps
    host_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ppk.kernel_stats(ppk.PPK_KERNEL_APPEND, reset=True)
    ppk.set_profiling(True)
    round_()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_APPEND, reset=True)
    append_us = kernel_ms / max(launches, 1) * 1e3
    arena_ids = {c.info().arena_id for caches in layers for c in caches}
    append_bytes = 2 * B * H * D * 2 + 2 * B * H * (D + 4)

    # Whole decode rounds, append and attention per layer (bf16 q, the current token bf16): the two-call
    # path (ppk_kv_query_batch writes the token, ppk_decode_attention reads the view) against the reserving
    # write and ppk_decode_step on the view (one launch per layer). Argument blocks are built once per
    # layer; each call refreshes the view's pointers, lengths vector and length bound.
    q_step = torch.randn((B * H, D), generator=g, device=dev, dtype=torch.bfloat16)
    out_step = torch.empty((B * H, 1, D), dtype=torch.float32, device=dev)
    reserve = _abi.PpkKvWrite(struct_size=ctypes.sizeof(_abi.PpkKvWrite), src_dtype=_abi.PPK_BF16, tokens=1,
                              commit=1, k=None, v=None)
    steps_ = [_abi.PpkDecodeStepArgs(struct_size=ctypes.sizeof(_abi.PpkDecodeStepArgs), new_dtype=_abi.PPK_BF16,
                                     k_new=kv.data_ptr(), v_new=kv.data_ptr(), flags=None) for _ in layers]
    for st_ in steps_:
        a = st_.attn
        a.struct_size, a.q_dtype, a.scratch_dtype, a.out_dtype = ctypes.sizeof(_abi.PpkAttentionArgs), 1, 1, 0
        a.rows, a.heads, a.head_dim, a.q, a.sk, a.sv, a.out = B * H, H, D, q_step.data_ptr(), kv.data_ptr(), \
            kv.data_ptr(), out_step.data_ptr()
    ws_step = torch.empty(1 << 24, dtype=torch.uint8, device=dev)

    def full_round(fused: bool):
        nonlocal past
        lens = (ctypes.c_uint32 * B)(*past)
        plan = ctypes.c_void_p()
        _abi.check(lib.ppk_write_plan_create(ctx, stream, lens, B, H, D, ctypes.byref(plan)), "plan")
        for h, st_ in zip(handles, steps_):
            _abi.check(fn(ctx, stream, h, B, lens, ctypes.byref(reserve if fused else write), plan,
                          ctypes.byref(view)), "ppk_kv_query_batch")
            a = st_.attn
            a.k_codes, a.v_codes, a.k_scales, a.v_scales = view.k, view.v, view.k_scales, view.v_scales
            a.capacity, a.past, a.max_past = view.capacity, view.past, view.length - 1
            a.workspace, a.workspace_bytes = ws_step.data_ptr(), ws_step.numel()
            if fused:
                _abi.check(lib.ppk_decode_step(ctx, stream, ctypes.byref(st_)), "ppk_decode_step")
            else:
                _abi.check(lib.ppk_decode_attention(ctx, stream, ctypes.byref(a)), "ppk_decode_attention")
        lib.ppk_write_plan_release(plan)
        past = [p + 1 for p in past]

    full = {"layers": Lyr, "tokens_at_start": past[0]}
    for fused in (False, True, False, True):
        for _ in range(10):
            full_round(fused)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            full_round(fused)
        e1.record()
        torch.cuda.synchronize()
        key = "reserve_then_decode_step" if fused else "write_then_attention"
        full.setdefault(key, []).append({"us": round(e0.elapsed_time(e1) / args.steps * 1e3, 1),
                                         "host_us": round((time.perf_counter() - t0) * 1e6 / args.steps, 1)})

    # The same prefill and join once more after every cache was released: the
    # context's pool keeps freed arenas mapped, so this join reuses memory
    # instead of mapping new pages (the first join's host time).
    del handles
    layers.clear()
    torch.cuda.synchronize()
    for _ in range(Lyr):
        caches = [LayerCache("int8", H, D, max_context=8192) for _ in range(B)]
        for c in caches:
            c.query(prefill, prefill, 0, True)
        layers.append(caches)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    past2 = [T0] * B
    plan2 = WritePlan(past2, H, D)
    for caches in layers:
        LayerCache.query_batch(caches, kv, kv, past2, True, plan2)
    e1.record()
    torch.cuda.synchronize()
    rejoin = {"ms": round(e0.elapsed_time(e1), 3), "host_ms": round((time.perf_counter() - t0) * 1e3, 2)}
    del plan2
    result = {
        "metric": f"KV arena decode round µs (append of one token per sequence into {Lyr} layers' batch arenas)",
        "value": round(round_ms * 1e3, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(round_ms, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded bf16 prefill and tokens on the device)",
        "config": {"workload": "KV arena manager (ppk_kv_query_batch with a shared ppk_write_plan per round)",
                   "batch": B, "heads": H, "head_dim": D, "layers": Lyr, "prefill": T0,
                   "arenas_after_join": len(arena_ids)},
        "host_us_per_round": round(host_ms * 1e3, 1),
        "append_kernel_us": round(append_us, 2),
        "decode_round_with_attention": full,
        "prefill": {"caches": Lyr * B, "tokens": T0, "ms": round(p0.elapsed_time(p1), 3),
                    "append_kernel_us": round(pre_us, 2), "append_bytes": pre_bytes,
                    "append_gbps": round(pre_bytes / (pre_us * 1e-6) / 1e9, 1) if pre_us else None},
        "join": {"ms": round(join_ms, 3), "host_ms": round(join_host_ms, 2), "copied_bytes": join_bytes,
                 "copy_launches": copy_launches, "copy_kernel_ms": round(copy_ms, 3),
                 "again_after_release": rejoin},
        "roofline": {"bound": "hbm", "kernel": "ppk_copy2d_batch (prefix copies at join)",
                     "achieved": round(join_bytes / (copy_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(join_bytes / (copy_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": None, "append_bytes_per_layer": append_bytes},
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # noqa: E402  (CPU baseline leg only)

        cap = 2048
        codes = np.zeros((B * H, cap, D), np.uint8)
        scales = np.zeros((B * H, cap), np.float32)
        src = kv.float().cpu().numpy()
        past_h = np.full(B, T0, np.uint32)
        reps, t_start = 0, time.perf_counter()
        while True:
            for _ in range(2 * Lyr):  # K and V of every layer
                oracle.append(src, past_h, codes, scales)
            reps += 1
            el = time.perf_counter() - t_start
            if el >= args.cpu_seconds or reps >= 10000:
                break
        result["cpu_baseline"] = {"value": round(el / reps * 1e6, 1), "unit": "us/step", "cores": 1, "kind": "port",
                                  "sample": f"one decode round: {2 * Lyr} quantize-appends of [B={B}, H={H}, 1, "
                                            f"D={D}] (oracle_append), {reps} reps in {el:.1f} s",
                                  "cpu_model": _cpu_model(), "host_cpus": _host_cpus()}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


# latency-bound shapes of the same path (the headline is config 5).
def parse_lengths(text: str) -> list:
    """--lengths: comma-separated lengths, NxL for L repeated N times, or uniform:B:LO:HI:SEED for B draws of
    numpy's default_rng(SEED).integers(LO, HI + 1)."""
    import numpy as np

    if text.startswith("uniform:"):
        b, lo, hi, seed = (int(x) for x in text.split(":")[1:])
        return [int(x) for x in np.random.default_rng(seed).integers(lo, hi + 1, size=b)]
    seq = []
    for part in text.split(","):
        n, _, length = part.strip().rpartition("x")
        seq += [int(length)] * (int(n) if n else 1)
    return seq


CONFIGS = {
    1: {"batch": 1, "heads": 16, "head_dim": 64, "lengths": [512], "layers": 1, "query": "f32",
        "workload": "BASELINE config 1: decode step (append + attention) over a 512-token int8 history, f32 q/K/V"},
    3: {"batch": 1, "heads": 16, "head_dim": 128, "lengths": [2048], "layers": 24, "query": "bf16",
        "workload": "BASELINE config 3: 24 layers x decode step (append + attention + merge) over 2048-token "
                    "int8 histories, one stream"},
    4: {"batch": 8, "heads": 16, "head_dim": 128, "lengths": None, "layers": 1, "query": "bf16",
        "workload": "BASELINE config 4: decode step over ragged int8 histories, lengths ~ U[256, 4096] (seeded)"},
}
COLD_BYTES = 1 << 30  # cold runs rotate over at least this much distinct history (>> the 256 MB MALL)


def _event_times(fn, steps: int, stream, per_step: bool):
    """Mean us over `steps` calls bracketed by two events, or the per-call durations with one event
    between consecutive calls (the event packets then count in every interval)."""
    import torch

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1 if per_step else 2)]
    torch.cuda.synchronize()
    ev[0].record(stream)
    for i in range(steps):
        fn(i)
        if per_step:
            ev[i + 1].record(stream)
    if not per_step:
        ev[1].record(stream)
    torch.cuda.synchronize()
    if per_step:
        return [ev[i].elapsed_time(ev[i + 1]) * 1e3 for i in range(steps)]
    return ev[0].elapsed_time(ev[1]) * 1e3 / steps


def bench_config(args) -> int:
    """BASELINE configs 1, 3, 4: decode steps (append of the current token + attention [+ merge]) at the
    shapes of the reference's decode calls; warm (history resident in cache where it fits) and cold
    (steps rotate over >= 1 GiB of distinct history copies, so every step reads HBM)."""
    import statistics

    import numpy as np
    import torch
    import ppk
    from ppk import synthetic

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate_copy:  # the known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        torch.neg(src, out=torch.empty_like(src))
        torch.cuda.synchronize()
        del src
    B, H, D, layers = cfg["batch"], cfg["heads"], cfg["head_dim"], cfg["layers"]
    if args.lengths:  # config 4's step over other ragged lengths (and head widths)
        lengths = parse_lengths(args.lengths)
        B, D = len(lengths), args.head_dim
    elif cfg["lengths"] is None:
        lengths = [int(x) for x in np.random.default_rng(SEED).integers(256, 4097, size=B)]
    else:
        lengths = cfg["lengths"] * B
    rows, L = B * H, max(lengths)
    cap = L + 1
    qdt = torch.float32 if cfg["query"] == "f32" else torch.bfloat16
    qb = 4 if qdt == torch.float32 else 2
    hist_bytes = sum(lengths) * H * (2 * D + 8)  # per layer: K + V codes and scales of the live history
    copies = 1 + -(-COLD_BYTES // (hist_bytes * layers))
    print(f"# bench config {args.config}: B={B} H={H} D={D} lengths={lengths} layers={layers}, "
          f"{copies} history copies for the cold runs", file=sys.stderr, flush=True)

    # One history per layer, replicated into `copies` distinct arenas.
    kc = torch.empty((copies, layers, rows, cap, D), dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty((copies, layers, rows, cap), dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    for li in range(layers):
        synthetic.fill_history(kc[0, li], vc[0, li], ks[0, li], vs[0, li], L, H, SEED + 100 * li)
    for c in range(1, copies):
        kc[c].copy_(kc[0])
        vc[c].copy_(vc[0])
        ks[c].copy_(ks[0])
        vs[c].copy_(vs[0])
    g = torch.Generator(device=dev).manual_seed(SEED + 1)
    q = [torch.randn((rows, 1, D), generator=g, device=dev).to(qdt) for _ in range(layers)]
    kn = [torch.randn((rows, 1, D), generator=g, device=dev).to(qdt) for _ in range(layers)]
    vn = [torch.randn((rows, 1, D), generator=g, device=dev).to(qdt) for _ in range(layers)]
    past = torch.tensor(lengths, dtype=torch.int32, device=dev)
    out = torch.empty((rows, 1, D), dtype=torch.float32, device=dev)
    # The caller's host copy of the lengths (the reference builds past on the host, batch.rs:152-161)
    # lets the library balance a ragged batch; --device-lengths times the plan without it.
    host = None if args.device_lengths else lengths
    steps = [[ppk.DecodeStep(q[li], kc[c, li], vc[c, li], ks[c, li], vs[c, li], kn[li], vn[li], past, H,
                             split_tokens=args.split, max_past=L, out=out, past_host=host, plan=args.plan)
              for li in range(layers)]
             for c in range(copies)]
    split, ngroups = steps[0][0].split_tokens, steps[0][0].ngroups
    # The library reports the plan it takes (ppk_attention_plan_info): per-row or balanced, its waves per
    # block and its launches (decode, + merge).
    info = steps[0][0].plan_info
    balanced = info["kind"] == "balanced"
    layer_launches = info["launches"]
    torch.cuda.synchronize()

    def warm(_i):
        for s in steps[0]:
            s()

    def cold(i):
        for s in steps[i % copies]:
            s()

    stream = torch.cuda.current_stream(dev)
    print("# bench: warmup", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        warm(i)
    warm_mean = _event_times(warm, args.steps, stream, per_step=False)
    warm_each = _event_times(warm, args.steps, stream, per_step=True)
    for i in range(copies):
        cold(i)
    cold_mean = _event_times(lambda i: cold(i + 1), args.steps, stream, per_step=False)
    cold_each = _event_times(lambda i: cold(i + 1), args.steps, stream, per_step=True)

    # Graph replay of the warm step: the same launches with the host side removed.
    graph_us = None
    try:
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            warm(0)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            warm(0)
        for _ in range(10):
            graph.replay()
        graph_us = _event_times(lambda _i: graph.replay(), args.steps, stream, per_step=False)
        del graph
    except RuntimeError as e:  # capture unsupported on this stack: report eager numbers only
        print(f"# bench: graph replay skipped: {e}", file=sys.stderr, flush=True)

    # Roofline of the decode kernel (and the merge kernel when rows span blocks), traced launches, warm.
    ppk.kernel_stats(ppk.PPK_KERNEL_ATTENTION, reset=True)
    ppk.kernel_stats(ppk.PPK_KERNEL_ATTN_MERGE, reset=True)
    ppk.set_profiling(True)
    for i in range(args.steps):
        warm(i)
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_ATTENTION, reset=True)
    m_launches, merge_ms = ppk.kernel_stats(ppk.PPK_KERNEL_ATTN_MERGE, reset=True)
    kernel_avg_us = kernel_ms / max(launches, 1) * 1e3

    # Algorithmic bytes of one layer: live history + q + current k, v + f32 out + appended codes/scales.
    layer_bytes = hist_bytes + rows * D * qb + 2 * rows * D * qb + rows * D * 4 + 2 * rows * (D + 4)
    kernel_bytes = layer_bytes if ngroups == 1 else layer_bytes - rows * D * 4
    step_bytes = layer_bytes * layers
    achieved = kernel_bytes / (kernel_avg_us * 1e-6) / 1e9
    tag = f"c{args.config}_b{B}_h{H}_d{D}"
    kbase = "ppk_decode_flat" if balanced else "ppk_decode"
    kname = f"{kbase}_d{D}"
    tpath = os.path.join(ROOT, "profiles", f"{kbase}_{tag}_traffic.json")
    traffic, traffic_source = committed_traffic(tpath, split=split, workload=tag)

    result = {
        "metric": METRIC, "value": round(warm_mean, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(warm_mean / 1e3, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) with 2% heavy-tailed 10*t3 channels, quantised on device; "
                f"{cfg['query']} q and current K/V)",
        "config": {"workload": (f"config 4's decode step over ragged int8 histories, lengths {args.lengths}"
                                if args.lengths else cfg["workload"]),
                   "batch": B, "heads": H, "head_dim": D, "lengths": lengths,
                   "layers": layers, "capacity": cap, "kv": "int8 + f32 scales", "query": cfg["query"],
                   "plan": "balanced work list (host lengths)" if balanced else "per-row blocks",
                   "tokens_per_wave": split, ("units_per_row_max" if balanced else "blocks_per_row"): ngroups,
                   "launches_per_step": layers * layer_launches},
        "median_us": round(statistics.median(warm_each), 2),
        "cold": {"mean_us": round(cold_mean, 2), "median_us": round(statistics.median(cold_each), 2),
                 "history_copies": copies, "rotated_bytes": copies * hist_bytes * layers,
                 "step_hbm_gbps": round(step_bytes / (cold_mean * 1e-6) / 1e9, 1)},
        "per_step_events_note": "median_us values come from a pass with one event between consecutive steps",
        "graph_replay_us": None if graph_us is None else round(graph_us, 2),
        "algorithmic_bytes_per_step": step_bytes,
        "step_hbm_gbps": round(step_bytes / (warm_mean * 1e-6) / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": kname,
                     "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": kernel_bytes,
                     "avg_launch_us": round(kernel_avg_us, 2), "launches": launches,
                     "merge_avg_launch_us": round(merge_ms / m_launches * 1e3, 2) if m_launches else None},
    }
    if args.wave_clock:
        print("# bench: wave clock", file=sys.stderr, flush=True)
        summary, md = wave_clock_run(lambda: warm(0), steps[0], min(args.steps, 10), dev,
                                     os.environ.get("PPK_WAVE_CLOCK_RAW"))
        result["wave_clock"] = summary
        cmd = "python3 bench.py " + " ".join(sys.argv[1:])
        with open(args.wave_clock, "w") as f:
            f.write(f"# Wave clock: BASELINE config {args.config} ({cfg['workload']})\n\n"
                    f"Command (from the repository root):\n\n    {cmd}\n\n"
                    f"{min(args.steps, 10)} warm steps ({summary['launches']} decode launches, "
                    f"{summary['records']} wave records) on a context made from "
                    "pop2-bezier_amd/ppk/ppk_kernels_clock.hsaco (the library's kernels built with "
                    "-DPPK_WAVE_CLOCK: each wave reads the 100 MHz real-time clock at fixed points and writes "
                    "one record to a slot of its own; layout in pop2-bezier_amd/csrc/ppk_kernel_args.h). A point "
                    "\"x here\" waits for "
                    "x first. Per-layer decode + merge launches, one stream, as the timed steps.\n\n" + md + "\n")
    if not args.no_cpu_baseline:
        print("# bench: cpu baseline", file=sys.stderr, flush=True)
        a = (q[0], kc[0, 0], vc[0, 0], ks[0, 0], vs[0, 0], kn[0], vn[0], past, H, args)
        what = f" x {L} tokens" if len(set(lengths)) == 1 else " (ragged)"
        what += f", one of {layers} identical layers" if layers > 1 else ""
        result["cpu_baseline"] = cpu_baseline(*a, rows=rows, context=L, repeat=layers, what=what,
                                              seconds=args.cpu_seconds / 2)
        result["cpu_baseline_1thread"] = cpu_baseline(*a, threads=1, rows=rows, context=L, repeat=layers, what=what,
                                                      seconds=args.cpu_seconds / 2)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def bench_append(args) -> int:
    """append only. One fp16 token of K and V for B=1, H=16, D=128 quantised into
    slot 1000 of capacity-4096 int8 arenas (ppk_quantize_append); latency-bound, its parity bar is
    bit-exactness (tests/test_gpu_quantize.py). Warm and cold (rotating arena copies) timings."""
    import statistics

    import numpy as np
    import torch
    import ppk
    from ppk import synthetic

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, D, cap, filled = 1, 16, 128, 4096, 1000
    rows = B * H
    copies = 1 + -(-COLD_BYTES // (2 * rows * cap * (D + 4)))
    kc = torch.zeros((copies, rows, cap, D), dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((copies, rows, cap), dtype=torch.float32, device=dev)
    vs = torch.zeros_like(ks)
    synthetic.fill_history(kc[0], vc[0], ks[0], vs[0], filled, H, SEED)
    kn = synthetic.history_chunk(SEED, 2, 0, rows, H, 0, 1, D, dev, torch.float16).reshape(B, H, 1, D).contiguous()
    vn = synthetic.history_chunk(SEED, 3, 0, rows, H, 0, 1, D, dev, torch.float16).reshape(B, H, 1, D).contiguous()
    past = torch.full((B,), filled, dtype=torch.int32, device=dev)
    calls = [ppk.AppendKV(kn, vn, past, kc[c], vc[c], ks[c], vs[c]) for c in range(copies)]
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        calls[0]()
    warm_mean = _event_times(lambda _i: calls[0](), args.steps, stream, per_step=False)
    warm_each = _event_times(lambda _i: calls[0](), args.steps, stream, per_step=True)
    cold_mean = _event_times(lambda i: calls[1 + i % (copies - 1)](), args.steps, stream, per_step=False)
    ppk.kernel_stats(ppk.PPK_KERNEL_APPEND, reset=True)
    ppk.set_profiling(True)
    for _ in range(args.steps):
        calls[0]()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_APPEND, reset=True)
    kernel_avg_us = kernel_ms / max(launches, 1) * 1e3
    nbytes = 2 * rows * D * 2 + 2 * rows * (D + 4)  # read fp16 K, V; write codes + scales
    achieved = nbytes / (kernel_avg_us * 1e-6) / 1e9
    result = {
        "metric": METRIC, "value": round(warm_mean, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(warm_mean / 1e3, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded N(0,1) with 2% heavy-tailed 10*t3 channels, fp16 new K/V)",
        "config": {"workload": "BASELINE config 2: append only, one fp16 token of K and V into slot 1000 of "
                               "capacity-4096 int8 arenas (ppk_quantize_append)",
                   "batch": B, "heads": H, "head_dim": D, "capacity": cap, "slot": filled},
        "median_us": round(statistics.median(warm_each), 2),
        "cold": {"mean_us": round(cold_mean, 2), "arena_copies": copies},
        "roofline": {"bound": "hbm", "kernel": "ppk_quantize_d%d (append)" % D, "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 6),
                     "traffic": None, "algorithmic_bytes_per_launch": nbytes,
                     "avg_launch_us": round(kernel_avg_us, 2), "launches": launches,
                     "note": "latency-bound: 8.7 KB per launch"},
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # noqa: E402  (CPU baseline leg only)

        src = np.stack([kn.float().cpu().numpy(), vn.float().cpu().numpy()])
        past_h = np.array([filled], np.uint32)
        arenas = [(kc[0].cpu().numpy(), ks[0].cpu().numpy()), (vc[0].cpu().numpy(), vs[0].cpu().numpy())]

        def cpu_append():
            for x, (codes, scales) in zip(src, arenas):
                oracle.append(x, past_h, codes, scales)

        reps, el = _time_cpu(cpu_append, args.cpu_seconds / 2, max_reps=100000)
        result["cpu_baseline"] = {"value": round(el / reps * 1e6, 2), "unit": "us/step", "cores": 1, "kind": "port",
                                  "sample": f"the whole append (K and V, 16 rows x {D}), C oracle oracle_append, "
                                            f"{reps} reps in {el:.1f} s",
                                  "cpu_model": _cpu_model(), "host_cpus": _host_cpus()}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def bench_quantize(args) -> int:
    """Dense quantization (ppk_quantize, the bit-exact contract of int8_kv_ops::quantize) of one history
    tensor at the headline shape: B*H rows x ctx tokens x D values of DTYPE -> codes + one f32 scale per
    token row."""
    import ctypes
    import statistics

    import torch
    import ppk
    from ppk import _abi, synthetic
    from ppk import int8_kv_ops as ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, D, L = args.batch, args.heads, args.head_dim, args.context
    rows = B * H
    dt = {"bf16": torch.bfloat16, "f32": torch.float32, "f16": torch.float16}[args.quantize]
    print(f"# bench quantize: {rows} rows x {L} tokens x {D} {args.quantize}", file=sys.stderr, flush=True)
    x = torch.empty((rows, L, D), dtype=dt, device=dev)
    for r0 in range(0, rows, 16):
        x[r0:r0 + 16].copy_(synthetic.history_chunk(SEED, 0, r0 // 16, min(16, rows - r0), H, r0, L, D, dev, dt))
    codes = torch.empty((rows, L, D), dtype=torch.uint8, device=dev)
    scales = torch.empty((rows, L), dtype=torch.float32, device=dev)
    a = _abi.PpkQuantizeArgs(struct_size=ctypes.sizeof(_abi.PpkQuantizeArgs), src_dtype=ops._DTYPES[dt],
                             src=x.data_ptr(), codes=codes.data_ptr(), scales=scales.data_ptr(), rows=rows * L,
                             head_dim=D, flags=None)
    ctx, fn, ref = ops.context(dev), ops.lib().ppk_quantize, ctypes.byref(a)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        torch.neg(src, out=torch.empty_like(src))
        torch.cuda.synchronize()
        del src

    def call(_i=0):
        ops.check(fn(ctx, sp, ref), "ppk_quantize")

    for _ in range(args.warmup):
        call()
    mean_us = _event_times(call, args.steps, stream, per_step=False)
    each = _event_times(call, args.steps, stream, per_step=True)
    ppk.kernel_stats(ppk.PPK_KERNEL_QUANTIZE, reset=True)
    ppk.set_profiling(True)
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_QUANTIZE, reset=True)
    kernel_us = kernel_ms / max(launches, 1) * 1e3
    nbytes = rows * L * D * x.element_size() + rows * L * D + rows * L * 4
    achieved = nbytes / (kernel_us * 1e-6) / 1e9
    tpath = os.path.join(ROOT, "profiles", f"ppk_quantize_{args.quantize}_b{B}_h{H}_d{D}_ctx{L}_traffic.json")
    traffic, traffic_source = committed_traffic(tpath, workload=f"B{B}H{H}D{D}L{L}{args.quantize}")
    result = {
        "metric": "%s -> int8 quantize, us per history tensor + achieved HBM GB/s" % args.quantize,
        "value": round(mean_us, 2), "unit": "us/call", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(mean_us / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": args.quantize, "data": "synthetic (seeded N(0,1) with 2% heavy-tailed 10*t3 channels)",
        "config": {"workload": "quantize one history tensor (ppk_quantize)", "rows": rows, "tokens": L,
                   "head_dim": D, "src": args.quantize},
        "median_us": round(statistics.median(each), 2),
        "step_hbm_gbps": round(nbytes / (mean_us * 1e-6) / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "ppk_quantize_d%d" % D, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(kernel_us, 2),
                     "launches": launches},
    }
    if not args.no_cpu_baseline:
        import numpy as np
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # noqa: E402  (CPU baseline leg only)

        n = min(rows, 4)
        xh = x[:n].float().cpu().numpy()
        reps, el = _time_cpu(lambda: oracle.quantize(xh), args.cpu_seconds / 2)
        result["cpu_baseline"] = {"value": round(el / reps * 1e6 * rows / n, 1), "unit": "us/call", "cores": 1,
                                  "kind": "port",
                                  "sample": f"{n} of {rows} rows x {L} tokens (C oracle oracle_quantize, the "
                                            f"reference's CPU branch restated), {reps} reps in {el:.1f} s, "
                                            f"scaled x{rows / n:g}",
                                  "cpu_model": _cpu_model(), "host_cpus": _host_cpus()}
        del np
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def bench_dequantize(args) -> int:
    """Int8 -> bf16/f32/f16 dequantization (ppk_dequantize, the prefill path's `dequantize`) of one history
    tensor at the headline shape: B*H rows x ctx tokens x D codes + one f32 scale per token."""
    import ctypes
    import statistics

    import numpy as np
    import torch
    import ppk
    from ppk import _abi, synthetic
    from ppk import int8_kv_ops as ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, D, L = args.batch, args.heads, args.head_dim, args.context
    rows = B * H
    dt = {"bf16": torch.bfloat16, "f32": torch.float32, "f16": torch.float16}[args.dequantize]
    print(f"# bench dequantize: {rows} rows x {L} tokens x {D} -> {args.dequantize}", file=sys.stderr, flush=True)
    kc = torch.empty((rows, L, D), dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty((rows, L), dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    synthetic.fill_history(kc, vc, ks, vs, L, H, SEED)
    del vc, vs
    out = torch.empty((rows, L, D), dtype=dt, device=dev)
    a = _abi.PpkDequantizeArgs(struct_size=ctypes.sizeof(_abi.PpkDequantizeArgs), out_dtype=ops._DTYPES[dt],
                               codes=kc.data_ptr(), scales=ks.data_ptr(), out=out.data_ptr(), rows=rows * L,
                               head_dim=D, round_bf16=0)
    ctx, fn, ref = ops.context(dev), ops.lib().ppk_dequantize, ctypes.byref(a)
    stream = torch.cuda.current_stream(dev)
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        torch.neg(src, out=torch.empty_like(src))
        torch.cuda.synchronize()
        del src
    sp = ctypes.c_void_p(stream.cuda_stream)

    def call(_i=0):
        ops.check(fn(ctx, sp, ref), "ppk_dequantize")

    for _ in range(args.warmup):
        call()
    mean_us = _event_times(call, args.steps, stream, per_step=False)
    each = _event_times(call, args.steps, stream, per_step=True)
    ppk.kernel_stats(ppk.PPK_KERNEL_DEQUANTIZE, reset=True)
    ppk.set_profiling(True)
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_DEQUANTIZE, reset=True)
    kernel_us = kernel_ms / max(launches, 1) * 1e3
    nbytes = rows * L * D + rows * L * 4 + rows * L * D * out.element_size()
    achieved = nbytes / (kernel_us * 1e-6) / 1e9
    tpath = os.path.join(ROOT, "profiles", f"ppk_dequantize_{args.dequantize}_b{B}_h{H}_d{D}_ctx{L}_traffic.json")
    traffic, traffic_source = committed_traffic(tpath, workload=f"B{B}H{H}D{D}L{L}{args.dequantize}")
    result = {
        "metric": "int8 -> %s dequantize, us per history tensor + achieved HBM GB/s" % args.dequantize,
        "value": round(mean_us, 2), "unit": "us/call", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(mean_us / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic (seeded N(0,1) with 2% heavy-tailed 10*t3 channels, quantised on device)",
        "config": {"workload": "dequantize one int8 history tensor (ppk_dequantize)", "rows": rows, "tokens": L,
                   "head_dim": D, "out": args.dequantize},
        "median_us": round(statistics.median(each), 2),
        "step_hbm_gbps": round(nbytes / (mean_us * 1e-6) / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "ppk_dequantize", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": nbytes, "avg_launch_us": round(kernel_us, 2),
                     "launches": launches},
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # noqa: E402  (CPU baseline leg only)

        n = min(rows, 16)
        c_h, s_h = kc[:n].cpu().numpy(), ks[:n].cpu().numpy()
        reps, el = _time_cpu(lambda: oracle.dequantize(c_h, s_h, round_bf16=dt == torch.bfloat16), args.cpu_seconds / 2)
        result["cpu_baseline"] = {"value": round(el / reps * 1e6 * rows / n, 1), "unit": "us/call", "cores": 1,
                                  "kind": "port",
                                  "sample": f"{n} of {rows} rows x {L} tokens (C oracle oracle_dequantize, f32 out"
                                            f"{' rounded to bf16' if dt == torch.bfloat16 else ''}), {reps} reps "
                                            f"in {el:.1f} s, scaled x{rows / n:g}",
                                  "cpu_model": _cpu_model(), "host_cpus": _host_cpus()}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the int8 KV decode path shards by "
                                   "sequence or head with no collective on the hot path; run it once per GPU",
                          "n_gpus": args.gpus}))
        return 2
    if args.plan == "balanced" and args.device_lengths:
        print("bench.py: --plan balanced needs the host lengths; drop --device-lengths", file=sys.stderr)
        return 2
    if args.sampler:
        return bench_sampler(args)
    if args.arena:
        return bench_arena(args)
    if args.dequantize:
        return bench_dequantize(args)
    if args.quantize:
        return bench_quantize(args)
    if args.kv != "int8":
        return bench_float(args)
    if args.config == 2:
        return bench_append(args)
    if args.lengths and args.config != 4:
        print("bench.py: --lengths takes --kv bf16|f32 or --config 4", file=sys.stderr)
        return 2
    if args.config != 5:
        return bench_config(args)
    import torch
    import ppk
    from ppk import synthetic

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, D, L = args.batch, args.heads, args.head_dim, args.context
    rows, cap = B * H, L + 1
    print(f"# bench: B={B} H={H} D={D} ctx={L} building arenas", file=sys.stderr, flush=True)
    kc = torch.empty((rows, cap, D), dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty((rows, cap), dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    synthetic.fill_history(kc, vc, ks, vs, L, H, SEED)
    g = torch.Generator(device=dev).manual_seed(SEED + 1)
    q = torch.randn((rows, 1, D), generator=g, device=dev).to(torch.bfloat16)
    kn = synthetic.history_chunk(SEED, 2, 0, rows, H, 0, 1, D, dev, torch.bfloat16).reshape(B, H, 1, D).contiguous()
    vn = synthetic.history_chunk(SEED, 3, 0, rows, H, 0, 1, D, dev, torch.bfloat16).reshape(B, H, 1, D).contiguous()
    past = torch.full((B,), L, dtype=torch.int32, device=dev)
    out = torch.empty((rows, 1, D), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    # The current token is both attended from its bf16 copy (sk, sv) and
    # committed into slot L of the arenas, in one launch; with --no-append it
    # is only attended (the reference's uncommitted partial queries).
    append = not args.no_append
    if append:
        step = ppk.DecodeStep(q, kc, vc, ks, vs, kn.reshape(rows, 1, D), vn.reshape(rows, 1, D), past, H,
                              split_tokens=args.split, max_past=L, out=out, bf16_history=args.bf16_history)
    else:
        step = ppk.DecodeAttention(q, kc, vc, ks, vs, kn.reshape(rows, 1, D), vn.reshape(rows, 1, D), past, H,
                                   split_tokens=args.split, max_past=L, out=out, bf16_history=args.bf16_history)
    split = step.split_tokens

    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    print("# bench: warmup", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region 1 (the reported value): K back-to-back steps bracketed by
    # events, synchronised on both sides.
    stream = torch.cuda.current_stream(dev)
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    step_ms = t_start.elapsed_time(t_end) / args.steps
    # Median from a second pass with an event between consecutive steps.
    import statistics
    median_us = statistics.median(_event_times(lambda _i: step(), args.steps, stream, per_step=True))

    # Timed region 2 (the roofline): the same K steps with the library's tracer
    # bracketing every launch of the decode kernel with HIP events on the
    # stream it is launched on. The extra event packets cost a few us per step,
    # which is why the step value comes from region 1.
    ppk.kernel_stats(ppk.PPK_KERNEL_ATTENTION, reset=True)
    ppk.set_profiling(True)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_ATTENTION, reset=True)
    kernel_avg_ms = kernel_ms / max(launches, 1)
    clock = None
    if args.wave_clock:
        print("# bench: wave clock", file=sys.stderr, flush=True)
        clock, md = wave_clock_run(step, [step], min(args.steps, 10), dev, os.environ.get("PPK_WAVE_CLOCK_RAW"))
        with open(args.wave_clock, "w") as f:
            f.write(f"# Wave clock: B={B} H={H} D={D} ctx={L} int8 decode "
                    f"{'step' if not args.no_append else 'attention'}\n\n"
                    f"Command (from the repository root):\n\n    python3 bench.py {' '.join(sys.argv[1:])}\n\n"
                    f"{min(args.steps, 10)} back-to-back steps on a context made from "
                    "pop2-bezier_amd/ppk/ppk_kernels_clock.hsaco (wave-clock build; record layout in "
                    "pop2-bezier_amd/csrc/ppk_kernel_args.h).\n\n" + md + "\n")

    # Algorithmic bytes of one step: history K+V codes and scales of every
    # row, the bf16 query, the bf16 current K/V token (read once: quantised
    # into the arena and scored as the current token), the f32 output and the
    # appended codes + scales: sum_b L_b*H*(2D+8) + q + current k,v + out + append.
    # Without the append: the same less the appended codes + scales.
    hist_bytes = rows * L * (2 * D + 8)
    app_bytes = 2 * rows * (D + 4) if append else 0
    step_bytes = hist_bytes + rows * D * 2 + 2 * rows * D * 2 + rows * D * 4 + app_bytes
    kernel_bytes = step_bytes if step.ngroups == 1 else hist_bytes + rows * D * 2 + app_bytes + 2 * rows * D * 2
    achieved = kernel_bytes / (kernel_avg_ms * 1e-3) / 1e9
    step_gbps = step_bytes / (step_ms * 1e-3) / 1e9

    kname = "ppk_decode" + ("_bf16h" if args.bf16_history else "") + f"_d{D}"
    tag = ("_bf16h" if args.bf16_history else "") + ("" if append else "_noappend")
    tpath = args.traffic or os.path.join(ROOT, "profiles", f"ppk_decode_d{D}_b{B}_h{H}_ctx{L}{tag}_traffic.json")
    traffic, traffic_source = committed_traffic(tpath, split=split, workload=f"B{B}H{H}D{D}L{L}", kernel=kname,
                                                algorithmic_bytes_per_launch=kernel_bytes)
    workload = ("BASELINE config 5: decode step = append of the current token + attention over the int8 history "
                "(ppk_decode_step)" if append else
                "BASELINE config 5 shape, uncommitted query: attention over the int8 history + the current token "
                "from its copy, nothing appended (ppk_decode_attention)")

    result = {
        "metric": METRIC,
        "value": round(step_ms * 1e3, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) with 2% heavy-tailed 10*t3 channels, quantised on device; bf16 q and new K/V)",
        "config": {"workload": workload,
                   "batch": B, "heads": H, "head_dim": D, "context": L, "capacity": cap, "kv": "int8 + f32 scales",
                   "history": "bf16-rounded (PPK_ATTN_BF16_HISTORY)" if args.bf16_history else "fp32 dequantised",
                   "query": "bf16", "tokens_per_wave": split, "blocks_per_row": step.ngroups,
                   "launches_per_step": 1 if step.ngroups == 1 else 2},
        "median_us": round(median_us, 2),
        "tokens_per_s": round(B / (step_ms * 1e-3), 1),
        "step_hbm_gbps": round(step_gbps, 1),
        "step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": kernel_bytes,
                     "avg_launch_us": round(kernel_avg_ms * 1e3, 2), "launches": launches},
    }
    if not args.no_cpu_baseline:
        print("# bench: cpu baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(q, kc, vc, ks, vs, kn, vn, past, H, args, what=f" x {L} tokens")
        result["cpu_baseline_1thread"] = cpu_baseline(q, kc, vc, ks, vs, kn, vn, past, H, args, threads=1,
                                                      seconds=args.cpu_seconds / 2, what=f" x {L} tokens")
    else:
        result["cpu_baseline"] = None
    if clock is not None:
        result["wave_clock"] = clock
    if args.probe:
        print("# bench: read probe", file=sys.stderr, flush=True)
        info = step.plan_info
        wpb = info["waves_per_block"]
        assert info["kind"] == "per-row" and step.ngroups == 1, "the probe mirrors the one-block-per-row plan"
        probe = read_probe(kc, vc, wpb, wpb, max(2, 8 // wpb), split, args.steps, dev)
        ring = 3  # the int8 decode kernel's batches in flight
        at_ring = probe["by_placement"]["arena"][str(ring)]["gbps"]
        probe["decode_ring"] = ring
        probe["decode_frac_of_probe"] = round(achieved / at_ring, 4)
        if wpb % 2 == 0 and wpb * split <= cap:  # wpb / 2 waves of 2 * split tokens per row
            # Half the waves per CU, each streaming twice the tokens: the same bytes with 16-24 KiB in flight
            # per wave at rings 4 and 6, for comparison with the decode's shape.
            half = read_probe(kc, vc, wpb // 2, wpb // 2, max(2, 8 // wpb), 2 * split, args.steps, dev,
                              packed=False)
            probe["half_waves_per_cu"] = {k: half[k] for k in ("waves", "waves_per_block", "blocks_per_cu",
                                                               "waves_per_cu", "tokens_per_wave", "by_placement")}
        result["read_probe"] = probe
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
