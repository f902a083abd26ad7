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
    p.add_argument("--kv", choices=("int8", "bf16", "f32"), default="int8",
                   help="int8 (default, the headline workload) or the float-KV decode path over a bf16/f32 store")
    p.add_argument("--sampler", action="store_true",
                   help="time the CFG + Renyi sampler instead (batch = --batch, --choices, --guidance)")
    p.add_argument("--arena", action="store_true",
                   help="time the KV arena manager: joining prefilled caches into batch arenas, then decode rounds "
                        "of one-token appends over --layers layers with a shared write plan")
    p.add_argument("--layers", type=int, default=24)
    p.add_argument("--prefill", type=int, default=1000)
    p.add_argument("--choices", type=int, default=2048)
    p.add_argument("--guidance", type=int, default=2)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-rows", type=int, default=64, help="head rows timed for the CPU baseline sample")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--calibrate-copy", action="store_true",
                   help="run one plain 1 GiB elementwise copy (torch.neg, f32) first: the known-size kernel that "
                        "scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings")
    p.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "ppk_decode_d128_b32_h16_ctx8192_traffic.json"),
                   help="JSON with measured HBM bytes per partial launch (rocprofv3 --pmc), if present")
    return p.parse_args()


def cpu_baseline(q, kc, vc, ks, vs, kn, vn, past, heads, args) -> dict:
    """The reference's Candle CPU decode (restated in C, oracle/) on a bounded sample of head rows."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # noqa: E402  (CPU baseline leg only)

    rows_total = q.shape[0]
    n = min(args.cpu_rows, rows_total)
    n -= n % heads
    n = max(n, heads)
    L = args.context
    q_h = q[:n].float().reshape(n, -1).cpu().numpy()
    k_h = kc[:n, :L].cpu().numpy()
    v_h = vc[:n, :L].cpu().numpy()
    ks_h = ks[:n, :L].cpu().numpy()
    vs_h = vs[:n, :L].cpu().numpy()
    sk_h = kn.float().reshape(rows_total, -1)[:n].cpu().numpy()
    sv_h = vn.float().reshape(rows_total, -1)[:n].cpu().numpy()
    past_h = past[: n // heads].cpu().numpy().astype(np.uint32)
    threads = max(1, min(os.cpu_count() or 1, 16))
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.cpu_baseline(q_h, k_h, v_h, ks_h, vs_h, sk_h, sv_h, past_h, heads, threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or reps >= 1000:
            break
    per_rep_us = el / reps * 1e6
    us_per_step = per_rep_us * rows_total / n
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(us_per_step, 1), "unit": "us/step", "cores": threads, "kind": "port",
            "sample": f"{n} of {rows_total} head rows x {L} tokens (Candle CPU path restated in C, "
                      f"oracle/ppk_oracle.c cpu_baseline_decode), {reps} reps in {el:.1f} s, scaled x{rows_total / n:g}",
            "cpu_model": model}


def bench_float(args) -> int:
    """The float-KV decode path (ppk_float_decode_attention) on a B x H x ctx bf16/f32 store that already
    holds the current token; one step = one attention call over every row's ctx tokens."""
    import numpy as np
    import torch
    import ppk

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, H, D, L = args.batch, args.heads, args.head_dim, args.context
    rows = B * H
    kv_dtype = torch.bfloat16 if args.kv == "bf16" else torch.float32
    eb = 2 if args.kv == "bf16" else 4
    print(f"# bench: float KV {args.kv} B={B} H={H} D={D} ctx={L} building store", file=sys.stderr, flush=True)
    g = torch.Generator(device=dev).manual_seed(SEED)
    k = torch.randn((rows, L, D), generator=g, device=dev, dtype=kv_dtype)
    v = torch.randn((rows, L, D), generator=g, device=dev, dtype=kv_dtype)
    q = torch.randn((rows, 1, D), generator=g, device=dev, dtype=torch.float32)
    lengths = torch.full((B,), L, dtype=torch.int32, device=dev)
    call = ppk.FloatDecodeAttention(q, k, v, lengths, H, args.split, max_length=L)
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

    ppk.kernel_stats(ppk.PPK_KERNEL_FLOAT_ATTENTION, reset=True)
    ppk.set_profiling(True)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    ppk.set_profiling(False)
    launches, kernel_ms = ppk.kernel_stats(ppk.PPK_KERNEL_FLOAT_ATTENTION, reset=True)
    kernel_avg_ms = kernel_ms / max(launches, 1)

    # Algorithmic bytes: every row's K and V (L tokens x D x element size), the f32 query and output.
    kv_bytes = rows * L * 2 * D * eb
    step_bytes = kv_bytes + rows * D * 4 + rows * D * 4
    kernel_bytes = step_bytes if call.ngroups == 1 else kv_bytes + rows * D * 4 + rows * call.ngroups * (D + 2) * 4
    achieved = kernel_bytes / (kernel_avg_ms * 1e-3) / 1e9
    step_gbps = step_bytes / (step_ms * 1e-3) / 1e9
    kname = f"ppk_fdecode_{args.kv}_d{D}"
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"ppk_fdecode_{args.kv}_d{D}_b{B}_h{H}_ctx{L}_traffic.json")
    if os.path.exists(tpath):
        try:
            with open(tpath) as f:
                t = json.load(f)
            if (t.get("split") == call.split_tokens and t.get("workload") == f"B{B}H{H}D{D}L{L}{args.kv}"
                    and t.get("kernel") == kname):
                traffic = t.get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    result = {
        "metric": f"float-KV decode-attention µs/step + achieved HBM GB/s (% of peak), B={B} ctx={L} {args.kv} KV",
        "value": round(step_ms * 1e3, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": args.kv,
        "data": f"synthetic (seeded torch.randn {args.kv} K/V and f32 q on the device)",
        "config": {"workload": "float-KV decode attention (ppk_float_decode_attention, the reference's "
                               "fused_attention::decode_attention)", "batch": B, "heads": H, "head_dim": D,
                   "context": L, "kv": args.kv, "query": "f32", "tokens_per_wave": call.split_tokens,
                   "blocks_per_row": call.ngroups, "launches_per_step": 1 if call.ngroups == 1 else 2},
        "step_hbm_gbps": round(step_gbps, 1), "step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": kernel_bytes, "avg_launch_us": round(kernel_avg_ms * 1e3, 2),
                     "launches": launches},
    }
    if not args.no_cpu_baseline:
        print("# bench: cpu baseline", file=sys.stderr, flush=True)
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle  # noqa: E402  (CPU baseline leg only)

        n = max(1, min(args.cpu_rows, rows))
        if eb == 2:
            k_h = k[:n].view(torch.int16).cpu().numpy().view(np.uint16)
            v_h = v[:n].view(torch.int16).cpu().numpy().view(np.uint16)
        else:
            k_h, v_h = k[:n].cpu().numpy(), v[:n].cpu().numpy()
        q_h = q[:n].cpu().numpy()
        threads = max(1, min(os.cpu_count() or 1, 16))
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.cpu_baseline_float(q_h, k_h, v_h, threads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds or reps >= 1000:
                break
        result["cpu_baseline"] = {
            "value": round(el / reps * 1e6 * rows / n, 1), "unit": "us/step", "cores": threads, "kind": "port",
            "sample": f"{n} of {rows} head rows x {L} tokens (Candle's ordinary CPU attention restated in C, "
                      f"cpu_baseline_float_decode), {reps} reps in {el:.1f} s, scaled x{rows / n:g}"}
    else:
        result["cpu_baseline"] = None
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
                                            f"oracle restated in C), {reps} reps in {el:.1f} s"}
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
    for _ in range(Lyr):
        caches = [LayerCache("int8", H, D, max_context=8192) for _ in range(B)]
        for c in caches:
            c.query(prefill, prefill, 0, True)
        layers.append(caches)
    torch.cuda.synchronize()
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
        "join": {"ms": round(join_ms, 3), "host_ms": round(join_host_ms, 2), "copied_bytes": join_bytes,
                 "copy_launches": copy_launches, "copy_kernel_ms": round(copy_ms, 3)},
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
                                            f"D={D}] (oracle_append), {reps} reps in {el:.1f} s"}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the int8 KV decode path shards by "
                                   "sequence or head with no collective on the hot path (see DESIGN.md)",
                          "n_gpus": args.gpus}))
        return 2
    if args.sampler:
        return bench_sampler(args)
    if args.arena:
        return bench_arena(args)
    if args.kv != "int8":
        return bench_float(args)
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
    # committed into slot L of the arenas, in one launch.
    step = ppk.DecodeStep(q, kc, vc, ks, vs, kn.reshape(rows, 1, D), vn.reshape(rows, 1, D), past, H,
                          split_tokens=args.split, max_past=L, out=out)
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

    # Algorithmic bytes of one step: history K+V codes and scales of every
    # row, the bf16 query, the bf16 current K/V token (read once: quantised
    # into the arena and scored as the current token), the f32 output and the
    # appended codes + scales: sum_b L_b*H*(2D+8) + q + current k,v + out + append.
    hist_bytes = rows * L * (2 * D + 8)
    step_bytes = hist_bytes + rows * D * 2 + 2 * rows * D * 2 + rows * D * 4 + 2 * rows * (D + 4)
    kernel_bytes = step_bytes if step.ngroups == 1 else hist_bytes + rows * D * 2 + 2 * rows * (D + 4) + 2 * rows * D * 2
    achieved = kernel_bytes / (kernel_avg_ms * 1e-3) / 1e9
    step_gbps = step_bytes / (step_ms * 1e-3) / 1e9

    kname = "ppk_decode_d%d" % D
    traffic = None
    if os.path.exists(args.traffic):
        try:
            with open(args.traffic) as f:
                t = json.load(f)
            if t.get("split") == split and t.get("workload") == f"B{B}H{H}D{D}L{L}" and t.get("kernel") == kname:
                traffic = t.get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

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
        "config": {"workload": "BASELINE config 5: decode step = append of the current token + attention over "
                               "the int8 history (ppk_decode_step)",
                   "batch": B, "heads": H, "head_dim": D, "context": L, "capacity": cap, "kv": "int8 + f32 scales",
                   "query": "bf16", "tokens_per_wave": split, "blocks_per_row": step.ngroups,
                   "launches_per_step": 1 if step.ngroups == 1 else 2},
        "tokens_per_s": round(B / (step_ms * 1e-3), 1),
        "step_hbm_gbps": round(step_gbps, 1),
        "step_hbm_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": kernel_bytes,
                     "avg_launch_us": round(kernel_avg_ms * 1e3, 2), "launches": launches},
    }
    if not args.no_cpu_baseline:
        print("# bench: cpu baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(q, kc, vc, ks, vs, kn, vn, past, H, args)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
