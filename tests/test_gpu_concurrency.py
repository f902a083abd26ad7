"""One context used from two host threads at once, each on its own stream (GPU).

The C-ABI promises calls on distinct streams may overlap (one context per
device, shared write-plan pool under a lock, thread-local error text, as the
reference's FFI keeps its last error per thread, painter_ffi.cpp:12,18-19).
Each thread's results must equal what the same calls produce alone, bit for
bit: the kernels are deterministic for fixed inputs and plans.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

import ppk
from ppk.kv_arena import LayerCache, WritePlan, read
from helpers import SEED

pytestmark = pytest.mark.gpu


def _attention_inputs(seed: int, device):
    g = torch.Generator(device=device).manual_seed(seed)
    rows, cap, d, heads = 64, 1500, 128, 16
    hist = torch.randn((rows, cap, d), generator=g, device=device)
    vh = torch.randn((rows, cap, d), generator=g, device=device)
    kc, ks = ppk.quantize(hist)
    vc, vs = ppk.quantize(vh)
    q = torch.randn((rows, 1, d), generator=g, device=device).to(torch.bfloat16)
    sk = torch.randn((rows, 1, d), generator=g, device=device).to(torch.bfloat16)
    sv = torch.randn((rows, 1, d), generator=g, device=device).to(torch.bfloat16)
    past = torch.tensor([1400, 17, 999, 1499], dtype=torch.int32, device=device)
    return (q, kc, vc, ks, vs, sk, sv, past, heads), hist


def _work(inputs, hist, iters: int):
    """Attention (split-K + merge and one-launch plans) and a quantize, `iters` times; last results."""
    out = None
    for i in range(iters):
        out = ppk.attention(*inputs, split_tokens=(0, 256)[i % 2])
        codes, scales = ppk.quantize(hist[: 40 + i])
    torch.cuda.current_stream().synchronize()
    return out, codes, scales


def _run_threads(fns):
    results, errors = [None] * len(fns), []

    def body(i, fn):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                results[i] = fn()
        except BaseException as e:  # surfaced in the main thread
            errors.append(e)

    threads = [threading.Thread(target=body, args=(i, fn)) for i, fn in enumerate(fns)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    if errors:
        raise errors[0]
    return results


def test_two_threads_on_two_streams_reproduce_their_lone_results(device):
    inputs = [_attention_inputs(SEED + 91 + i, device) for i in range(2)]
    alone = [_work(inp, h, 6) for inp, h in inputs]
    together = _run_threads([lambda inp=inp, h=h: _work(inp, h, 6) for inp, h in inputs])
    for (a_out, a_c, a_s), (t_out, t_c, t_s) in zip(alone, together):
        assert torch.equal(a_out.view(torch.int32), t_out.view(torch.int32))
        assert torch.equal(a_c, t_c) and torch.equal(a_s.view(torch.int32), t_s.view(torch.int32))


def _arena_rounds(seed: int, device, rounds: int = 12):
    """Four int8 caches: prefill, then decode rounds with one shared write plan each; final contents."""
    g = torch.Generator(device=device).manual_seed(seed)
    heads, d = 4, 64
    caches = [LayerCache("int8", heads, d, device=device) for _ in range(4)]
    for i, c in enumerate(caches):
        p = torch.randn((heads, 20 + 7 * i, d), generator=g, device=device)
        c.query(p, p, 0, True)
    for _ in range(rounds):
        past = [len(c) for c in caches]
        plan = WritePlan(past, heads, d, device=device)
        cur = torch.randn((4, heads, 1, d), generator=g, device=device)
        LayerCache.query_batch(caches, cur, cur, past, True, plan)
        del plan
    out = [(read(c.view(), "k"), read(c.view(), "k_scales")) for c in caches]
    torch.cuda.current_stream().synchronize()  # the copies are read from another thread
    return out


def test_arena_rounds_with_pooled_write_plans_from_two_threads(device):
    alone = [_arena_rounds(SEED + 95 + i, device) for i in range(2)]
    together = _run_threads([lambda i=i: _arena_rounds(SEED + 95 + i, device) for i in range(2)])
    for a, t in zip(alone, together):
        for (ak, asc), (tk, tsc) in zip(a, t):
            assert torch.equal(ak, tk) and torch.equal(asc.view(torch.int32), tsc.view(torch.int32))
    assert np.isfinite(together[0][0][1].cpu().numpy()).all()
