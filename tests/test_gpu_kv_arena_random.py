"""Seeded random sequences of KV arena operations against a host model (GPU).

The model is the reference's own test oracle for LayerCache (cache.rs:551-556:
the committed history is the concatenation of what was committed): each
cache is a list of committed token rows. Operations follow the LayerCache
API (cache.rs:194-531): commit and scratch writes, snapshots (clone),
metadata truncation, one-token batch writes over a subset of caches (with
and without a shared write plan), release. After every operation each live
cache's committed history must equal the model bit for bit (f32 storage
exactly, int8 storage as the oracle's quantisation of the committed rows),
which exercises copy-on-write, growth, in-place writes, batch-arena reuse
and orphan slots, and reuse of released storage.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from ppk.kv_arena import LayerCache, WritePlan

pytestmark = pytest.mark.gpu
HEADS, D = 2, 64


def _tokens(rng, n, device):
    return torch.from_numpy(rng.standard_normal((HEADS, n, D)).astype(np.float32)).to(device)


def _check(live, kind):
    for c, hist in live:
        key = c.key()
        if not hist:
            assert key is None or key.shape[1] == 0
            continue
        want = torch.cat(hist, 1)
        if kind == "int8":  # codes of the committed rows: the oracle's quantisation of each (head, token) row
            codes, _, _ = oracle.quantize(want.cpu().numpy())
            want = torch.from_numpy(codes).to(key.device)
        assert key is not None and torch.equal(key, want)


@pytest.mark.parametrize("kind", ["f32", "int8"])
@pytest.mark.parametrize("seed", range(8))
def test_random_arena_operation_sequences_match_the_cat_model(device, seed, kind):
    rng = np.random.default_rng(9000 + seed)
    make = lambda: LayerCache(torch.float32 if kind == "f32" else "int8", HEADS, D, max_context=512,  # noqa: E731
                              min_capacity=8, device=device)
    live: list[tuple[LayerCache, list[torch.Tensor]]] = [(make(), []) for _ in range(4)]
    for step in range(150):
        op = rng.choice(["commit", "scratch", "clone", "truncate", "batch", "batch_plan", "release", "new"],
                        p=[0.22, 0.08, 0.12, 0.1, 0.2, 0.13, 0.07, 0.08])
        length = lambda h: sum(t.shape[1] for t in h)  # noqa: E731
        if op in ("commit", "scratch") and live:
            i = int(rng.integers(len(live)))
            c, hist = live[i]
            n = int(rng.integers(1, 20)) if op == "commit" else 1
            if length(hist) + n > 512:
                continue
            x = _tokens(rng, n, device)
            c.query(x, x, length(hist), op == "commit")
            if op == "commit":
                live[i] = (c, hist + [x])
        elif op == "clone" and live:
            c, hist = live[int(rng.integers(len(live)))]
            live.append((c.clone(), list(hist)))
        elif op == "truncate" and live:
            i = int(rng.integers(len(live)))
            c, hist = live[i]
            n = length(hist)
            if n == 0:
                continue
            new_len = int(rng.integers(0, n + 1))
            c.truncate_committed(new_len)
            cut = torch.cat(hist, 1)[:, :new_len] if hist else None
            live[i] = (c, [cut] if new_len else [])
        elif op in ("batch", "batch_plan") and len(live) >= 2:
            k = int(rng.integers(2, min(len(live), 5) + 1))
            idx = [int(j) for j in rng.choice(len(live), size=k, replace=False)]
            caches = [live[j][0] for j in idx]
            past = [length(live[j][1]) for j in idx]
            if max(past) + 1 > 512:
                continue
            cur = torch.from_numpy(rng.standard_normal((k, HEADS, 1, D)).astype(np.float32)).to(device)
            plan = WritePlan(past, HEADS, D, device=device) if op == "batch_plan" else None
            LayerCache.query_batch(caches, cur, cur, past, True, plan)
            for b, j in enumerate(idx):
                c, hist = live[j]
                live[j] = (c, hist + [cur[b]])
        elif op == "release" and len(live) > 2:
            live.pop(int(rng.integers(len(live))))
        elif op == "new":
            live.append((make(), []))
        torch.cuda.synchronize()
        try:
            _check(live, kind)
        except AssertionError:
            raise AssertionError(f"{kind} seed {seed}: history differs after step {step} ({op})")
