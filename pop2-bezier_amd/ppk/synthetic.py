"""Seeded synthetic KV workloads on the GPU (benchmark and large parity tests).

History values follow the heavy-tail rule of the benchmark configs: N(0,1),
except round(0.02*H*D) (head, channel) pairs per K and per V tensor that hold
10 * Student-t(3) for every token. Values are drawn chunk by chunk from
torch generators seeded by (seed, tensor, chunk), so a test can regenerate the
exact source rows of any chunk, and are quantised into the arenas by the
library's own quantize kernel.
"""
from __future__ import annotations

import torch

from . import int8_kv_ops


def chunk_seed(seed: int, tensor: int, chunk: int) -> int:
    return (seed * 1_000_003 + tensor * 7_919 + chunk) % (2**63 - 1)


def heavy_pairs(seed: int, tensor: int, heads: int, d: int, frac: float = 0.02) -> torch.Tensor:
    """Flat (h*d + c) indices of the heavy-tailed pairs of one tensor (CPU, int64)."""
    g = torch.Generator().manual_seed(chunk_seed(seed, tensor, 10**6))
    n = int(round(frac * heads * d))
    return torch.randperm(heads * d, generator=g)[:n].sort().values


def history_chunk(seed: int, tensor: int, chunk: int, rows: int, heads: int, row0: int, tokens: int, d: int,
                  device: torch.device, dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Source values [rows, tokens, d] for head rows row0 .. row0+rows-1 (row = b*heads + h)."""
    g = torch.Generator(device=device).manual_seed(chunk_seed(seed, tensor, chunk))
    x = torch.randn((rows, tokens, d), generator=g, device=device, dtype=torch.float32)
    pairs = heavy_pairs(seed, tensor, heads, d).to(device)
    hh, cc = pairs // d, pairs % d
    for r in range(rows):
        h = (row0 + r) % heads
        sel = cc[hh == h]
        if sel.numel() == 0:
            continue
        z = torch.randn((tokens, sel.numel()), generator=g, device=device)
        chi = torch.randn((3, tokens, sel.numel()), generator=g, device=device).square().sum(0)
        x[r][:, sel] = 10.0 * z / torch.sqrt(chi / 3.0)
    return x.to(dtype)


def fill_history(k_codes: torch.Tensor, v_codes: torch.Tensor, k_scales: torch.Tensor, v_scales: torch.Tensor,
                 tokens: int, heads: int, seed: int, chunk_rows: int = 16,
                 dtype: torch.dtype = torch.float16) -> None:
    """Quantise seeded heavy-tailed history into slots [0, tokens) of every row of the arenas."""
    rows, cap, d = k_codes.shape
    assert tokens <= cap
    for tensor, (codes, scales) in enumerate(((k_codes, k_scales), (v_codes, v_scales))):
        for chunk, row0 in enumerate(range(0, rows, chunk_rows)):
            n = min(chunk_rows, rows - row0)
            x = history_chunk(seed, tensor, chunk, n, heads, row0, tokens, d, codes.device, dtype)
            c, s = int8_kv_ops.quantize(x)
            codes[row0:row0 + n, :tokens].copy_(c)
            scales[row0:row0 + n, :tokens].copy_(s)
            del x, c, s
