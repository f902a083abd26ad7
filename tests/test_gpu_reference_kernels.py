"""The float-KV decode attention against the reference's own kernels
(pp_attention_f32/bf16 + pp_attention_merge, app/src/model/decode_attention.hip),
built unchanged from their source into oracle/_ref and launched with the
reference's geometry, on the same device buffers. Bar: the reference's own
acceptance tolerance for this kernel pair, 1e-4 absolute
(hip_attention.rs:36-41); both also sit within it of the f64 oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import ppk
import refkernels
from helpers import SEED

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("split", [0, 128])
@pytest.mark.parametrize("lengths", [None, [1, 300, 1024, 777]])
def test_float_attention_matches_reference_kernel(device, kv, split, lengths):
    gen = torch.Generator(device=device).manual_seed(SEED)
    B, H, size = 4, 16, 1024
    rows = B * H
    store_k = torch.randn((rows, 1040, 64), generator=gen, device=device).to(kv)
    store_v = torch.randn((rows, 1040, 64), generator=gen, device=device).to(kv)
    k, v = store_k[:, :size], store_v[:, :size]  # the graph-decode view of a longer store
    q = torch.randn((rows, 1, 64), generator=gen, device=device)
    lt = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    ours = ppk.fused_attention.decode_attention(q, k, v, lt, H, split).reshape(rows, 64)
    ref = refkernels.decode_attention(q, k, v, lt, H, split)
    torch.cuda.synchronize()
    ours, ref = ours.cpu().numpy(), ref.cpu().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.max(np.abs(ours[fin] - ref[fin])) <= 1e-4
    # Both against the f64 oracle.
    kh = k.float().cpu().numpy() if kv == torch.float32 else k.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    vh = v.float().cpu().numpy() if kv == torch.float32 else v.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    truth = oracle.attention_float(q.cpu().numpy(), kh, vh, None if lengths is None else np.array(lengths, np.uint32), H)
    assert np.max(np.abs(ours[fin] - truth[fin])) <= 1e-4
    assert np.max(np.abs(ref[fin] - truth[fin])) <= 1e-4


def test_invalid_lengths_nan_like_reference_kernel(device):
    gen = torch.Generator(device=device).manual_seed(SEED + 1)
    rows, size = 8, 200
    k = torch.randn((rows, size, 64), generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn((rows, size, 64), generator=gen, device=device, dtype=torch.bfloat16)
    q = torch.randn((rows, 1, 64), generator=gen, device=device)
    lt = torch.tensor([0, 200, 201, 5], dtype=torch.int32, device=device)
    for split in (0, 64):
        ours = ppk.fused_attention.decode_attention(q, k, v, lt, 2, split).reshape(rows, 64).cpu().numpy()
        ref = refkernels.decode_attention(q, k, v, lt, 2, split).cpu().numpy()
        assert np.array_equal(np.isnan(ours), np.isnan(ref))
        fin = ~np.isnan(ref)
        assert np.max(np.abs(ours[fin] - ref[fin])) <= 1e-4
