"""ctypes access to oracle/_ref/libppk_ref.so: the reference's own HIP kernels
(float-KV decode attention, CFG + Renyi sampler) built unchanged from the
reference sources by oracle/build_ref.py. A checker for tests only."""
from __future__ import annotations

import ctypes
import os

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref")
_lib = None


def available() -> bool:
    return os.path.exists(os.path.join(REF, "libppk_ref.so"))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = os.path.join(REF, "libppk_ref.so")
        if not os.path.exists(path):
            pytest.skip("oracle/_ref not built (python oracle/build_ref.py needs the reference tree)")
        L = ctypes.CDLL(path)
        P, U32, U64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
        L.ref_last_error.restype = ctypes.c_char_p
        L.ref_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
        L.ref_decode_attention.argtypes = [P, ctypes.c_int, P, P, P, P, P, P, U32, U32, U32, U32, U64, U64, U64]
        L.ref_renyi_sample.argtypes = [P, P, P, P, P, U32, U32, U32, ctypes.c_float, ctypes.c_float, U32]
        if L.ref_load(os.path.join(REF, "decode_attention.hsaco").encode(),
                      os.path.join(REF, "renyi_sample.hsaco").encode()) != 0:
            raise RuntimeError(L.ref_last_error().decode())
        _lib = L
    return _lib


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def decode_attention(q, k, v, lengths, heads: int, split_tokens: int = 0) -> torch.Tensor:
    """pp_attention_{f32,bf16} (+ pp_attention_merge) at the reference's geometry; F32 [rows, 64]."""
    rows, length = k.shape[0], k.shape[1]
    split = min(max(split_tokens, 32), 1024) if split_tokens else length
    splits = -(-length // split)
    out = torch.empty((rows, 64), dtype=torch.float32, device=q.device)
    partial = torch.empty(max(rows * splits * 66, 1), dtype=torch.float32, device=q.device)
    rc = lib().ref_decode_attention(_stream(q), int(k.dtype == torch.bfloat16), q.data_ptr(), k.data_ptr(),
                                    v.data_ptr(), lengths.data_ptr() if lengths is not None else None,
                                    out.data_ptr(), partial.data_ptr(), heads, rows, length, split_tokens,
                                    q.stride(0), k.stride(0), v.stride(0))
    if rc != 0:
        raise RuntimeError(lib().ref_last_error().decode())
    return out


def renyi_sample(raw, uniforms, bounds, alpha: float, cfg: float, guidance: int, offset: int) -> torch.Tensor:
    """pp_hip_renyi_sample at the reference's geometry; U32 [3, batch] (int32 storage)."""
    batch = raw.shape[0] // guidance
    out = torch.full((3, batch), -1, dtype=torch.int32, device=raw.device)
    rc = lib().ref_renyi_sample(_stream(raw), raw.data_ptr(), uniforms.data_ptr(), bounds.data_ptr(),
                                out.data_ptr(), batch, raw.shape[1], guidance, alpha, cfg, offset)
    if rc != 0:
        raise RuntimeError(lib().ref_last_error().decode())
    return out
