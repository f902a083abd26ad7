"""Torch-tensor mirror of the reference's HIP CFG + Renyi sampler.

hip_sampling::sample(raw, uniforms, bounds, alpha, cfg, guidance, offset)
(app/src/inference/hip_sampling.rs:18-106): raw F32 [B*guidance, choices]
with interleaved (conditional, unconditional) rows when guidance = 2,
uniforms F32 [B, 1], bounds U32 [B, 2] of relative (start, count) legal
ranges. Returns absolute tokens, valid flags and effective supports, each
U32 [B, 1] (int32 storage viewed as uint32 where torch allows). Runs in the
gfx950 kernel behind libppk.so (ppk_renyi_sample); CPU tensors are refused
as the reference refuses them (hip_sampling.rs:94-96).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _abi
from ._abi import check, lib
from .int8_kv_ops import _require, _stream, context, current_stream_handle

_U32 = (torch.int32, torch.uint32)


def sample_args(raw, uniforms, bounds, alpha: float, cfg: float, guidance: int, offset: int,
                out: torch.Tensor | None = None) -> tuple[_abi.PpkRenyiSampleArgs, torch.Tensor]:
    """Validate like hip_sampling::validate (hip_sampling.rs:18-69) and build the ABI block."""
    _require(raw.dim() == 2, "HIP sampler needs 1/2 guidance rows and a nonempty head of at most 2048 choices")
    physical, choices = raw.shape
    _require(guidance in (1, 2) and physical > 0 and physical % guidance == 0 and 1 <= choices <= 2048,
             "HIP sampler needs 1/2 guidance rows and a nonempty head of at most 2048 choices")
    batch = physical // guidance
    _require(batch <= 2**31 - 1 and tuple(uniforms.shape) == (batch, 1) and tuple(bounds.shape) == (batch, 2),
             "HIP sampler logical row, uniform or bounds shape mismatch")
    _require(raw.dtype == torch.float32 and uniforms.dtype == torch.float32 and bounds.dtype in _U32,
             "HIP sampler expects FP32 logits/uniforms and U32 bounds")
    _require(raw.device == uniforms.device == bounds.device, "HIP sampler inputs must share the same device")
    _require(raw.is_contiguous() and uniforms.is_contiguous() and bounds.is_contiguous(),
             "HIP sampler inputs must be contiguous; nonzero view offsets are supported")
    _require(math.isfinite(alpha) and alpha > 1.0 and math.isfinite(cfg) and cfg >= 0.0
             and (guidance != 1 or cfg == 1.0), "invalid HIP sampler alpha/CFG/guidance combination")
    _require(0 <= offset and offset + choices - 1 <= 2**32 - 1, "HIP sampler token range overflow")
    if raw.device.type != "cuda":
        raise RuntimeError("HIP fused Renyi sampler requires ROCm device storage; no CPU/CUDA fallback")
    if out is None:
        out = torch.empty((3, batch), dtype=torch.int32, device=raw.device)
    _require(tuple(out.shape) == (3, batch) and out.dtype in _U32 and out.is_contiguous()
             and out.device == raw.device, "HIP sampler output must be U32 [3, batch]")
    a = _abi.PpkRenyiSampleArgs(struct_size=ctypes.sizeof(_abi.PpkRenyiSampleArgs), batch=batch, choices=choices,
                                guidance=guidance, alpha=alpha, cfg=cfg, token_offset=offset, reserved=0,
                                raw=raw.data_ptr(), uniforms=uniforms.data_ptr(), bounds=bounds.data_ptr(),
                                out=out.data_ptr())
    return a, out


def sample(raw, uniforms, bounds, alpha: float, cfg: float, guidance: int, offset: int
           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """hip_sampling::sample -> (tokens, valid, support), each [B, 1] (32-bit)."""
    a, out = sample_args(raw, uniforms, bounds, alpha, cfg, guidance, offset)
    check(lib().ppk_renyi_sample(context(raw.device), _stream(raw), ctypes.byref(a)), "ppk_renyi_sample")
    b = out.shape[1]
    return out[0].reshape(b, 1), out[1].reshape(b, 1), out[2].reshape(b, 1)


class RenyiSampler:
    """A prepared sampler call for fixed buffers (bench and serving loops, graph capture)."""

    def __init__(self, raw, uniforms, bounds, alpha: float, cfg: float, guidance: int, offset: int):
        self.args, self.out = sample_args(raw, uniforms, bounds, alpha, cfg, guidance, offset)
        self.ctx = context(raw.device)
        self._keep = (raw, uniforms, bounds)
        self._ref = ctypes.byref(self.args)
        self._fn = lib().ppk_renyi_sample
        self.device = raw.device

    def __call__(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        s = current_stream_handle(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(self._fn(self.ctx, s, self._ref), "ppk_renyi_sample")
        return self.out
