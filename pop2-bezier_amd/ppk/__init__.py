"""ppk: MI355X-native int8 KV-cache quantize/append and split-K decode attention
(plus the same attention over float bf16/f32 KV, ppk.fused_attention).

The product path is libppk.so (C-ABI, include/ppk_int8_kv.h) plus the gfx950
code object ppk_kernels.hsaco; this package binds them for torch callers.
"""
from . import fused_attention, kv_arena, sampling
from ._abi import (PPK_ABI_VERSION, PPK_ATTN_BF16_HISTORY, PPK_ATTN_PLAN_BALANCED, PPK_ATTN_PLAN_PER_ROW,
                   PPK_FLAG_NONFINITE, PPK_FLAG_OVERFLOW, PPK_FLAG_STALE_LENGTHS,
                   PPK_KERNEL_APPEND, PPK_KERNEL_ATTN_MERGE, PPK_KERNEL_ATTENTION, PPK_KERNEL_COPY,
                   PPK_KERNEL_DEQUANTIZE, PPK_KERNEL_FLOAT_ATTENTION, PPK_KERNEL_FLOAT_MERGE, PPK_KERNEL_QUANTIZE,
                   PPK_KERNEL_RENYI_SAMPLE, PpkError,
                   PpkExecutionUncertainError, PpkInvalidOutputError, PpkPreconditionError)
from .fused_attention import FloatDecodeAttention, FloatDecodeStep
from .kv_arena import LayerCache, WritePlan
from .sampling import RenyiSampler
from .int8_kv_ops import (AppendKV, DecodeAttention, DecodeStep, append, attention, context, decode_step,
                          dequantize, kernel_stats, prepare, prepare_int8_kv, quantize, set_profiling)

__all__ = [
    "PPK_ABI_VERSION", "PPK_ATTN_BF16_HISTORY", "PPK_ATTN_PLAN_BALANCED", "PPK_ATTN_PLAN_PER_ROW",
    "PPK_FLAG_NONFINITE", "PPK_FLAG_OVERFLOW", "PPK_FLAG_STALE_LENGTHS",
    "PPK_KERNEL_APPEND", "PPK_KERNEL_ATTN_MERGE", "PPK_KERNEL_ATTENTION", "PPK_KERNEL_COPY", "PPK_KERNEL_DEQUANTIZE",
    "PPK_KERNEL_FLOAT_ATTENTION", "PPK_KERNEL_FLOAT_MERGE", "PPK_KERNEL_QUANTIZE", "PPK_KERNEL_RENYI_SAMPLE",
    "PpkError", "PpkExecutionUncertainError", "PpkInvalidOutputError", "PpkPreconditionError",
    "AppendKV", "DecodeAttention", "DecodeStep", "FloatDecodeAttention", "FloatDecodeStep", "LayerCache",
    "RenyiSampler", "WritePlan",
    "fused_attention", "kv_arena", "sampling",
    "append", "attention", "context", "decode_step", "dequantize", "kernel_stats", "prepare", "prepare_int8_kv",
    "quantize",
    "set_profiling",
]
