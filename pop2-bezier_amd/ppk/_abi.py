"""ctypes binding of include/ppk_int8_kv.h (libppk.so beside this file).

The structures below mirror the C layout field for field; tests/ compares
their sizes and offsets with the C compiler's.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libppk.so")
HSACO_PATH = os.path.join(HERE, "ppk_kernels.hsaco")

PPK_ABI_VERSION = 1
PPK_OK, PPK_PRECONDITION, PPK_INVALID_OUTPUT, PPK_EXECUTION_UNCERTAIN = 0, 1, 2, 3
PPK_F32, PPK_BF16, PPK_F16 = 0, 1, 2
PPK_FLAG_NONFINITE, PPK_FLAG_OVERFLOW, PPK_FLAG_STALE_LENGTHS = 1, 2, 4
PPK_ATTN_BF16_HISTORY = 1
PPK_ATTN_PLAN_PER_ROW, PPK_ATTN_PLAN_BALANCED = 2, 4
PPK_NOALLOC_SCRATCH_BYTES = 8 << 20
(PPK_KERNEL_QUANTIZE, PPK_KERNEL_APPEND, PPK_KERNEL_DEQUANTIZE, PPK_KERNEL_ATTENTION, PPK_KERNEL_ATTN_MERGE,
 PPK_KERNEL_FLOAT_ATTENTION, PPK_KERNEL_FLOAT_MERGE, PPK_KERNEL_RENYI_SAMPLE, PPK_KERNEL_COPY,
 PPK_KERNEL_COUNT) = range(10)

_u32, _u64, _ptr, _f32 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_float


class PpkQuantizeArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("src_dtype", _u32), ("src", _ptr), ("codes", _ptr), ("scales", _ptr),
                ("rows", _u64), ("head_dim", _u32), ("reserved", _u32), ("flags", _ptr)]


class PpkAppendArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("src_dtype", _u32), ("k_src", _ptr), ("v_src", _ptr), ("past", _ptr),
                ("k_codes", _ptr), ("v_codes", _ptr), ("k_scales", _ptr), ("v_scales", _ptr),
                ("batch", _u32), ("heads", _u32), ("tokens", _u32), ("head_dim", _u32), ("capacity", _u32),
                ("reserved", _u32), ("flags", _ptr)]


class PpkDequantizeArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("out_dtype", _u32), ("codes", _ptr), ("scales", _ptr), ("out", _ptr),
                ("rows", _u64), ("head_dim", _u32), ("round_bf16", _u32)]


class PpkAttentionArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("q_dtype", _u32), ("scratch_dtype", _u32), ("out_dtype", _u32),
                ("flags", _u32), ("rows", _u32), ("heads", _u32), ("capacity", _u32), ("head_dim", _u32),
                ("split_tokens", _u32), ("max_past", _u32), ("softmax_scale", _f32),
                ("q", _ptr), ("k_codes", _ptr), ("v_codes", _ptr), ("k_scales", _ptr), ("v_scales", _ptr),
                ("sk", _ptr), ("sv", _ptr), ("past", _ptr), ("out", _ptr), ("workspace", _ptr),
                ("workspace_bytes", _u64), ("past_host", _ptr)]


class PpkDecodeStepArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("new_dtype", _u32), ("k_new", _ptr), ("v_new", _ptr), ("flags", _ptr),
                ("attn", PpkAttentionArgs)]


class PpkFloatAttentionArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("kv_dtype", _u32), ("q_dtype", _u32), ("out_dtype", _u32),
                ("rows", _u32), ("heads", _u32), ("size", _u32), ("head_dim", _u32), ("split_tokens", _u32),
                ("max_length", _u32), ("softmax_scale", _f32), ("flags", _u32),
                ("q_row_stride", _u64), ("k_row_stride", _u64), ("v_row_stride", _u64),
                ("q", _ptr), ("k", _ptr), ("v", _ptr), ("lengths", _ptr), ("out", _ptr), ("workspace", _ptr),
                ("workspace_bytes", _u64), ("lengths_host", _ptr)]


class PpkFloatDecodeStepArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("new_dtype", _u32), ("k_new", _ptr), ("v_new", _ptr), ("flags", _ptr),
                ("attn", PpkFloatAttentionArgs)]


class PpkRenyiSampleArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("batch", _u32), ("choices", _u32), ("guidance", _u32), ("alpha", _f32),
                ("cfg", _f32), ("token_offset", _u32), ("reserved", _u32), ("raw", _ptr), ("uniforms", _ptr),
                ("bounds", _ptr), ("out", _ptr)]


PPK_KV_INT8, PPK_KV_BF16, PPK_KV_F16, PPK_KV_F32 = 0, 1, 2, 3


class PpkKvConfig(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("kind", _u32), ("heads", _u32), ("head_dim", _u32), ("max_context", _u32),
                ("min_capacity", _u32)]


class PpkKvView(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("kind", _u32), ("rows", _u32), ("capacity", _u32), ("head_dim", _u32),
                ("length", _u32), ("batch", _u32), ("reserved", _u32), ("k", _ptr), ("v", _ptr),
                ("k_scales", _ptr), ("v_scales", _ptr), ("past", _ptr), ("lengths", _ptr)]


class PpkKvInfo(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("length", _u32), ("capacity", _u32), ("grouped", _u32), ("slot", _u32),
                ("shared", _u32), ("reserved_bytes", _u64), ("storage_id", _u64), ("arena_id", _u64),
                ("arena_copied_rows", _u64), ("arena_offset_uploads", _u64), ("scale_bytes", _u64)]


class PpkKvWrite(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("src_dtype", _u32), ("tokens", _u32), ("commit", _u32), ("k", _ptr),
                ("v", _ptr)]


class PpkInt8KvStatus(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("requested", _u32), ("available", _u32), ("ready", _u32), ("enabled", _u32),
                ("packed_bytes_per_token_head", _u32), ("scale_bytes_per_token_head", _u32), ("reserved", _u32),
                ("format", ctypes.c_char * 64), ("reason", ctypes.c_char * 256)]


class PpkAttentionPlanInfo(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("kind", _u32), ("split_tokens", _u32), ("nsplits", _u32),
                ("waves_per_block", _u32), ("blocks", _u32), ("launches", _u32), ("reserved", _u32),
                ("workspace_bytes", _u64)]


# Every function the header declares: name -> (restype, argtypes).
FUNCTIONS = {
    "ppk_abi_version": (_u32, []),
    "ppk_last_error": (ctypes.c_char_p, []),
    "ppk_context_create": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_char_p, ctypes.POINTER(_ptr)]),
    "ppk_context_release": (ctypes.c_int32, [_ptr]),
    "ppk_context_trim": (ctypes.c_int32, [_ptr, ctypes.POINTER(_u64)]),
    "ppk_quantize": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkQuantizeArgs)]),
    "ppk_quantize_append": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkAppendArgs)]),
    "ppk_dequantize": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkDequantizeArgs)]),
    "ppk_attention_workspace_bytes": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkAttentionArgs),
                                                       ctypes.POINTER(_u64)]),
    "ppk_attention_plan": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkAttentionArgs), ctypes.POINTER(_u32),
                                            ctypes.POINTER(_u32), ctypes.POINTER(_u64)]),
    "ppk_attention_plan_info": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkAttentionArgs),
                                                 ctypes.POINTER(PpkAttentionPlanInfo)]),
    "ppk_decode_attention": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkAttentionArgs)]),
    "ppk_decode_step": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkDecodeStepArgs)]),
    "ppk_decode_step_noalloc": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkDecodeStepArgs)]),
    "ppk_float_attention_plan": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkFloatAttentionArgs), ctypes.POINTER(_u32),
                                                  ctypes.POINTER(_u32), ctypes.POINTER(_u64)]),
    "ppk_float_attention_plan_info": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkFloatAttentionArgs),
                                                       ctypes.POINTER(PpkAttentionPlanInfo)]),
    "ppk_float_decode_attention": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkFloatAttentionArgs)]),
    "ppk_float_decode_step": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkFloatDecodeStepArgs)]),
    "ppk_float_attention_prepare": (ctypes.c_int32, [_ptr]),
    "ppk_renyi_sample": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(PpkRenyiSampleArgs)]),
    "ppk_kv_cache_create": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkKvConfig), ctypes.POINTER(_ptr)]),
    "ppk_kv_cache_clone": (ctypes.c_int32, [_ptr, ctypes.POINTER(_ptr)]),
    "ppk_kv_cache_release": (ctypes.c_int32, [_ptr]),
    "ppk_kv_cache_info": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkKvInfo)]),
    "ppk_kv_cache_truncate": (ctypes.c_int32, [_ptr, _u32]),
    "ppk_kv_cache_adopt": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkKvConfig), _ptr, _ptr, _u32, _u32,
                                            ctypes.POINTER(_ptr)]),
    "ppk_kv_cache_advance": (ctypes.c_int32, [_ptr, _u32, _u32]),
    "ppk_kv_cache_view": (ctypes.c_int32, [_ptr, ctypes.POINTER(PpkKvView)]),
    "ppk_kv_query": (ctypes.c_int32, [_ptr, _ptr, _ptr, _u32, ctypes.POINTER(PpkKvWrite), ctypes.POINTER(PpkKvView)]),
    "ppk_write_plan_create": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(_u32), _u32, _u32, _u32,
                                               ctypes.POINTER(_ptr)]),
    "ppk_write_plan_release": (ctypes.c_int32, [_ptr]),
    "ppk_kv_query_batch": (ctypes.c_int32, [_ptr, _ptr, ctypes.POINTER(_ptr), _u32, ctypes.POINTER(_u32),
                                            ctypes.POINTER(PpkKvWrite), _ptr, ctypes.POINTER(PpkKvView)]),
    "ppk_prepare": (ctypes.c_int32, [_ptr]),
    "ppk_prepare_int8_kv": (ctypes.c_int32, [_ptr, _u32, _u32, ctypes.POINTER(PpkInt8KvStatus)]),
    "ppk_context_set_profiling": (ctypes.c_int32, [_ptr, ctypes.c_int32]),
    "ppk_context_set_wave_clock": (ctypes.c_int32, [_ptr, _ptr, _u64]),
    "ppk_context_kernel_stats": (ctypes.c_int32, [_ptr, _u32, ctypes.POINTER(_u64), ctypes.POINTER(ctypes.c_double),
                                                  _u32]),
}


class PpkError(RuntimeError):
    status = -1


class PpkPreconditionError(PpkError):
    """Status 1: invalid arguments or preparation failure; nothing was enqueued."""
    status = PPK_PRECONDITION


class PpkInvalidOutputError(PpkError):
    """Status 2: a numeric self-check failed."""
    status = PPK_INVALID_OUTPUT


class PpkExecutionUncertainError(PpkError):
    """Status 3: a launch was attempted and failed; never replay the work."""
    status = PPK_EXECUTION_UNCERTAIN


_ERRORS = {1: PpkPreconditionError, 2: PpkInvalidOutputError, 3: PpkExecutionUncertainError}
_lib = None


def lib() -> ctypes.CDLL:
    """Load libppk.so. Raises if it was not built: there is no fallback path."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libppk.so missing at {LIB_PATH}: run python pop2-bezier_amd/build.py "
                               "(the int8 KV path has no CPU or eager fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in FUNCTIONS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.ppk_abi_version() != PPK_ABI_VERSION:
            raise RuntimeError(f"libppk ABI {L.ppk_abi_version()} != expected {PPK_ABI_VERSION}")
        _lib = L
    return _lib


def last_error() -> str:
    """ppk_last_error() of the calling thread."""
    return (lib().ppk_last_error() or b"").decode("utf-8", "replace")


def check(status: int, what: str) -> None:
    if status != PPK_OK:
        msg = (lib().ppk_last_error() or b"").decode("utf-8", "replace")
        raise _ERRORS.get(status, PpkError)(f"{what} failed with status {status}: {msg}")


def plan_flags(plan: str) -> int:
    """PPK_ATTN_PLAN_* bits of a plan choice: "auto" (the library decides from the host lengths), "per-row" or
    "balanced"."""
    flags = {"auto": 0, "per-row": PPK_ATTN_PLAN_PER_ROW, "balanced": PPK_ATTN_PLAN_BALANCED}.get(plan)
    if flags is None:
        raise ValueError(f"plan must be 'auto', 'per-row' or 'balanced', got {plan!r}")
    return flags
