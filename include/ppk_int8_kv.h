/*
 * ppk_int8_kv.h -- C-ABI of the MI355X (gfx950) int8 KV-cache decode path.
 *
 * Two hand-written CDNA4 kernels sit behind this boundary:
 *   1. quantize(-and-append): per (head, token) row of D channels,
 *        s    = max(absmax / 127, 1e-12)            (IEEE fp32 division)
 *        code = clamp(round_half_even(x / s), -127, 127) stored as a byte
 *      written either densely or into a KV arena at slot past[b] + j;
 *   2. split-K single-query decode attention over the int8 arena
 *      (partial kernel + cross-split merge kernel).
 * The same attention kernel design also serves the float (bf16/f32) KV
 * decode path (ppk_float_decode_attention); the decode loop's next step, the
 * CFG + Renyi sampler, is ppk_renyi_sample.
 *
 * Every device buffer is caller-owned; the library never frees or allocates
 * caller memory. All work is stream-ordered on the hipStream_t passed in
 * (as void*), with no implicit synchronisation. Code objects for gfx950 are
 * built ahead of time and loaded with hipModuleLoad by ppk_context_create.
 *
 * Status codes follow the reference C-ABI (app/native/aten_hip/cpp/painter_ffi.h:20-25):
 *   0 success; 1 precondition/preparation failure, nothing was enqueued;
 *   2 invalid output (self-check mismatch); 3 execution uncertain, never replay.
 * Error text is thread-local (app/native/aten_hip/cpp/painter_ffi.cpp:12,18-19).
 *
 * Reference semantics: app/src/model/int8_kv_ops.rs:5-103 and
 * app/src/model/int8_kv.cu:1-59 (head_dim 64, capacity <= 1024 there; this
 * library extends them to head_dim 64/128/256 and any capacity < 2^31 / D).
 */
#ifndef PPK_INT8_KV_H
#define PPK_INT8_KV_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define PPK_API __attribute__((visibility("default")))
#else
#define PPK_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define PPK_ABI_VERSION 1u

enum {
  PPK_OK = 0,
  PPK_PRECONDITION = 1,
  PPK_INVALID_OUTPUT = 2,
  PPK_EXECUTION_UNCERTAIN = 3
};

/* Element types of floating tensors crossing the boundary. */
enum { PPK_F32 = 0, PPK_BF16 = 1, PPK_F16 = 2 };

/* Device-side status bits written by the quantize kernels when a flag word is supplied. */
enum {
  PPK_FLAG_NONFINITE = 1u, /* an input row held NaN or +-Inf (reference CPU path rejects these, int8_kv_ops.rs:16) */
  PPK_FLAG_OVERFLOW = 2u,  /* past[b] + tokens > capacity: that row was not written */
  PPK_FLAG_STALE_LENGTHS = 4u /* decode step: a device length differed from the host copy (past_host / lengths_host) and its rows gave NaN */
};

/* Attention flags. */
enum {
  /* Dequantise history as bf16(code * scale) before the dot products, exactly as
     pp_i8_load does (app/src/model/int8_kv.cu:23-27). Default (0) dequantises in
     fp32 with the per-token scale folded into the score and the probability. */
  PPK_ATTN_BF16_HISTORY = 1u,
  /* Launch plan (no counterpart in the reference; the result does not depend
     on it beyond fp32 summation order). With host lengths (past_host /
     lengths_host) the library chooses between its per-row plan and the
     balanced plan for ragged batches, and sizes its per-row plan for the
     longest live host length; these bits fix the choice. PER_ROW ignores
     the host lengths for planning: it is the plan of the same call without
     them, so its result is bit for bit that call's. BALANCED needs the host
     lengths, split_tokens == 0, at most 64
     sequences and rows at most 4 per CU; otherwise the call fails with status
     1 and nothing enqueued. Setting both is an error. */
  PPK_ATTN_PLAN_PER_ROW = 2u,
  PPK_ATTN_PLAN_BALANCED = 4u
};

typedef struct ppk_context ppk_context;

/* ABI version, checked by loaders like pp_aten_abi_version
   (painter_ffi.h:58, app/src/inference/aten_ffi.rs:277-280). */
PPK_API uint32_t ppk_abi_version(void);

/* Last error of the calling thread, UTF-8, at most 6000 bytes (pp_aten_last_error). */
PPK_API const char* ppk_last_error(void);

/* Load the gfx950 code object (code_object_path may be NULL: the .hsaco beside
   this library) on HIP device `device` and resolve every kernel before any
   launch. Replaces the runtime JIT + module cache of int8_kv_ops.rs:111-119 and
   app/src/model/hip_kernel.rs:99-149 with an ahead-of-time code object. */
PPK_API int32_t ppk_context_create(int32_t device, const char* code_object_path, ppk_context** out);
PPK_API int32_t ppk_context_release(ppk_context* ctx);
/* No counterpart in the reference: returns to the device the storage of
   released KV caches that the context keeps for reuse (see the KV arena
   notes below) and the unused memory of its pool, once the work that last
   used it has finished. For long-lived callers that need that memory
   elsewhere. *released_bytes (may be NULL) receives the bytes of kept
   storage freed. Caches and plans stay valid. */
PPK_API int32_t ppk_context_trim(ppk_context* ctx, uint64_t* released_bytes);

/* Dense quantize: src[rows, tokens, D] -> codes[rows, tokens, D], scales[rows, tokens].
   Replaces int8_kv_ops::quantize (app/src/model/int8_kv_ops.rs:11-29), i.e. the
   cuda::Scale + cuda::Pack custom ops (int8_kv_ops.rs:120-142, int8_kv.cu:8-18). */
typedef struct PpkQuantizeArgs {
  uint32_t struct_size;
  uint32_t src_dtype;      /* PPK_F32 / PPK_BF16 / PPK_F16 */
  const void* src;         /* [rows * tokens, D] contiguous */
  uint8_t* codes;          /* [rows * tokens, D] two's-complement int8 */
  float* scales;           /* [rows * tokens] */
  uint64_t rows;           /* number of (head, token) rows: heads * tokens */
  uint32_t head_dim;       /* D: 64, 128 or 256 */
  uint32_t reserved;
  uint32_t* flags;         /* optional device word, PPK_FLAG_* bits OR-ed in */
} PpkQuantizeArgs;
PPK_API int32_t ppk_quantize(ppk_context* ctx, void* stream, const PpkQuantizeArgs* args);

/* Fused quantize + append of new K and V tokens into the int8 arenas at slot
   past[b] + j (the commit path of Int8LayerCache::query/query_batch,
   app/src/model/int8_cache.rs:293-359, writing through LayerCache slot
   placement, app/src/model/cache.rs:122-154,301-478; AMD variant kv_i8_commit,
   app/native/aten_hip/cpp/kv_int8.cpp:47-54, whose x(1/127) scale this does
   NOT follow). Uncommitted (partial) queries need no call: their placeholder
   slot is never read (int8_cache.rs:304-310). */
typedef struct PpkAppendArgs {
  uint32_t struct_size;
  uint32_t src_dtype;      /* PPK_F32 / PPK_BF16 / PPK_F16 */
  const void* k_src;       /* [batch, heads, tokens, D] contiguous */
  const void* v_src;       /* [batch, heads, tokens, D] contiguous */
  const uint32_t* past;    /* device U32[batch]: committed length of each sequence */
  uint8_t* k_codes;        /* arena [batch*heads, capacity, D] */
  uint8_t* v_codes;        /* arena [batch*heads, capacity, D] */
  float* k_scales;         /* arena [batch*heads, capacity] */
  float* v_scales;         /* arena [batch*heads, capacity] */
  uint32_t batch, heads, tokens, head_dim, capacity;
  uint32_t reserved;
  uint32_t* flags;         /* optional device word, PPK_FLAG_* bits OR-ed in */
} PpkAppendArgs;
PPK_API int32_t ppk_quantize_append(ppk_context* ctx, void* stream, const PpkAppendArgs* args);

/* Dequantize codes[rows, tokens, D] * scales[rows, tokens] to out_dtype;
   round_bf16 != 0 rounds the fp32 product to bf16 first (the reference's
   dequantize(.., BF16)). Replaces int8_kv_ops::dequantize
   (int8_kv_ops.rs:30-40, pp_i8_unpack int8_kv.cu:19-22). */
typedef struct PpkDequantizeArgs {
  uint32_t struct_size;
  uint32_t out_dtype;
  const uint8_t* codes;
  const float* scales;
  void* out;
  uint64_t rows;           /* heads * tokens */
  uint32_t head_dim;
  uint32_t round_bf16;
} PpkDequantizeArgs;
PPK_API int32_t ppk_dequantize(ppk_context* ctx, void* stream, const PpkDequantizeArgs* args);

/* Single-query decode attention over int8 history plus the current token.
   For row r (sequence b = r / heads, p = past[b]):
     scores_t = softmax_scale * <q_r, K_r[t]>    t < p   (dequantised history)
     score_p  = softmax_scale * <q_r, sk_r>              (current token, unquantised)
     out_r    = sum_t softmax(scores)_t * V_r[t]  with V_r[p] = sv_r
   Rows with p > capacity produce NaN (int8_kv.cu:33,51).
   Replaces int8_kv_ops::attention (int8_kv_ops.rs:41-55) / cuda::Attention
   (int8_kv_ops.rs:143-161) and kernels pp_i8_attention + pp_i8_merge
   (int8_kv.cu:28-59). */
typedef struct PpkAttentionArgs {
  uint32_t struct_size;
  uint32_t q_dtype;        /* dtype of q */
  uint32_t scratch_dtype;  /* dtype of sk and sv */
  uint32_t out_dtype;      /* PPK_F32 (reference) or PPK_BF16 / PPK_F16 */
  uint32_t flags;          /* PPK_ATTN_* */
  uint32_t rows;           /* batch * heads */
  uint32_t heads;
  uint32_t capacity;       /* arena tokens per row */
  uint32_t head_dim;       /* 64, 128 or 256 */
  uint32_t split_tokens;   /* history tokens per wave; 0 = automatic. Result does not depend on it. */
  uint32_t max_past;       /* host upper bound of max(past); 0 = capacity. Rows beyond it give NaN. */
  float softmax_scale;     /* 0 = 1/sqrt(head_dim) */
  const void* q;           /* [rows, D] */
  const uint8_t* k_codes;  /* [rows, capacity, D], 16-byte aligned */
  const uint8_t* v_codes;  /* [rows, capacity, D], 16-byte aligned */
  const float* k_scales;   /* [rows, capacity] */
  const float* v_scales;   /* [rows, capacity] */
  const void* sk;          /* [rows, D] current key (not yet quantised) */
  const void* sv;          /* [rows, D] current value */
  const uint32_t* past;    /* device U32[rows / heads] */
  void* out;               /* [rows, D] */
  void* workspace;         /* ppk_attention_workspace_bytes() bytes, 256-byte aligned (may be NULL if 0) */
  uint64_t workspace_bytes;
  /* Optional (NULL, or absent when struct_size ends before it): a host copy
     of past[], the lengths the caller built before copying them to the
     device (app/src/model/batch.rs:152-161). With it the library balances a
     ragged batch: the plan, the workspace size and the work each wave takes
     follow the actual lengths (the per-row plan covers the longest live
     one). Each device past[b] is still read; a sequence whose device value
     differs gives its exact rows when the plan still covers them, and NaN
     rows otherwise (with PPK_FLAG_STALE_LENGTHS in a decode step's flags),
     never a wrong result. Only read during the call (a captured graph keeps
     the plan it saw). */
  const uint32_t* past_host;
} PpkAttentionArgs;
PPK_API int32_t ppk_attention_workspace_bytes(ppk_context* ctx, const PpkAttentionArgs* args, uint64_t* bytes);
/* The launch plan the library would use for args: history tokens per wave,
   number of blocks (groups) per row and workspace bytes (ctx may be NULL:
   assumes 256 CUs). One group per row means a single launch. The
   reference chooses split = 128 by default, clamped to 32..1024
   (int8_kv_ops.rs:52); its result does not depend on the split. */
PPK_API int32_t ppk_attention_plan(ppk_context* ctx, const PpkAttentionArgs* args, uint32_t* split_tokens,
                                   uint32_t* nsplits, uint64_t* workspace_bytes);
PPK_API int32_t ppk_decode_attention(ppk_context* ctx, void* stream, const PpkAttentionArgs* args);
/* The whole launch plan (no counterpart in the reference; for benchmarks and
   callers that size their own buffers): which of the two plans the library
   takes for args (PPK_ATTN_PLAN_PER_ROW, or PPK_ATTN_PLAN_BALANCED for a
   ragged batch's work list), the fields of ppk_attention_plan, the decode
   launch's grid and the number of launches a call makes (2 when a merge
   launch follows). info->struct_size must be set. */
typedef struct PpkAttentionPlanInfo {
  uint32_t struct_size;
  uint32_t kind;             /* PPK_ATTN_PLAN_PER_ROW or PPK_ATTN_PLAN_BALANCED */
  uint32_t split_tokens;     /* as ppk_attention_plan */
  uint32_t nsplits;          /* as ppk_attention_plan */
  uint32_t waves_per_block;
  uint32_t blocks;           /* blocks of the decode launch */
  uint32_t launches;         /* 1, or 2 with the merge launch */
  uint32_t reserved;
  uint64_t workspace_bytes;  /* as ppk_attention_plan */
} PpkAttentionPlanInfo;
PPK_API int32_t ppk_attention_plan_info(ppk_context* ctx, const PpkAttentionArgs* args, PpkAttentionPlanInfo* info);

/* One decode step in as few launches as the plan allows (one when a block of
   waves covers a whole row): quantise the current token k_new/v_new[row] and
   append it at slot past[b] of the attention arenas, then attend over
   [0, past[b]) plus the unquantised current token (attn.sk / attn.sv).
   Equivalent to ppk_quantize_append(tokens = 1) followed by
   ppk_decode_attention on the same arenas: the commit path of
   forward_embedding / forward_batched_embedding (app/src/model/mod.rs:699-705,
   app/src/model/batch.rs:152-161), where query_int8 appends before
   int8_kv_ops::attention reads the pre-append history. past[b] >= capacity
   skips that row's append and sets PPK_FLAG_OVERFLOW. */
typedef struct PpkDecodeStepArgs {
  uint32_t struct_size;
  uint32_t new_dtype;      /* dtype of k_new / v_new */
  const void* k_new;       /* [rows, D] */
  const void* v_new;       /* [rows, D] */
  uint32_t* flags;         /* optional device word, PPK_FLAG_* bits OR-ed in */
  PpkAttentionArgs attn;
} PpkDecodeStepArgs;
PPK_API int32_t ppk_decode_step(ppk_context* ctx, void* stream, const PpkDecodeStepArgs* args);

/* No counterpart in the reference. ppk_decode_step for callers that cannot
   allocate device memory (code under HIP graph capture, tight serving loops,
   harnesses that forbid hipMalloc): the same launches and results, but the
   partial records of rows that span several blocks go to a library-owned
   device array of PPK_NOALLOC_SCRATCH_BYTES per GPU (held from the first
   context on that GPU until the process ends) instead of attn.workspace,
   which is ignored. A plan that needs more (ppk_attention_plan's
   workspace_bytes) returns status 1 with nothing enqueued. Calls no
   hipMalloc / hipFree and never traces (ppk_context_set_profiling is ignored
   here). Every call on one GPU shares that GPU's array, which keeps the last
   call's records: calls that overlap in time on one GPU (two streams, two
   threads, two contexts) race and must be serialised by the caller. */
#define PPK_NOALLOC_SCRATCH_BYTES (8u << 20)
PPK_API int32_t ppk_decode_step_noalloc(ppk_context* ctx, void* stream, const PpkDecodeStepArgs* args);

/* Float-KV decode attention: the non-int8 decode path over unquantised bf16
   or f32 K/V, where the current token is already stored. For row r
   (sequence b = r / heads):
     n     = lengths ? lengths[b] : size        (total attended tokens)
     out_r = sum_{t<n} softmax_t(softmax_scale * <q_r, K_r[t]>) * V_r[t]
   n == 0 or n > size gives NaN (decode_attention.hip:15,50); so does n beyond
   max_length when max_length is set. Replaces fused_attention::decode_attention
   (app/src/model/fused_attention.rs:8-30) / hip_attention::decode_attention
   (app/src/model/hip_attention.rs:47-113) and kernels pp_attention_f32/bf16 +
   pp_attention_merge (app/src/model/decode_attention.hip:9-66). The reference
   requires head_dim 64, size <= 1024, F32 q and F32 output; this entry point
   also takes head_dim 128/256, any size and bf16/f16 q or output. Row strides
   are in elements (Candle's stride()[0]); within a row, tokens are dense. */
typedef struct PpkFloatAttentionArgs {
  uint32_t struct_size;
  uint32_t kv_dtype;       /* PPK_BF16 or PPK_F32 (dtype of k and v) */
  uint32_t q_dtype;        /* PPK_F32 (reference), PPK_BF16 or PPK_F16 */
  uint32_t out_dtype;      /* PPK_F32 (reference), PPK_BF16 or PPK_F16 */
  uint32_t rows;           /* batch * heads */
  uint32_t heads;
  uint32_t size;           /* stored tokens per row (the K/V view's length) */
  uint32_t head_dim;       /* 64, 128 or 256 */
  uint32_t split_tokens;   /* tokens per wave; 0 = automatic. Result does not depend on it. */
  uint32_t max_length;     /* host upper bound of max(lengths); 0 = size. Needs lengths. */
  float softmax_scale;     /* 0 = 1/sqrt(head_dim) (the reference's 0.125 at head_dim 64) */
  uint32_t flags;          /* PPK_ATTN_PLAN_* (PPK_ATTN_BF16_HISTORY does not apply) */
  uint64_t q_row_stride;   /* elements between rows of q; 0 = head_dim */
  uint64_t k_row_stride;   /* elements between rows of k; 0 = size * head_dim; 16-byte multiple */
  uint64_t v_row_stride;   /* elements between rows of v; 0 = size * head_dim; 16-byte multiple */
  const void* q;           /* rows x [head_dim] */
  const void* k;           /* rows x [size, head_dim], 16-byte aligned */
  const void* v;           /* rows x [size, head_dim], 16-byte aligned */
  const uint32_t* lengths; /* device U32[rows / heads], or NULL (every row attends size tokens) */
  void* out;               /* [rows, head_dim] */
  void* workspace;         /* ppk_float_attention_plan() bytes, 256-byte aligned (may be NULL if 0) */
  uint64_t workspace_bytes;
  /* Optional (NULL, or absent when struct_size ends before it): a host copy
     of lengths[] (needs lengths). With it a ragged batch is balanced as in
     PpkAttentionArgs.past_host: the plan and the workspace size follow the
     actual lengths, each device lengths[b] is still read, and a sequence
     whose device value differs gives its exact rows when the plan still
     covers them and NaN rows otherwise (with PPK_FLAG_STALE_LENGTHS in a
     decode step's flags), never a wrong result. Only read during the call. */
  const uint32_t* lengths_host;
} PpkFloatAttentionArgs;
/* Launch plan for args (ctx may be NULL: assumes 256 CUs), as ppk_attention_plan. */
PPK_API int32_t ppk_float_attention_plan(ppk_context* ctx, const PpkFloatAttentionArgs* args,
                                         uint32_t* split_tokens, uint32_t* nsplits, uint64_t* workspace_bytes);
PPK_API int32_t ppk_float_decode_attention(ppk_context* ctx, void* stream, const PpkFloatAttentionArgs* args);
/* The float path's launch plan, as ppk_attention_plan_info. */
PPK_API int32_t ppk_float_attention_plan_info(ppk_context* ctx, const PpkFloatAttentionArgs* args,
                                              PpkAttentionPlanInfo* info);

/* The float path's fused decode step: the caller's commit and attention in
   one launch per layer (two when rows span blocks). Replaces the graph-decode
   session's per-layer pair scatter_set(write_indices, k / v) +
   decode_attention(valid_lengths = lengths + 1)
   (app/src/model/graph_decode.rs:290-305) and the float cache's commit +
   fused_attention::decode_attention of forward_embedding
   (app/src/model/mod.rs:699-720). With attn.lengths[b] = p, the tokens
   already stored for sequence b (required), row r's current key and value
   (k_new / v_new [rows, head_dim] of new_dtype, rounded to kv_dtype) are
   written at slot p of attn.k / attn.v, which the call writes, when p < size
   (otherwise PPK_FLAG_OVERFLOW in *flags, if given, and nothing is written),
   and out_r is attention over the p stored tokens plus that token, exactly
   what ppk_float_decode_attention gives after the write with lengths p + 1.
   A row gives NaN unless p < size and p + 1 <= max_length (when set).
   attn.lengths_host, if given, holds p, and the plan and workspace are those
   of ppk_float_attention_plan(attn). No counterpart fuses these in the
   reference. */
typedef struct PpkFloatDecodeStepArgs {
  uint32_t struct_size;
  uint32_t new_dtype;      /* PPK_F32, PPK_BF16 or PPK_F16 */
  const void* k_new;       /* [rows, head_dim] current keys */
  const void* v_new;       /* [rows, head_dim] current values */
  uint32_t* flags;         /* optional device word, PPK_FLAG_* bits OR-ed in */
  PpkFloatAttentionArgs attn;
} PpkFloatDecodeStepArgs;
PPK_API int32_t ppk_float_decode_step(ppk_context* ctx, void* stream, const PpkFloatDecodeStepArgs* args);
/* The float path's private known-answer check: hip_attention::validate_split_k
   (app/src/model/hip_attention.rs:18-45; bf16 and f32 stores of 257 tokens,
   split 0 and 128 within 1e-4 of an f32 softmax reference and of each other)
   and the zero-input check of prepare_optional_kernels (app/src/model/mod.rs:440-451).
   Returns 2 with the failing check in ppk_last_error() on a numeric mismatch. */
PPK_API int32_t ppk_float_attention_prepare(ppk_context* ctx);

/* CFG + Renyi effective-support sampler, the decode loop's step after
   attention. Replaces hip_sampling::sample (app/src/inference/hip_sampling.rs:71-106)
   and kernel pp_hip_renyi_sample (app/src/inference/renyi_sample.hip:23-204).
   For logical row b (raw rows b*guidance [+1] = conditional [, unconditional]):
     v_c = guidance == 2 ? u_c + cfg * (c_c - u_c) : c_c      over all choices
     legal candidates [start_b, start_b + count_b) from bounds[b] = (start, count)
     H = log Z + max(0, log Z - log Z_alpha) / (alpha - 1), clamped to [0, ln count]
     support = clamp((u32)(exp(H) + 0.5), 1, count); rank = min((u32)(uniform_b * support), support - 1)
     token = token_offset + the rank-th legal column by (v descending, column ascending)
   out = U32 [3, batch]: tokens, valid flags, supports. A non-finite logit
   anywhere in the head, a uniform outside [0, 1) or bounds outside the head
   give valid = 0, support = 1 and a placeholder token (the reference's rule).
   Host checks: guidance 1 or 2 (cfg == 1 for 1), 1 <= choices <= 2048,
   finite alpha > 1, finite cfg >= 0, token_offset + choices - 1 < 2^32. */
typedef struct PpkRenyiSampleArgs {
  uint32_t struct_size;
  uint32_t batch;          /* logical rows */
  uint32_t choices;        /* head width, 1..2048 */
  uint32_t guidance;       /* 1, or 2 for interleaved (conditional, unconditional) rows */
  float alpha;             /* Renyi order, > 1 */
  float cfg;               /* guidance scale, >= 0 (1 when guidance == 1) */
  uint32_t token_offset;   /* added to the selected column */
  uint32_t reserved;
  const float* raw;        /* F32 [batch * guidance, choices], contiguous */
  const float* uniforms;   /* F32 [batch] */
  const uint32_t* bounds;  /* U32 [batch, 2] */
  uint32_t* out;           /* U32 [3, batch] */
} PpkRenyiSampleArgs;
PPK_API int32_t ppk_renyi_sample(ppk_context* ctx, void* stream, const PpkRenyiSampleArgs* args);

/* ---------------------------------------------------------------------------
   KV arenas: per-(sequence, layer) caches over shared device arenas, with
   copy-on-write snapshots, slot reuse and one write plan shared by every
   layer of a decode round. Replaces LayerCache (app/src/model/cache.rs:40-531),
   Int8LayerCache's commit path (app/src/model/int8_cache.rs:292-359) and
   BatchWritePlan (app/src/model/write_plan.rs:12-102).

   A cache is one sequence's K/V history for one layer: heads rows of
   capacity token slots, each slot head_dim values (int8 codes + one f32 scale
   per slot for PPK_KV_INT8, raw bf16/f16/f32 otherwise). Rules kept from the
   reference:
   * capacity starts at min_capacity (64) and doubles up to max_context (1024 in
     the reference, MAX_CONTEXT, app/src/model/mod.rs:55);
   * ppk_kv_cache_clone is a snapshot sharing storage; a write through a cache
     whose storage is shared (or too small) first copies the committed prefix
     (never uncommitted scratch) into storage of its own;
   * commit = 0 writes scratch at slot `past` without advancing the length;
     truncation is metadata only;
   * ppk_kv_query_batch writes one token per sequence into one batch arena
     [batch * heads, capacity, head_dim], reusing the arena the caches already
     share when every row is provably theirs alone (no live snapshot of a
     replaced slot, same row order, same capacity), otherwise moving every row
     into a fresh arena (committed prefixes copied once);
   * every shape, length and plan check completes before any device write.
   The context must outlive its caches and plans. Calls that touch caches
   sharing an arena must be serialised by the caller, on one stream; storage
   is released stream-ordered (hipFreeAsync) on the stream that last wrote or
   copied it, so that stream must still exist when the last cache or plan
   using the storage is released, and work reading a view on another stream
   must be ordered before that release by the caller. Calls that allocate
   (a first write, growth, copy-on-write, a new batch arena) refuse to run
   under HIP graph capture. Arenas and plan vectors come from a memory pool
   owned by the context (not the runtime's default pool); the storage of
   released caches is kept by the context (up to 32 GiB, or an eighth of the
   device's memory if less; the oldest goes first) for the next arena of the
   same size (the reusing stream first waits for an event recorded on the
   stream that last used it), handed back when an allocation would otherwise
   run out of device memory, and returned at ppk_context_release. */
enum { PPK_KV_INT8 = 0, PPK_KV_BF16 = 1, PPK_KV_F16 = 2, PPK_KV_F32 = 3 };

typedef struct ppk_kv_cache ppk_kv_cache;
typedef struct ppk_write_plan ppk_write_plan;

typedef struct PpkKvConfig {
  uint32_t struct_size;
  uint32_t kind;          /* PPK_KV_* */
  uint32_t heads;
  uint32_t head_dim;      /* 64/128/256 for PPK_KV_INT8; any >= 1 for float kinds */
  uint32_t max_context;   /* 0 = 1024 (the reference's MAX_CONTEXT) */
  uint32_t min_capacity;  /* 0 = 64 (the reference's MIN_CAPACITY) */
} PpkKvConfig;

/* Device view of cache storage. For a single cache: rows = heads, the
   cache's own row block; for a batch: rows = batch * heads, the whole arena,
   with past[b] (the slot just written) and lengths[b] = past[b] + 1 as device
   U32[batch] vectors ready for ppk_decode_attention (past) and
   ppk_float_decode_attention (lengths). Pointers stay valid until the next
   write through any cache of the arena or the arena's release. */
typedef struct PpkKvView {
  uint32_t struct_size;
  uint32_t kind;
  uint32_t rows;
  uint32_t capacity;      /* slots per row: the row stride is capacity * head_dim elements */
  uint32_t head_dim;
  uint32_t length;        /* slots holding data: end of the write (single) or max(past) + 1 (batch); committed length (ppk_kv_cache_view) */
  uint32_t batch;         /* 0 for a single-cache view */
  uint32_t reserved;
  void* k;                /* [rows, capacity, head_dim]: codes (u8) or floats */
  void* v;
  float* k_scales;        /* [rows, capacity] (PPK_KV_INT8), else NULL */
  float* v_scales;
  const uint32_t* past;   /* batch views: device U32[batch] */
  const uint32_t* lengths;/* batch views: device U32[batch] */
} PpkKvView;

typedef struct PpkKvInfo {
  uint32_t struct_size;
  uint32_t length;        /* committed tokens */
  uint32_t capacity;      /* 0 when no storage */
  uint32_t grouped;       /* 1 when the storage is a row of a batch arena */
  uint32_t slot;          /* row (sequence) index in its arena */
  uint32_t shared;        /* 1 when another cache (a snapshot) shares the storage */
  uint64_t reserved_bytes;/* device bytes of this cache's rows (reserve included) */
  uint64_t storage_id;    /* identity of the storage owner (changes on copy-on-write) */
  uint64_t arena_id;      /* identity of the arena */
  uint64_t arena_copied_rows;   /* sequences whose committed history was copied into this arena */
  uint64_t arena_offset_uploads;/* device offset vectors uploaded by this arena (writes without a plan) */
  uint64_t scale_bytes;   /* of reserved_bytes, the f32 scale planes (int8 caches; int8_cache.rs:291) */
} PpkKvInfo;

/* Source of a write: K and V [heads, tokens, head_dim] (single) or
   [batch, heads, 1, head_dim] (batch), dense, in src_dtype. INT8 caches
   quantise the source (any of f32/bf16/f16) as ppk_quantize does; float
   caches take the storage dtype only, as the reference's query does. */
typedef struct PpkKvWrite {
  uint32_t struct_size;
  uint32_t src_dtype;     /* PPK_F32 / PPK_BF16 / PPK_F16 */
  uint32_t tokens;        /* single writes; 1 for batch writes */
  uint32_t commit;        /* 0 = scratch write at slot past, length unchanged */
  const void* k;
  const void* v;
} PpkKvWrite;

PPK_API int32_t ppk_kv_cache_create(ppk_context* ctx, const PpkKvConfig* config, ppk_kv_cache** out);
PPK_API int32_t ppk_kv_cache_clone(const ppk_kv_cache* cache, ppk_kv_cache** out);
PPK_API int32_t ppk_kv_cache_release(ppk_kv_cache* cache);
PPK_API int32_t ppk_kv_cache_info(const ppk_kv_cache* cache, PpkKvInfo* out);
/* LayerCache::truncate_committed: new_len <= length; storage untouched. */
PPK_API int32_t ppk_kv_cache_truncate(ppk_kv_cache* cache, uint32_t new_len);
/* LayerCache::adopt_graph_view (app/src/model/cache.rs:55-64): a cache over
   caller-owned f32 K and V, each [heads, capacity, head_dim] (a graph decode
   session's buffers, config->kind = PPK_KV_F32), holding committed_len tokens.
   The library never frees or reallocates that memory; it must stay valid
   while the cache or a snapshot of it lives. Writes that fit go into it in
   place; growth, a write through a shared snapshot, or a batch write moves
   the cache into storage of its own (committed prefix copied). PpkKvInfo's
   storage_id is the graph storage identity (cache.rs:51-53). Errors:
   "invalid graph KV view" (not f32, null or misaligned, K and V overlapping,
   committed_len > capacity, capacity > max_context). */
PPK_API int32_t ppk_kv_cache_adopt(ppk_context* ctx, const PpkKvConfig* config, void* k, void* v,
                                   uint32_t capacity, uint32_t committed_len, ppk_kv_cache** out);
/* LayerCache::advance_graph_length (cache.rs:66-73): metadata-only commit of
   the slot a graph wrote; requires length == previous, next == previous + 1
   and next <= capacity ("graph KV commit length differs from validated host
   state"). */
PPK_API int32_t ppk_kv_cache_advance(ppk_kv_cache* cache, uint32_t previous, uint32_t next);
/* The cache's own rows, length = committed tokens (LayerCache::key / value / arena). */
PPK_API int32_t ppk_kv_cache_view(const ppk_kv_cache* cache, PpkKvView* out);
/* LayerCache::query / Int8LayerCache::query: write tokens at slot past
   (past must equal the committed length), growing or detaching first. */
PPK_API int32_t ppk_kv_query(ppk_context* ctx, void* stream, ppk_kv_cache* cache, uint32_t past,
                             const PpkKvWrite* write, PpkKvView* out);
/* BatchWritePlan::new: the write offsets of one decode round as a device
   vector (uploaded on stream), shared by every layer's ppk_kv_query_batch,
   which must run on the same stream (status 1 otherwise). Release returns
   the vector to the context, which hands it to the next plan created on the
   same stream (stream order keeps the new upload behind the old plan's work);
   plans are released before their context. */
PPK_API int32_t ppk_write_plan_create(ppk_context* ctx, void* stream, const uint32_t* past_lens, uint32_t batch,
                                      uint32_t heads, uint32_t head_dim, ppk_write_plan** out);
PPK_API int32_t ppk_write_plan_release(ppk_write_plan* plan);
/* LayerCache::query_batch_with_plan / Int8LayerCache::query_batch: one token
   per sequence at slot past_lens[b] (= each cache's committed length). A plan
   (optional) must match past_lens, heads and head_dim (checked on the host,
   no device read).
   No counterpart in the reference: for int8, bf16 and f32 caches, write->k
   and write->v both NULL reserve the slot instead — every step of the write
   happens (growth, copy-on-write, joins, the device past / lengths of the
   view, the commit) except storing the token, which the caller's fused step
   on the returned view then writes into slot past[b] in the same launch as
   the attention: ppk_decode_step for int8 caches (attn.k_codes = view.k,
   attn.past = view.past, k_new / v_new = the new token; the same codes,
   scales and output as the two calls), ppk_float_decode_step for bf16 / f32
   caches (attn.k = view.k, attn.size = view.capacity, attn.lengths =
   view.past, attn.max_length = view.length). The step must follow on the
   same stream before anything reads the slot. The reservation is a commit:
   if the step is then refused (status 1, nothing enqueued), each cache's
   slot past[b] stays committed and unwritten. Check the step's arguments
   first (ppk_attention_plan / ppk_float_attention_plan run every check the
   step runs on them), or undo the reservation with
   ppk_kv_cache_truncate(cache, past_lens[b]) on every cache of the batch
   before anything reads the slot. */
PPK_API int32_t ppk_kv_query_batch(ppk_context* ctx, void* stream, ppk_kv_cache* const* caches, uint32_t batch,
                                   const uint32_t* past_lens, const PpkKvWrite* write, const ppk_write_plan* plan,
                                   PpkKvView* out);

/* Known-answer self-check on the context's device, the three checks of
   int8_kv_ops::prepare (int8_kv_ops.rs:56-103) plus their fp32-history twins.
   Returns 2 with the failing check in ppk_last_error() on a numeric mismatch. */
PPK_API int32_t ppk_prepare(ppk_context* ctx);

/* The int8 KV capability gate: PrimitiveModel::prepare_int8_kv / Int8KvStatus
   (app/src/model/int8_policy.rs:3-56). Decision order as the reference:
   not requested -> disabled (status 0); requested but unavailable (head_dim
   not 64/128/256) -> disabled with the reason (status 0); requested and
   available -> the known-answer self-check of ppk_prepare runs once per
   context (its failure is returned with its status: 1, 2 or 3, and the
   reason says why), then enabled. Bytes per token and head: 2 * head_dim
   packed (K and V codes), 8 for the two f32 scales. */
typedef struct PpkInt8KvStatus {
  uint32_t struct_size;
  uint32_t requested;
  uint32_t available;
  uint32_t ready;
  uint32_t enabled;
  uint32_t packed_bytes_per_token_head;
  uint32_t scale_bytes_per_token_head;
  uint32_t reserved;
  char format[64];        /* "INT8 symmetric per-token/head + FP32 scales" when enabled */
  char reason[256];       /* UTF-8, NUL-terminated */
} PpkInt8KvStatus;
PPK_API int32_t ppk_prepare_int8_kv(ppk_context* ctx, uint32_t requested, uint32_t head_dim, PpkInt8KvStatus* out);

/* Tracing: when enabled, the library brackets every launch of the named kernel
   with HIP events on the launch stream; stats resolve them (blocking on the
   recorded events only) and report the number of traced launches and their
   total time. Kernel ids below. The reference keeps launch counters only
   (app/src/model/hip_kernel.rs:8-21). */
enum { PPK_KERNEL_QUANTIZE = 0, PPK_KERNEL_APPEND = 1, PPK_KERNEL_DEQUANTIZE = 2,
       PPK_KERNEL_ATTENTION = 3, /* the decode kernel, with or without the fused append */
       PPK_KERNEL_ATTN_MERGE = 4, PPK_KERNEL_FLOAT_ATTENTION = 5, PPK_KERNEL_FLOAT_MERGE = 6,
       PPK_KERNEL_RENYI_SAMPLE = 7,
       PPK_KERNEL_COPY = 8, /* arena prefix copies (joins, growth, copy-on-write) */
       PPK_KERNEL_COUNT = 9 };
PPK_API int32_t ppk_context_set_profiling(ppk_context* ctx, int32_t enable);
PPK_API int32_t ppk_context_kernel_stats(ppk_context* ctx, uint32_t kernel, uint64_t* launches,
                                 double* total_ms, uint32_t reset);
/* Wave-clock diagnostics (no counterpart in the reference). A context created
   with the diagnostics code object (ppk_kernels_clock.hsaco beside the
   library, built from the same sources with PPK_WAVE_CLOCK) makes every wave
   of the int8 per-row decode and merge kernels append a record of its
   real-time clock at fixed points (entry, first loads issued, past[b] here,
   first K data here, stream done, block joined, output stored) to `buffer`:
   16 u64 words per record at a slot of its own, u64 word 0 the slots per
   launch and kernel kind, word 1 the most records the caller wants kept
   (both set by the caller; records past bytes / 128 - 1 are dropped whatever
   word 1 says), records from word 16 (layout in
   pop2-bezier_amd/csrc/ppk_kernel_args.h). Each call starts the launch
   sequence numbers at 0. buffer NULL stops it; the library's own code object
   ignores it. Launches that overlap on one context write the same slots. */
PPK_API int32_t ppk_context_set_wave_clock(ppk_context* ctx, void* buffer, uint64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* PPK_INT8_KV_H */
