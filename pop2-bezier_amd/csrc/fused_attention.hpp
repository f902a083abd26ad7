// C++ host mirror of the reference's float-KV decode attention
// (app/src/model/fused_attention.rs:8-30, hip_attention.rs:7-113) over the
// C-ABI launch path, plus its private Split-K validation.
#pragma once
#include "int8_kv_ops.hpp"

namespace ppk::fused_attention {

using int8_kv_ops::DType;
using int8_kv_ops::Tensor;

// fused_attention::decode_attention: q F32 [rows,1,D], k/v BF16|F32 [rows,length,D]
// (the current token already stored), lengths U32 [rows/heads] or nullptr.
// split_tokens 0 = automatic. Output F32 [rows,1,D].
Tensor decode_attention(ppk_context* ctx, hipStream_t stream, const Tensor& q, const Tensor& k, const Tensor& v,
                        const Tensor* lengths, size_t heads, size_t split_tokens);

// hip_attention::validate_split_k (hip_attention.rs:18-45) and the zero-input
// check of prepare_optional_kernels (app/src/model/mod.rs:440-451).
void validate_split_k(ppk_context* ctx);

}  // namespace ppk::fused_attention
