// C++ host mirror of the reference's int8 KV custom-op API
// (app/src/model/int8_kv_ops.rs:5-103): the same four entry points with the
// same argument meaning and validation messages, over device tensors,
// calling the C-ABI launch paths. Candle allocates outputs per call
// (int8_kv_ops.rs:126,139-140,153); so does this mirror.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <utility>
#include <vector>

#include "ppk_internal.hpp"

namespace ppk::int8_kv_ops {

enum class DType { F32, BF16, F16, U8, U32 };
size_t dtype_size(DType t);

// A dense device tensor or a dim-0 view of one (Candle's narrow + start_offset).
class Tensor {
 public:
  static Tensor empty(std::vector<size_t> dims, DType dtype);
  static Tensor from_host(const void* data, std::vector<size_t> dims, DType dtype, hipStream_t stream);

  Tensor narrow0(size_t start, size_t len) const;
  template <class T>
  std::vector<T> to_host(hipStream_t stream) const {
    std::vector<T> out(numel());
    copy_to_host(out.data(), stream);
    return out;
  }

  void* data() const { return static_cast<char*>(storage_.get()) + offset_; }
  const std::vector<size_t>& dims() const { return dims_; }
  DType dtype() const { return dtype_; }
  size_t numel() const;
  size_t bytes() const { return numel() * dtype_size(dtype_); }

 private:
  void copy_to_host(void* dst, hipStream_t stream) const;
  std::shared_ptr<void> storage_;
  size_t offset_ = 0;
  std::vector<size_t> dims_;
  DType dtype_ = DType::F32;
};

// int8_kv_ops::quantize: input [heads, tokens, D] float -> (U8 codes [heads, tokens, D], F32 scales [heads, tokens]).
std::pair<Tensor, Tensor> quantize(ppk_context* ctx, hipStream_t stream, const Tensor& input);

// int8_kv_ops::dequantize: codes * scales, converted (round-to-nearest-even) to dtype.
Tensor dequantize(ppk_context* ctx, hipStream_t stream, const Tensor& packed, const Tensor& scale, DType dtype);

// int8_kv_ops::attention: q/sk/sv [rows,1,D], k/v U8 [rows,cap,D], ks/vs F32 [rows,cap],
// past U32 [rows/heads]; split_tokens 0 = automatic. Output F32 [rows,1,D].
Tensor attention(ppk_context* ctx, hipStream_t stream, const Tensor& q, const Tensor& k, const Tensor& v,
                 const Tensor& ks, const Tensor& vs, const Tensor& sk, const Tensor& sv, const Tensor& past,
                 size_t heads, size_t split_tokens, uint32_t flags = 0);

// int8_kv_ops::prepare: private known-answer checks on the context's device.
void prepare(ppk_context* ctx);

}  // namespace ppk::int8_kv_ops
