// C++ host mirror of fused_attention::decode_attention over
// run_float_attention, and the float path's private known-answer check.
#include "fused_attention.hpp"

#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace ppk::fused_attention {

namespace {

void check_exec(hipError_t st, const char* what) {
  if (st != hipSuccess) throw UncertainError(std::string(what) + ": " + hipGetErrorString(st));
}

uint16_t bf16_bits(float x) {  // round to nearest even, as Candle's to_dtype(BF16)
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if (std::isnan(x)) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
float bf16_value(uint16_t h) {
  const uint32_t u = uint32_t(h) << 16;
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

}  // namespace

Tensor decode_attention(ppk_context* ctx, hipStream_t stream, const Tensor& q, const Tensor& k, const Tensor& v,
                        const Tensor* lengths, size_t heads, size_t split_tokens) {
  const auto& qd = q.dims();
  const auto& kd = k.dims();
  require(heads > 0 && qd.size() == 3 && kd.size() == 3 && qd[0] > 0 && qd[0] <= 0xffffffffu && qd[0] % heads == 0 &&
              qd[1] == 1 && (qd[2] == 64 || qd[2] == 128 || qd[2] == 256) && kd[0] == qd[0] && kd[2] == qd[2] &&
              kd[1] > 0 && kd[1] <= 0xffffffffu && v.dims() == kd && q.dtype() == DType::F32 &&
              (k.dtype() == DType::BF16 || k.dtype() == DType::F32) && k.dtype() == v.dtype(),
          "fused decode attention requires F32[batch*heads,1,D] and same-device BF16/F32 K/V");
  const size_t rows = qd[0], length = kd[1], d = qd[2];
  if (lengths)
    require(lengths->dims() == std::vector<size_t>{rows / heads} && lengths->dtype() == DType::U32,
            "fused attention row lengths require same-device U32[batch]");
  Tensor out = Tensor::empty({rows, 1, d}, DType::F32);
  PpkFloatAttentionArgs a{};
  a.struct_size = sizeof(a);
  a.kv_dtype = k.dtype() == DType::BF16 ? PPK_BF16 : PPK_F32;
  a.q_dtype = PPK_F32;
  a.out_dtype = PPK_F32;
  a.rows = uint32_t(rows);
  a.heads = uint32_t(heads);
  a.size = uint32_t(length);
  a.head_dim = uint32_t(d);
  a.split_tokens = uint32_t(split_tokens);
  a.q = q.data();
  a.k = k.data();
  a.v = v.data();
  a.lengths = lengths ? static_cast<const uint32_t*>(lengths->data()) : nullptr;
  a.out = out.data();
  const AttentionPlan plan = plan_float_attention(ctx, a);
  Tensor workspace = Tensor::empty({plan.workspace_bytes}, DType::U8);
  a.workspace = workspace.data();
  a.workspace_bytes = plan.workspace_bytes;
  run_float_attention(ctx, stream, a);
  // The workspace must outlive the kernels that use it.
  check_exec(hipStreamSynchronize(stream), "hipStreamSynchronize");
  return out;
}

void validate_split_k(ppk_context* ctx) {
  DeviceGuard guard(ctx->device);
  hipStream_t stream = nullptr;
  check_exec(hipStreamCreate(&stream), "hipStreamCreate");
  struct StreamOwner {
    hipStream_t s;
    ~StreamOwner() { (void)hipStreamDestroy(s); }
  } owner{stream};

  // values(count, salt, scale) of hip_attention.rs:21.
  auto values = [](size_t count, size_t salt, float scale) {
    std::vector<float> out(count);
    for (size_t i = 0; i < count; ++i) out[i] = (float((i * 37 + salt) % 107) - 53.f) * scale;
    return out;
  };
  const auto qh = values(64, 17, 0.013f);
  const auto kh = values(257 * 64, 23, 0.011f);
  const auto vh = values(257 * 64, 31, 0.017f);
  Tensor q = Tensor::from_host(qh.data(), {1, 1, 64}, DType::F32, stream);
  for (DType dtype : {DType::BF16, DType::F32}) {
    std::vector<float> kf = kh, vf = vh;  // the values the store holds, widened to f32
    Tensor k, v;
    if (dtype == DType::BF16) {
      std::vector<uint16_t> kb(kh.size()), vb(vh.size());
      for (size_t i = 0; i < kh.size(); ++i) {
        kb[i] = bf16_bits(kh[i]);
        vb[i] = bf16_bits(vh[i]);
        kf[i] = bf16_value(kb[i]);
        vf[i] = bf16_value(vb[i]);
      }
      k = Tensor::from_host(kb.data(), {1, 257, 64}, DType::BF16, stream);
      v = Tensor::from_host(vb.data(), {1, 257, 64}, DType::BF16, stream);
    } else {
      k = Tensor::from_host(kh.data(), {1, 257, 64}, DType::F32, stream);
      v = Tensor::from_host(vh.data(), {1, 257, 64}, DType::F32, stream);
    }
    // softmax(q K^T / 8) V in f32 on the host.
    std::vector<float> scores(257);
    float mx = -INFINITY;
    for (size_t t = 0; t < 257; ++t) {
      float s = 0.f;
      for (size_t i = 0; i < 64; ++i) s += qh[i] * kf[t * 64 + i];
      scores[t] = s / 8.f;
      mx = std::max(mx, scores[t]);
    }
    float z = 0.f;
    for (float& s : scores) z += (s = std::exp(s - mx));
    std::vector<float> reference(64, 0.f);
    for (size_t t = 0; t < 257; ++t)
      for (size_t i = 0; i < 64; ++i) reference[i] += scores[t] / z * vf[t * 64 + i];
    const auto ordinary = decode_attention(ctx, stream, q, k, v, nullptr, 1, 0).to_host<float>(stream);
    const auto split = decode_attention(ctx, stream, q, k, v, nullptr, 1, 128).to_host<float>(stream);
    float pair = 0.f, ord = 0.f, spl = 0.f;
    bool finite = true;
    for (size_t i = 0; i < 64; ++i) {
      finite = finite && std::isfinite(ordinary[i]) && std::isfinite(split[i]) && std::isfinite(reference[i]);
      pair = std::max(pair, std::fabs(ordinary[i] - split[i]));
      ord = std::max(ord, std::fabs(reference[i] - ordinary[i]));
      spl = std::max(spl, std::fabs(reference[i] - split[i]));
    }
    if (!finite || pair > 1e-4f || ord > 1e-4f || spl > 1e-4f)
      throw InvalidOutputError(std::string(dtype == DType::BF16 ? "BF16" : "F32") +
                               " Split-K private numerical check failed, pair=" + std::to_string(pair) +
                               ", ordinary_vs_reference=" + std::to_string(ord) +
                               ", split_vs_reference=" + std::to_string(spl));

    // prepare_optional_kernels: all-zero q/K/V must give (near) zero.
    std::vector<uint8_t> zeros(257 * 64 * 4, 0);
    Tensor zq = Tensor::from_host(zeros.data(), {1, 1, 64}, DType::F32, stream);
    Tensor zk = Tensor::from_host(zeros.data(), {1, 257, 64}, dtype, stream);
    const auto zo = decode_attention(ctx, stream, zq, zk, zk, nullptr, 1, 128).to_host<float>(stream);
    for (float x : zo)
      if (!std::isfinite(x) || std::fabs(x) > 1e-6f) throw InvalidOutputError("fused attention preparation check failed");
  }
}

}  // namespace ppk::fused_attention

namespace ppk {
void float_attention_self_check(ppk_context* ctx) { fused_attention::validate_split_k(ctx); }
}  // namespace ppk
