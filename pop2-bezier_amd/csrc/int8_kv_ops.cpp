// C++ host mirror of app/src/model/int8_kv_ops.rs over the C-ABI launch
// paths, plus the private known-answer self-check (int8_kv_ops.rs:56-103).
#include "int8_kv_ops.hpp"

#include <cmath>
#include <cstring>
#include <limits>
#include <string>

namespace ppk::int8_kv_ops {

namespace {

void check_exec(hipError_t st, const char* what) {
  if (st != hipSuccess) throw UncertainError(std::string(what) + ": " + hipGetErrorString(st));
}

uint32_t abi_dtype(DType t) {
  switch (t) {
    case DType::F32: return PPK_F32;
    case DType::BF16: return PPK_BF16;
    case DType::F16: return PPK_F16;
    default: throw PreconditionError("INT8 KV floating operand has an integer dtype");
  }
}
bool is_float(DType t) { return t == DType::F32 || t == DType::BF16 || t == DType::F16; }

// geometry() of int8_kv_ops.rs:5-10, extended to D in {64, 128, 256}.
std::pair<size_t, size_t> geometry(const Tensor& t) {
  const auto& d = t.dims();
  require(d.size() == 3 && d[0] > 0 && d[1] > 0 && (d[2] == 64 || d[2] == 128 || d[2] == 256),
          "INT8 KV requires dense [heads,tokens,D] with D in {64,128,256}");
  return {d[0], d[1]};
}

std::vector<float> bf16_bits_to_f32(const std::vector<uint16_t>& h) {
  std::vector<float> out(h.size());
  for (size_t i = 0; i < h.size(); ++i) {
    const uint32_t u = uint32_t(h[i]) << 16;
    std::memcpy(&out[i], &u, 4);
  }
  return out;
}

}  // namespace

size_t dtype_size(DType t) {
  switch (t) {
    case DType::F32: case DType::U32: return 4;
    case DType::BF16: case DType::F16: return 2;
    case DType::U8: return 1;
  }
  return 1;
}

size_t Tensor::numel() const {
  size_t n = 1;
  for (size_t d : dims_) n *= d;
  return n;
}

Tensor Tensor::empty(std::vector<size_t> dims, DType dtype) {
  Tensor t;
  t.dims_ = std::move(dims);
  t.dtype_ = dtype;
  void* p = nullptr;
  const size_t bytes = std::max<size_t>(t.bytes(), 256);
  check_exec(hipMalloc(&p, bytes), "hipMalloc");
  t.storage_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
  return t;
}

Tensor Tensor::from_host(const void* data, std::vector<size_t> dims, DType dtype, hipStream_t stream) {
  Tensor t = empty(std::move(dims), dtype);
  check_exec(hipMemcpyAsync(t.data(), data, t.bytes(), hipMemcpyHostToDevice, stream), "hipMemcpyAsync H2D");
  check_exec(hipStreamSynchronize(stream), "hipStreamSynchronize");
  return t;
}

Tensor Tensor::narrow0(size_t start, size_t len) const {
  require(!dims_.empty() && start + len <= dims_[0], "narrow out of range");
  Tensor t = *this;
  size_t inner = dtype_size(dtype_);
  for (size_t i = 1; i < dims_.size(); ++i) inner *= dims_[i];
  t.offset_ = offset_ + start * inner;
  t.dims_[0] = len;
  return t;
}

void Tensor::copy_to_host(void* dst, hipStream_t stream) const {
  check_exec(hipMemcpyAsync(dst, data(), bytes(), hipMemcpyDeviceToHost, stream), "hipMemcpyAsync D2H");
  check_exec(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

std::pair<Tensor, Tensor> quantize(ppk_context* ctx, hipStream_t stream, const Tensor& input) {
  const auto [h, n] = geometry(input);
  require(is_float(input.dtype()), "INT8 KV quantize input must be f32, bf16 or f16");
  const size_t d = input.dims()[2];
  Tensor codes = Tensor::empty({h, n, d}, DType::U8);
  Tensor scales = Tensor::empty({h, n}, DType::F32);
  PpkQuantizeArgs a{};
  a.struct_size = sizeof(a);
  a.src_dtype = abi_dtype(input.dtype());
  a.src = input.data();
  a.codes = static_cast<uint8_t*>(codes.data());
  a.scales = static_cast<float*>(scales.data());
  a.rows = uint64_t(h) * n;
  a.head_dim = uint32_t(d);
  run_quantize(ctx, stream, a);
  return {codes, scales};
}

Tensor dequantize(ppk_context* ctx, hipStream_t stream, const Tensor& packed, const Tensor& scale, DType dtype) {
  const auto [h, n] = geometry(packed);
  require(packed.dtype() == DType::U8 && scale.dtype() == DType::F32 && scale.dims() == std::vector<size_t>{h, n},
          "INT8 KV scales differ");
  const size_t d = packed.dims()[2];
  Tensor out = Tensor::empty({h, n, d}, dtype);
  PpkDequantizeArgs a{};
  a.struct_size = sizeof(a);
  a.out_dtype = abi_dtype(dtype);
  a.codes = static_cast<const uint8_t*>(packed.data());
  a.scales = static_cast<const float*>(scale.data());
  a.out = out.data();
  a.rows = uint64_t(h) * n;
  a.head_dim = uint32_t(d);
  run_dequantize(ctx, stream, a);
  return out;
}

Tensor attention(ppk_context* ctx, hipStream_t stream, const Tensor& q, const Tensor& k, const Tensor& v,
                 const Tensor& ks, const Tensor& vs, const Tensor& sk, const Tensor& sv, const Tensor& past,
                 size_t heads, size_t split_tokens, uint32_t flags) {
  const auto [rows, capacity] = geometry(k);
  const size_t d = k.dims()[2];
  require(heads > 0 && rows % heads == 0 && v.dims() == k.dims() && k.dtype() == DType::U8 && v.dtype() == DType::U8,
          "INT8 attention geometry differs");
  for (const Tensor* t : {&q, &sk, &sv})
    require(t->dims() == std::vector<size_t>{rows, 1, d} && is_float(t->dtype()),
            "INT8 scratch must be float[head_rows,1,D]");
  require(sk.dtype() == sv.dtype(), "INT8 scratch key/value dtypes differ");
  for (const Tensor* t : {&ks, &vs})
    require(t->dims() == std::vector<size_t>{rows, capacity} && t->dtype() == DType::F32,
            "INT8 scales must be F32[head_rows,capacity]");
  require(past.dims() == std::vector<size_t>{rows / heads} && past.dtype() == DType::U32,
          "INT8 attention lengths differ");
  require(rows <= 0xffffffffu && capacity <= 0xffffffffu, "INT8 attention row grid overflow");

  Tensor out = Tensor::empty({rows, 1, d}, DType::F32);
  PpkAttentionArgs a{};
  a.struct_size = sizeof(a);
  a.q_dtype = abi_dtype(q.dtype());
  a.scratch_dtype = abi_dtype(sk.dtype());
  a.out_dtype = PPK_F32;
  a.flags = flags;
  a.rows = uint32_t(rows);
  a.heads = uint32_t(heads);
  a.capacity = uint32_t(capacity);
  a.head_dim = uint32_t(d);
  a.split_tokens = uint32_t(split_tokens);
  a.q = q.data();
  a.k_codes = static_cast<const uint8_t*>(k.data());
  a.v_codes = static_cast<const uint8_t*>(v.data());
  a.k_scales = static_cast<const float*>(ks.data());
  a.v_scales = static_cast<const float*>(vs.data());
  a.sk = sk.data();
  a.sv = sv.data();
  a.past = static_cast<const uint32_t*>(past.data());
  a.out = out.data();
  const AttentionPlan plan = plan_attention(ctx, a);
  Tensor workspace = Tensor::empty({plan.workspace_bytes}, DType::U8);
  a.workspace = workspace.data();
  a.workspace_bytes = plan.workspace_bytes;
  run_attention(ctx, stream, a);
  // The workspace must outlive the kernels that use it.
  check_exec(hipStreamSynchronize(stream), "hipStreamSynchronize");
  return out;
}

namespace {

// Host formula of int8_kv_ops.rs:69-73,95-98: f32 dot products summed in
// order, times 0.125, max-subtracted exp, probability-weighted values / z.
// hist(row, t, d) gives history element t < len; cur(row, d) the scratch.
template <class Hist, class Key, class Val, class VHist>
std::vector<float> host_attention(size_t rows, const std::vector<float>& qcpu, const std::vector<size_t>& lens,
                                  Hist khist, Key kcur, VHist vhist, Val vcur) {
  std::vector<float> out;
  for (size_t row = 0; row < rows; ++row) {
    const size_t len = lens[row];
    std::vector<float> scores;
    for (size_t t = 0; t <= len; ++t) {
      float s = 0.f;
      for (size_t d = 0; d < 64; ++d) s += qcpu[row * 64 + d] * (t == len ? kcur(row, d) : khist(row, t, d));
      scores.push_back(s * 0.125f);
    }
    float mx = -std::numeric_limits<float>::infinity();
    for (float s : scores) mx = std::max(mx, s);
    std::vector<float> p;
    float z = 0.f;
    for (float s : scores) {
      p.push_back(std::exp(s - mx));
    }
    for (float x : p) z += x;
    for (size_t d = 0; d < 64; ++d) {
      float acc = 0.f;
      for (size_t t = 0; t <= len; ++t) acc += p[t] * (t == len ? vcur(row, d) : vhist(row, t, d));
      out.push_back(acc / z);
    }
  }
  return out;
}

void expect_close(const std::vector<float>& actual, const std::vector<float>& expected, float tol, const char* what) {
  if (actual.size() != expected.size()) throw InvalidOutputError(std::string(what) + ": size mismatch");
  for (size_t i = 0; i < actual.size(); ++i)
    if (!std::isfinite(actual[i]) || std::fabs(actual[i] - expected[i]) >= tol)
      throw InvalidOutputError(std::string(what) + " failed at element " + std::to_string(i) + ": got " +
                               std::to_string(actual[i]) + ", expected " + std::to_string(expected[i]));
}

}  // namespace

void prepare(ppk_context* ctx) {
  DeviceGuard guard(ctx->device);
  hipStream_t stream = nullptr;
  check_exec(hipStreamCreate(&stream), "hipStreamCreate");
  struct StreamOwner {
    hipStream_t s;
    ~StreamOwner() { (void)hipStreamDestroy(s); }
  } owner{stream};

  // (i) Quantize round trip, int8_kv_ops.rs:59-62.
  std::vector<float> data(384);
  for (size_t i = 0; i < data.size(); ++i) data[i] = std::sin(float(i) * 0.17f) * 2.f;
  Tensor x = Tensor::from_host(data.data(), {2, 3, 64}, DType::F32, stream);
  auto [k, s] = quantize(ctx, stream, x);
  const auto restored = dequantize(ctx, stream, k, s, DType::F32).to_host<float>(stream);
  for (size_t i = 0; i < data.size(); ++i)
    if (!std::isfinite(restored[i]) || std::fabs(restored[i] - data[i]) >= 0.009f)
      throw InvalidOutputError("KV INT8 quantization self-check failed");

  // (ii) Attention vs the host formula, int8_kv_ops.rs:63-74.
  std::vector<float> qdata(128), scratch(128);
  for (size_t i = 0; i < 128; ++i) {
    qdata[i] = std::cos(float(i) * 0.07f);
    scratch[i] = std::sin(float(i) * 0.09f);
  }
  Tensor q = Tensor::from_host(qdata.data(), {2, 1, 64}, DType::F32, stream);
  Tensor sk = Tensor::from_host(scratch.data(), {2, 1, 64}, DType::F32, stream);
  const uint32_t past_host[2] = {2, 1};
  Tensor past = Tensor::from_host(past_host, {2}, DType::U32, stream);
  const auto rounded = bf16_bits_to_f32(dequantize(ctx, stream, k, s, DType::BF16).to_host<uint16_t>(stream));
  const std::vector<size_t> lens2 = {2, 1};
  for (int mode = 0; mode < 2; ++mode) {
    const std::vector<float>& hist = mode ? rounded : restored;
    auto kh = [&](size_t row, size_t t, size_t d) { return hist[(row * 3 + t) * 64 + d]; };
    auto cur = [&](size_t row, size_t d) { return scratch[row * 64 + d]; };
    const auto expected = host_attention(2, qdata, lens2, kh, cur, kh, cur);
    const auto actual =
        attention(ctx, stream, q, k, k, s, s, sk, sk, past, 1, 32, mode ? PPK_ATTN_BF16_HISTORY : 0)
            .to_host<float>(stream);
    expect_close(actual, expected, 2e-5f, mode ? "KV INT8 attention self-check (bf16 history)"
                                               : "KV INT8 attention self-check (fp32 history)");
  }

  // (iii) Nonzero view offsets, two heads per sequence, an empty committed
  // history, unequal lengths and split reduction, int8_kv_ops.rs:75-101.
  const size_t rows = 4, capacity = 67, heads = 2;
  std::vector<float> history((rows + 1) * capacity * 64), values(history.size());
  for (size_t i = 0; i < history.size(); ++i) {
    history[i] = std::sin(float(i) * 0.013f) * 1.7f;
    values[i] = std::cos(float(i) * 0.019f) * 0.8f;
  }
  Tensor hist_t = Tensor::from_host(history.data(), {rows + 1, capacity, 64}, DType::F32, stream).narrow0(1, rows);
  Tensor vals_t = Tensor::from_host(values.data(), {rows + 1, capacity, 64}, DType::F32, stream).narrow0(1, rows);
  auto [kq, ksq] = quantize(ctx, stream, hist_t);
  auto [vq, vsq] = quantize(ctx, stream, vals_t);
  // Re-home the packed tensors and scales at a one-row offset too.
  auto offset_copy = [&](const Tensor& t) {
    std::vector<size_t> dims = t.dims();
    dims[0] += 1;
    Tensor big = Tensor::empty(dims, t.dtype());
    check_exec(hipMemsetAsync(big.data(), 0, big.bytes(), stream), "hipMemsetAsync");
    Tensor view = big.narrow0(1, rows);
    check_exec(hipMemcpyAsync(view.data(), t.data(), t.bytes(), hipMemcpyDeviceToDevice, stream), "hipMemcpyAsync");
    return view;
  };
  Tensor kv = offset_copy(kq), vv = offset_copy(vq), ksv = offset_copy(ksq), vsv = offset_copy(vsq);
  auto vector = [&](float factor, float phase) {
    std::vector<float> h((rows + 1) * 64);
    for (size_t i = 0; i < h.size(); ++i) h[i] = std::sin(float(i) * factor + phase);
    return h;
  };
  const auto qh = vector(0.027f, 0.4f), skh = vector(0.031f, 1.1f), svh = vector(0.047f, -0.8f);
  Tensor q3 = Tensor::from_host(qh.data(), {rows + 1, 1, 64}, DType::F32, stream).narrow0(1, rows);
  Tensor sk3 = Tensor::from_host(skh.data(), {rows + 1, 1, 64}, DType::F32, stream).narrow0(1, rows);
  Tensor sv3 = Tensor::from_host(svh.data(), {rows + 1, 1, 64}, DType::F32, stream).narrow0(1, rows);
  const uint32_t past3_host[3] = {999, 0, 66};
  Tensor past3 = Tensor::from_host(past3_host, {3}, DType::U32, stream).narrow0(1, 2);
  const auto kc_bf = bf16_bits_to_f32(dequantize(ctx, stream, kv, ksv, DType::BF16).to_host<uint16_t>(stream));
  const auto vc_bf = bf16_bits_to_f32(dequantize(ctx, stream, vv, vsv, DType::BF16).to_host<uint16_t>(stream));
  const auto kc_f = dequantize(ctx, stream, kv, ksv, DType::F32).to_host<float>(stream);
  const auto vc_f = dequantize(ctx, stream, vv, vsv, DType::F32).to_host<float>(stream);
  std::vector<size_t> lens3(rows);
  for (size_t row = 0; row < rows; ++row) lens3[row] = (row / heads == 0) ? 0 : 66;
  std::vector<float> qcpu(qh.begin() + 64, qh.end());
  for (int mode = 0; mode < 2; ++mode) {
    const auto& kc = mode ? kc_bf : kc_f;
    const auto& vc = mode ? vc_bf : vc_f;
    auto kh = [&](size_t row, size_t t, size_t d) { return kc[(row * capacity + t) * 64 + d]; };
    auto vh = [&](size_t row, size_t t, size_t d) { return vc[(row * capacity + t) * 64 + d]; };
    auto kcur = [&](size_t row, size_t d) { return skh[(row + 1) * 64 + d]; };
    auto vcur = [&](size_t row, size_t d) { return svh[(row + 1) * 64 + d]; };
    const auto expected = host_attention(rows, qcpu, lens3, kh, kcur, vh, vcur);
    for (size_t split : {32u, 128u}) {
      const auto actual = attention(ctx, stream, q3, kv, vv, ksv, vsv, sk3, sv3, past3, heads, split,
                                    mode ? PPK_ATTN_BF16_HISTORY : 0)
                              .to_host<float>(stream);
      expect_close(actual, expected, 2e-5f, "KV INT8 offset/split attention self-check");
    }
  }
}

}  // namespace ppk::int8_kv_ops

namespace ppk {
void prepare_self_check(ppk_context* ctx) { int8_kv_ops::prepare(ctx); }
}  // namespace ppk
