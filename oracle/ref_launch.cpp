// TEST INFRASTRUCTURE ONLY (checker, never the product): launches the
// reference's own HIP kernels, built unchanged from /root/reference into
// oracle/_ref/*.hsaco by oracle/build_ref.py, with the launch geometry of the
// reference's host code:
//   pp_attention_f32/bf16 + pp_attention_merge  (app/src/model/hip_attention.rs:98-112):
//     split = split_tokens ? clamp(split_tokens, 32, 1024) : length (hip_attention.rs:55),
//     grid (rows, ceil(length / split)), block 256, dynamic LDS (split + 256) * 4 bytes;
//     with more than one split, 66-float partial records and a (rows) x 64 merge launch.
//   pp_hip_renyi_sample (app/src/inference/hip_sampling.rs:183-214):
//     grid (batch), block 256, dynamic LDS next_pow2(choices) * 8 + 256 * 16 bytes.
// Used by tests/ to compare this repository's kernels with the reference's
// on the same device buffers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <string>

namespace {

thread_local std::string g_error;
hipModule_t g_attn = nullptr, g_sample = nullptr;

int fail(const std::string& what, hipError_t st) {
  g_error = what + ": " + hipGetErrorString(st);
  return 1;
}

int load(hipModule_t* m, const char* path) {
  if (*m) return 0;
  const hipError_t st = hipModuleLoad(m, path);
  if (st != hipSuccess) return fail(std::string("hipModuleLoad ") + path, st);
  return 0;
}

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

int ref_load(const char* attention_hsaco, const char* sampler_hsaco) {
  if (load(&g_attn, attention_hsaco)) return 1;
  return load(&g_sample, sampler_hsaco);
}

// q F32 rows x [64] (row stride qs), k/v bf16 or f32 rows x [length, 64]
// (row strides ks/vs), lengths U32[rows/heads] or null, out F32 [rows, 64].
// partial: F32 scratch of rows * splits * 66 floats when splits > 1.
int ref_decode_attention(void* stream, int kv_bf16, const float* q, const void* k, const void* v,
                         const uint32_t* lengths, float* out, float* partial, uint32_t heads, uint32_t rows,
                         uint32_t length, uint32_t split_tokens, uint64_t qs, uint64_t ks, uint64_t vs) {
  if (!g_attn) {
    g_error = "reference attention module not loaded";
    return 1;
  }
  uint32_t split = split_tokens ? std::min(std::max(split_tokens, 32u), 1024u) : length;
  uint32_t splits = (length + split - 1) / split;
  hipFunction_t fn = nullptr, merge = nullptr;
  hipError_t st = hipModuleGetFunction(&fn, g_attn, kv_bf16 ? "pp_attention_bf16" : "pp_attention_f32");
  if (st != hipSuccess) return fail("pp_attention", st);
  st = hipModuleGetFunction(&merge, g_attn, "pp_attention_merge");
  if (st != hipSuccess) return fail("pp_attention_merge", st);
  if (splits > 1 && !partial) {
    g_error = "partial buffer required";
    return 1;
  }
  const void* lp = lengths;
  float* op = splits > 1 ? partial : out;
  uint32_t dynamic = lengths ? 1u : 0u;
  void* args[] = {&q, &k, &v, &lp, &op, &heads, &length, &split, &splits, &dynamic, &qs, &ks, &vs};
  st = hipModuleLaunchKernel(fn, rows, splits, 1, 256, 1, 1, (split + 256) * 4, static_cast<hipStream_t>(stream),
                             args, nullptr);
  if (st != hipSuccess) return fail("launch pp_attention", st);
  if (splits > 1) {
    const float* in = partial;
    void* margs[] = {&in, &out, &splits};
    st = hipModuleLaunchKernel(merge, rows, 1, 1, 64, 1, 1, 0, static_cast<hipStream_t>(stream), margs, nullptr);
    if (st != hipSuccess) return fail("launch pp_attention_merge", st);
  }
  return 0;
}

int ref_renyi_sample(void* stream, const float* raw, const float* uniforms, const uint32_t* bounds, uint32_t* out,
                     uint32_t batch, uint32_t choices, uint32_t guidance, float alpha, float cfg, uint32_t offset) {
  if (!g_sample) {
    g_error = "reference sampler module not loaded";
    return 1;
  }
  hipFunction_t fn = nullptr;
  hipError_t st = hipModuleGetFunction(&fn, g_sample, "pp_hip_renyi_sample");
  if (st != hipSuccess) return fail("pp_hip_renyi_sample", st);
  uint32_t padded = 1;
  while (padded < choices) padded <<= 1;
  void* args[] = {&raw, &uniforms, &bounds, &out, &batch, &choices, &guidance, &alpha, &cfg, &offset, &padded};
  st = hipModuleLaunchKernel(fn, batch, 1, 1, 256, 1, 1, padded * 8 + 256 * 16, static_cast<hipStream_t>(stream),
                             args, nullptr);
  if (st != hipSuccess) return fail("launch pp_hip_renyi_sample", st);
  return 0;
}

}  // extern "C"
