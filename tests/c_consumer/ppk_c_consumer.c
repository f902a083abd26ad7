/*
 * A plain C host of the C-ABI (no Python, no torch): device memory from the
 * HIP runtime's C API, every call through include/ppk_int8_kv.h, the way the
 * reference's Rust side would bind it (the quantize op of int8_kv_ops.rs:11-29
 * and the attention op of int8_kv_ops.rs:41-55 / :143-161).
 *
 * Test infrastructure: the results are checked against the CPU oracle
 * (oracle/ppk_oracle.c) — codes and scales bit for bit, attention within
 * max |err| <= 2e-3 and max relative error <= 1e-2 where |oracle| >= 1e-3.
 * Exit status 0 when every check passes; each check prints one line.
 *
 * Shapes: B = 2 sequences, H = 4 heads, D = 128, capacity 300, past = {257, 100}
 * (ragged), under the library's plan, 8-token splits (several blocks per row
 * joined by the merge kernel) and host lengths; dequantize; and the fused
 * decode step (commit of the current token + attention).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "ppk_int8_kv.h"

/* The oracle's entry points (oracle/ppk_oracle.c). */
size_t oracle_quantize(const float* x, size_t rows, size_t d, uint8_t* codes, float* scales);
void oracle_attention(const float* q, const uint8_t* k, const uint8_t* v, const float* ks, const float* vs,
                      const float* sk, const float* sv, const uint32_t* past, size_t rows, size_t heads,
                      size_t capacity, size_t d, float scale, int history_bf16, double* out);
void oracle_dequantize(const uint8_t* codes, const float* scales, size_t rows, size_t d, int round, float* out);

enum { B = 2, H = 4, D = 128, CAP = 300, ROWS = B * H };

static int failures = 0;

static void check(int ok, const char* what) {
  printf("%s: %s\n", ok ? "pass" : "FAIL", what);
  if (!ok) ++failures;
}

static int hip_ok(hipError_t st, const char* what) {
  if (st != hipSuccess) {
    printf("FAIL: %s: %s\n", what, hipGetErrorString(st));
    ++failures;
    return 0;
  }
  return 1;
}

static int ppk_ok(int32_t st, const char* what) {
  if (st != 0) {
    printf("FAIL: %s: status %d: %s\n", what, (int)st, ppk_last_error());
    ++failures;
    return 0;
  }
  return 1;
}

/* Seeded uniform values in [-2, 2) with every 37th channel ten times larger. */
static void fill(float* x, size_t n, uint64_t seed) {
  uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
  for (size_t i = 0; i < n; ++i) {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    const float u = (float)((s >> 40) & 0xFFFFFF) / 16777216.0f;
    x[i] = (4.0f * u - 2.0f) * ((i % D) % 37 == 0 ? 10.0f : 1.0f);
  }
}

static void* dev_alloc(size_t bytes) {
  void* p = NULL;
  return hip_ok(hipMalloc(&p, bytes), "hipMalloc") ? p : NULL;
}

/* One attention call through the C-ABI with the given split (0 = the library's plan), compared with ref. */
static void attend(ppk_context* ctx, const PpkAttentionArgs* base, uint32_t split, const double* ref,
                   float* out_host, const char* what) {
  PpkAttentionArgs a = *base;
  a.split_tokens = split;
  uint32_t plan_split = 0, nsplits = 0;
  uint64_t ws = 0;
  if (!ppk_ok(ppk_attention_plan(ctx, &a, &plan_split, &nsplits, &ws), "ppk_attention_plan")) return;
  void* workspace = ws ? dev_alloc(ws) : NULL;
  if (ws && !workspace) return;
  a.workspace = workspace;
  a.workspace_bytes = ws;
  if (ppk_ok(ppk_decode_attention(ctx, NULL, &a), "ppk_decode_attention") &&
      hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize") &&
      hip_ok(hipMemcpy(out_host, a.out, sizeof(float) * ROWS * D, hipMemcpyDeviceToHost), "copy out")) {
    double max_abs = 0.0, max_rel = 0.0;
    int finite = 1;
    for (size_t i = 0; i < (size_t)ROWS * D; ++i) {
      if (!isfinite(out_host[i])) finite = 0;
      const double err = fabs((double)out_host[i] - ref[i]);
      if (err > max_abs) max_abs = err;
      if (fabs(ref[i]) >= 1e-3 && err / fabs(ref[i]) > max_rel) max_rel = err / fabs(ref[i]);
    }
    char line[256];
    snprintf(line, sizeof line, "%s (split %u, %u block(s) per row): max abs %.3e, max rel %.3e", what,
             plan_split, nsplits, max_abs, max_rel);
    check(finite && max_abs <= 2e-3 && max_rel <= 1e-2, line);
  }
  if (workspace) hipFree(workspace);
}

int main(void) {
  check(ppk_abi_version() == PPK_ABI_VERSION, "ppk_abi_version matches the header");
  ppk_context* ctx = NULL;
  if (!ppk_ok(ppk_context_create(0, NULL, &ctx), "ppk_context_create")) return 1;

  const size_t hist_rows = (size_t)ROWS * CAP;
  float* hist_k = malloc(sizeof(float) * hist_rows * D);
  float* hist_v = malloc(sizeof(float) * hist_rows * D);
  float* q = malloc(sizeof(float) * ROWS * D);
  float* sk = malloc(sizeof(float) * ROWS * D);
  float* sv = malloc(sizeof(float) * ROWS * D);
  uint8_t* kc = malloc(hist_rows * D);
  uint8_t* vc = malloc(hist_rows * D);
  float* ks = malloc(sizeof(float) * hist_rows);
  float* vs = malloc(sizeof(float) * hist_rows);
  uint8_t* okc = malloc(hist_rows * D);
  float* oks = malloc(sizeof(float) * hist_rows);
  double* ref = malloc(sizeof(double) * ROWS * D);
  float* out = malloc(sizeof(float) * ROWS * D);
  const uint32_t past[B] = {257, 100};
  fill(hist_k, hist_rows * D, 1);
  fill(hist_v, hist_rows * D, 2);
  fill(q, (size_t)ROWS * D, 3);
  fill(sk, (size_t)ROWS * D, 4);
  fill(sv, (size_t)ROWS * D, 5);

  float* d_src = dev_alloc(sizeof(float) * hist_rows * D);
  uint8_t* d_kc = dev_alloc(hist_rows * D);
  uint8_t* d_vc = dev_alloc(hist_rows * D);
  float* d_ks = dev_alloc(sizeof(float) * hist_rows);
  float* d_vs = dev_alloc(sizeof(float) * hist_rows);
  float* d_q = dev_alloc(sizeof(float) * ROWS * D);
  float* d_sk = dev_alloc(sizeof(float) * ROWS * D);
  float* d_sv = dev_alloc(sizeof(float) * ROWS * D);
  float* d_out = dev_alloc(sizeof(float) * ROWS * D);
  uint32_t* d_past = dev_alloc(sizeof past);
  if (failures) return 1;

  /* Quantize K, then V, of every slot (int8_kv_ops.rs:11-29), bit-exact against the oracle. */
  PpkQuantizeArgs qa;
  memset(&qa, 0, sizeof qa);
  qa.struct_size = sizeof qa;
  qa.src_dtype = PPK_F32;
  qa.src = d_src;
  qa.rows = hist_rows;
  qa.head_dim = D;
  float* srcs[2] = {hist_k, hist_v};
  uint8_t* d_codes[2] = {d_kc, d_vc};
  float* d_scales[2] = {d_ks, d_vs};
  uint8_t* codes[2] = {kc, vc};
  float* scales[2] = {ks, vs};
  for (int t = 0; t < 2; ++t) {
    qa.codes = d_codes[t];
    qa.scales = d_scales[t];
    if (!hip_ok(hipMemcpy(d_src, srcs[t], sizeof(float) * hist_rows * D, hipMemcpyHostToDevice), "copy src") ||
        !ppk_ok(ppk_quantize(ctx, NULL, &qa), "ppk_quantize") || !hip_ok(hipDeviceSynchronize(), "sync") ||
        !hip_ok(hipMemcpy(codes[t], d_codes[t], hist_rows * D, hipMemcpyDeviceToHost), "copy codes") ||
        !hip_ok(hipMemcpy(scales[t], d_scales[t], sizeof(float) * hist_rows, hipMemcpyDeviceToHost), "copy scales"))
      return 1;
    oracle_quantize(srcs[t], hist_rows, D, okc, oks);
    check(memcmp(codes[t], okc, hist_rows * D) == 0 && memcmp(scales[t], oks, sizeof(float) * hist_rows) == 0,
          t == 0 ? "ppk_quantize K: codes and scales bit-exact against the oracle"
                 : "ppk_quantize V: codes and scales bit-exact against the oracle");
  }

  /* Attention over the ragged history plus the current token (int8_kv_ops.rs:41-55). */
  if (!hip_ok(hipMemcpy(d_q, q, sizeof(float) * ROWS * D, hipMemcpyHostToDevice), "copy q") ||
      !hip_ok(hipMemcpy(d_sk, sk, sizeof(float) * ROWS * D, hipMemcpyHostToDevice), "copy sk") ||
      !hip_ok(hipMemcpy(d_sv, sv, sizeof(float) * ROWS * D, hipMemcpyHostToDevice), "copy sv") ||
      !hip_ok(hipMemcpy(d_past, past, sizeof past, hipMemcpyHostToDevice), "copy past"))
    return 1;
  oracle_attention(q, kc, vc, ks, vs, sk, sv, past, ROWS, H, CAP, D, 1.0f / sqrtf((float)D), 0, ref);
  PpkAttentionArgs aa;
  memset(&aa, 0, sizeof aa);
  aa.struct_size = sizeof aa;
  aa.q_dtype = aa.scratch_dtype = aa.out_dtype = PPK_F32;
  aa.rows = ROWS;
  aa.heads = H;
  aa.capacity = CAP;
  aa.head_dim = D;
  aa.q = d_q;
  aa.k_codes = d_kc;
  aa.v_codes = d_vc;
  aa.k_scales = d_ks;
  aa.v_scales = d_vs;
  aa.sk = d_sk;
  aa.sv = d_sv;
  aa.past = d_past;
  aa.out = d_out;
  attend(ctx, &aa, 0, ref, out, "ppk_decode_attention, library plan");
  attend(ctx, &aa, 8, ref, out, "ppk_decode_attention, 8-token splits (merge kernel)");
  aa.past_host = past;
  attend(ctx, &aa, 0, ref, out, "ppk_decode_attention, host lengths");

  /* A refused call: status 1 and an error text, before anything is enqueued. */
  PpkAttentionArgs bad = aa;
  bad.head_dim = 100;
  const int32_t st = ppk_decode_attention(ctx, NULL, &bad);
  check(st == 1 && strlen(ppk_last_error()) > 0, "head_dim 100 refused with status 1 and an error text");

  /* Dequantize the K codes back to f32 (int8_kv_ops.rs:30-40), bit-exact against the oracle. */
  PpkDequantizeArgs da;
  memset(&da, 0, sizeof da);
  da.struct_size = sizeof da;
  da.out_dtype = PPK_F32;
  da.codes = d_kc;
  da.scales = d_ks;
  da.out = d_src;
  da.rows = hist_rows;
  da.head_dim = D;
  if (ppk_ok(ppk_dequantize(ctx, NULL, &da), "ppk_dequantize") && hip_ok(hipDeviceSynchronize(), "sync") &&
      hip_ok(hipMemcpy(hist_v, d_src, sizeof(float) * hist_rows * D, hipMemcpyDeviceToHost), "copy dq")) {
    oracle_dequantize(kc, ks, hist_rows, D, 0, hist_k);
    check(memcmp(hist_v, hist_k, sizeof(float) * hist_rows * D) == 0,
          "ppk_dequantize to f32 bit-exact against the oracle");
  }

  /* The fused decode step (commit of the current token at slot past[b], then attention; the callers'
     commit + attend, app/src/model/mod.rs:699-705): the output is the attention above (the committed
     slot lies past every history), the committed codes and scales are the oracle's of the token. */
  uint32_t* d_flags = dev_alloc(sizeof(uint32_t));
  if (d_flags && hip_ok(hipMemset(d_flags, 0, sizeof(uint32_t)), "clear flags")) {
    PpkDecodeStepArgs sa;
    memset(&sa, 0, sizeof sa);
    sa.struct_size = sizeof sa;
    sa.new_dtype = PPK_F32;
    sa.k_new = d_sk;
    sa.v_new = d_sv;
    sa.flags = d_flags;
    sa.attn = aa;
    sa.attn.past_host = NULL;
    uint32_t split = 0, nsplits = 0;
    uint64_t ws = 0;
    void* workspace = NULL;
    if (ppk_ok(ppk_attention_plan(ctx, &sa.attn, &split, &nsplits, &ws), "plan") &&
        (!ws || (workspace = dev_alloc(ws)) != NULL)) {
      sa.attn.workspace = workspace;
      sa.attn.workspace_bytes = ws;
      uint32_t flags = ~0u;
      if (ppk_ok(ppk_decode_step(ctx, NULL, &sa), "ppk_decode_step") && hip_ok(hipDeviceSynchronize(), "sync") &&
          hip_ok(hipMemcpy(out, d_out, sizeof(float) * ROWS * D, hipMemcpyDeviceToHost), "copy out") &&
          hip_ok(hipMemcpy(kc, d_kc, hist_rows * D, hipMemcpyDeviceToHost), "copy codes") &&
          hip_ok(hipMemcpy(ks, d_ks, sizeof(float) * hist_rows, hipMemcpyDeviceToHost), "copy scales") &&
          hip_ok(hipMemcpy(&flags, d_flags, sizeof flags, hipMemcpyDeviceToHost), "copy flags")) {
        double max_abs = 0.0;
        for (size_t i = 0; i < (size_t)ROWS * D; ++i) {
          const double err = fabs((double)out[i] - ref[i]);
          if (!(err <= max_abs)) max_abs = err; /* NaN propagates */
        }
        int committed = 1;
        for (size_t r = 0; r < ROWS; ++r) {
          const size_t slot = r * CAP + past[r / H];
          oracle_quantize(sk + r * D, 1, D, okc, oks);
          committed = committed && memcmp(kc + slot * D, okc, D) == 0 && ks[slot] == oks[0];
        }
        char line[160];
        snprintf(line, sizeof line, "ppk_decode_step: output max abs %.3e, committed K bit-exact %s, flags %u",
                 max_abs, committed ? "yes" : "no", flags);
        check(max_abs <= 2e-3 && committed && flags == 0, line);
      }
    }
    if (workspace) hipFree(workspace);
  }
  if (d_flags) hipFree(d_flags);

  hipFree(d_src);
  hipFree(d_kc);
  hipFree(d_vc);
  hipFree(d_ks);
  hipFree(d_vs);
  hipFree(d_q);
  hipFree(d_sk);
  hipFree(d_sv);
  hipFree(d_out);
  hipFree(d_past);
  check(ppk_context_release(ctx) == 0, "ppk_context_release");
  free(hist_k);
  free(hist_v);
  free(q);
  free(sk);
  free(sv);
  free(kc);
  free(vc);
  free(ks);
  free(vs);
  free(okc);
  free(oks);
  free(ref);
  free(out);
  printf("%s\n", failures ? "c consumer FAILED" : "c consumer ok");
  return failures ? 1 : 0;
}
