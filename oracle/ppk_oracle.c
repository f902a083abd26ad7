/*
 * ppk_oracle.c -- CPU restatement of the reference's int8 KV decode path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline), never as the product path.
 *
 * Each function names the reference lines it restates. The reference
 * (Rust/Candle + NVRTC CUDA + Windows HIPRTC) cannot be compiled in this
 * image, so this restatement is pinned by closed forms, an independent numpy
 * restatement and the reference's own known-answer checks (tests/).
 *
 * Built with: gcc -O2 -fno-fast-math -ffp-contract=off (oracle/build.py),
 * so every float operation is the single IEEE-754 binary32 operation written.
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* bf16 round-to-nearest-even of an f32, kept in f32 (Candle's to_dtype(BF16),
   i.e. half::bf16::from_f32, and pp_round_bf16, app/src/model/int8_kv.cu:3-7). */
static float round_bf16(float x) {
  if (x != x) return x;
  uint32_t u;
  memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&x, &u, 4);
  return x;
}

/*
 * quantize, app/src/model/int8_kv_ops.rs:11-21 (CPU branch), one row of d
 * channels at a time:
 *   s = (max_i |x_i| / 127).max(1e-12)            -- :17, f32::max ignores NaN
 *   code_i = (x_i / s).round_ties_even().clamp(-127, 127) as i8 as u8   -- :18
 * Rust's `as i8` maps NaN to 0 (f32::clamp keeps NaN); the CUDA path does the
 * same through __float2int_rn (int8_kv.cu:17). The CPU branch rejects
 * non-finite rows first (:16); nonfinite_rows counts them instead so callers
 * can assert the same condition. Returns the number of non-finite rows.
 */
size_t oracle_quantize(const float* x, size_t rows, size_t d, uint8_t* codes, float* scales) {
  size_t bad = 0;
  for (size_t r = 0; r < rows; ++r) {
    const float* row = x + r * d;
    float amax = 0.0f;
    int finite = 1;
    for (size_t i = 0; i < d; ++i) {
      /* f32::max skips a NaN argument of either kind; glibc's fmaxf returns
       * NaN for a signalling one, so the fold is written as a comparison. */
      const float a = fabsf(row[i]);
      if (a > amax) amax = a;
      if (!isfinite(row[i])) finite = 0;
    }
    bad += finite ? 0 : 1;
    const float s = fmaxf(amax / 127.0f, 1e-12f);
    scales[r] = s;
    for (size_t i = 0; i < d; ++i) {
      float q = rintf(row[i] / s); /* default rounding mode: ties to even */
      int code;
      if (q != q) code = 0;
      else code = (int)fminf(fmaxf(q, -127.0f), 127.0f);
      codes[r * d + i] = (uint8_t)(int8_t)code;
    }
  }
  return bad;
}

/*
 * dequantize, int8_kv_ops.rs:33-35 (CPU branch) / pp_i8_unpack int8_kv.cu:19-22:
 *   y = (code as i8) as f32 * s[row]   (one f32 multiply)
 * round_bf16 != 0 applies Candle's .to_dtype(BF16) (int8_kv_ops.rs:35,68).
 */
void oracle_dequantize(const uint8_t* codes, const float* scales, size_t rows, size_t d, int round,
                       float* out) {
  for (size_t r = 0; r < rows; ++r)
    for (size_t i = 0; i < d; ++i) {
      const float y = (float)(int8_t)codes[r * d + i] * scales[r];
      out[r * d + i] = round ? round_bf16(y) : y;
    }
}

/*
 * append placement, Int8LayerCache::query_batch commit path
 * (app/src/model/int8_cache.rs:326-359) through LayerCache slot placement
 * (app/src/model/cache.rs:301-478): the new tokens of sequence b are
 * quantized (a1) and land at slots past[b] .. past[b]+tokens-1 of every head
 * row bh = b*heads + h of the [B*H, capacity, d] arenas; nothing else changes.
 * Rows whose slots would pass capacity are skipped (the reference refuses the
 * whole call on the host before writing, cache.rs:221-223). Returns the
 * number of skipped (row, token) pairs.
 */
size_t oracle_append(const float* src, size_t batch, size_t heads, size_t tokens, size_t d, const uint32_t* past,
                     size_t capacity, uint8_t* codes, float* scales) {
  size_t skipped = 0;
  uint8_t* tmp = (uint8_t*)malloc(d);
  for (size_t b = 0; b < batch; ++b)
    for (size_t h = 0; h < heads; ++h)
      for (size_t t = 0; t < tokens; ++t) {
        const size_t bh = b * heads + h;
        const uint64_t slot = (uint64_t)past[b] + t;
        if (slot >= capacity) {
          ++skipped;
          continue;
        }
        float s;
        oracle_quantize(src + (bh * tokens + t) * d, 1, d, tmp, &s);
        memcpy(codes + (bh * capacity + slot) * d, tmp, d);
        scales[bh * capacity + slot] = s;
      }
  free(tmp);
  return skipped;
}

/*
 * Decode attention, the semantics of int8_kv_ops::attention
 * (int8_kv_ops.rs:41-55) as computed by pp_i8_attention + pp_i8_merge
 * (int8_kv.cu:28-59) and checked by the host formula of int8_kv_ops.rs:69-73,
 * 94-98, accumulated in f64:
 *   row r, sequence b = r / heads, p = past[b]
 *   K_t = dequant(k[r, t]) for t < p,  K_p = sk[r]  (current token unquantized, :36-37)
 *   V_t likewise with sv[r]                         (:49)
 *   s_t = scale * <q_r, K_t>;  out_r = sum_t e^{s_t - max s} V_t / sum_t e^{s_t - max s}
 * dequant is the f32 product code * scale (history_bf16 = 0; Candle's CPU
 * dequantize to F32) or its bf16 rounding (history_bf16 = 1; pp_i8_load,
 * int8_kv.cu:23-27). p > capacity yields NaN (:33,51,58).
 */
typedef struct {
  const float *q, *ks, *vs, *sk, *sv;
  const uint8_t *k, *v;
  const uint32_t* past;
  size_t r0, r1, heads, capacity, d;
  float scale;
  int history_bf16;
  double* out;
} AttentionJob;

static void attention_rows(const AttentionJob* j) {
  const size_t capacity = j->capacity, d = j->d;
  double* scores = NULL;
  size_t cap_scores = 0;
  for (size_t r = j->r0; r < j->r1; ++r) {
    const uint32_t p = j->past[r / j->heads];
    double* o = j->out + r * d;
    if (p > capacity) {
      for (size_t i = 0; i < d; ++i) o[i] = NAN;
      continue;
    }
    if (cap_scores < (size_t)p + 1) {
      cap_scores = (size_t)p + 1;
      scores = (double*)realloc(scores, cap_scores * sizeof(double));
    }
    const float* qr = j->q + r * d;
    double mx = -INFINITY;
    for (size_t t = 0; t <= p; ++t) {
      double acc = 0.0;
      for (size_t i = 0; i < d; ++i) {
        float kv;
        if (t == p) kv = j->sk[r * d + i];
        else {
          kv = (float)(int8_t)j->k[(r * capacity + t) * d + i] * j->ks[r * capacity + t];
          if (j->history_bf16) kv = round_bf16(kv);
        }
        acc += (double)qr[i] * (double)kv;
      }
      scores[t] = acc * (double)j->scale;
      if (scores[t] > mx) mx = scores[t];
    }
    double z = 0.0;
    for (size_t t = 0; t <= p; ++t) {
      scores[t] = exp(scores[t] - mx);
      z += scores[t];
    }
    for (size_t i = 0; i < d; ++i) o[i] = 0.0;
    for (size_t t = 0; t <= p; ++t) {
      const double w = scores[t];
      for (size_t i = 0; i < d; ++i) {
        float vv;
        if (t == p) vv = j->sv[r * d + i];
        else {
          vv = (float)(int8_t)j->v[(r * capacity + t) * d + i] * j->vs[r * capacity + t];
          if (j->history_bf16) vv = round_bf16(vv);
        }
        o[i] += w * (double)vv;
      }
    }
    for (size_t i = 0; i < d; ++i) o[i] /= z;
  }
  free(scores);
}

static void* attention_worker(void* job) {
  attention_rows((const AttentionJob*)job);
  return NULL;
}

/* The same computation with the rows shared out over `threads` POSIX threads
   (contiguous row ranges, each row computed exactly as above, so the result
   does not depend on the thread count). Returns 0, or -1 if a thread could
   not be started (its rows were then computed on the calling thread). */
int oracle_attention_mt(const float* q, const uint8_t* k, const uint8_t* v, const float* ks, const float* vs,
                        const float* sk, const float* sv, const uint32_t* past, size_t rows, size_t heads,
                        size_t capacity, size_t d, float scale, int history_bf16, size_t threads, double* out) {
  if (threads < 1) threads = 1;
  if (threads > rows) threads = rows ? rows : 1;
  AttentionJob* jobs = (AttentionJob*)malloc(threads * sizeof(AttentionJob));
  pthread_t* tid = (pthread_t*)malloc(threads * sizeof(pthread_t));
  int* started = (int*)calloc(threads, sizeof(int));
  int rc = 0;
  for (size_t t = 0; t < threads; ++t) {
    AttentionJob j = {q, ks, vs, sk, sv, k, v, past, rows * t / threads, rows * (t + 1) / threads,
                      heads, capacity, d, scale, history_bf16, out};
    jobs[t] = j;
    if (t + 1 < threads && pthread_create(&tid[t], NULL, attention_worker, &jobs[t]) == 0) started[t] = 1;
  }
  for (size_t t = 0; t < threads; ++t) {
    if (started[t]) continue;
    if (t + 1 < threads) rc = -1;
    attention_rows(&jobs[t]);
  }
  for (size_t t = 0; t < threads; ++t)
    if (started[t]) pthread_join(tid[t], NULL);
  free(started);
  free(tid);
  free(jobs);
  return rc;
}

void oracle_attention(const float* q, const uint8_t* k, const uint8_t* v, const float* ks, const float* vs,
                      const float* sk, const float* sv, const uint32_t* past, size_t rows, size_t heads,
                      size_t capacity, size_t d, float scale, int history_bf16, double* out) {
  AttentionJob j = {q, ks, vs, sk, sv, k, v, past, 0, rows, heads, capacity, d, scale, history_bf16, out};
  attention_rows(&j);
}

/*
 * The reference kernel's own f32 split-K arithmetic, restated operation by
 * operation (int8_kv.cu:28-59 generalised from 64 channels to d and from the
 * 0.125 constant to `scale`): partitions of `split` tokens over [0, capacity]
 * (cuda::Attention launches ceil((capacity+1)/split), int8_kv_ops.rs:153);
 * per partition the local max m, z = sum e^{s-m} (expf), y_d = sum e^{s-m} v_d,
 * bf16-rounded history (pp_i8_load); merge M = max m, out = sum e^{m-M} y / sum
 * e^{m-M} z, NaN when the denominator is not positive or p > capacity.
 * Summation order differs from the device's (a tree of shuffles); results
 * agree with the f64 oracle to the reference's own 2e-5 check tolerance.
 */
void oracle_attention_splitk_reference(const float* q, const uint8_t* k, const uint8_t* v, const float* ks,
                                       const float* vs, const float* sk, const float* sv, const uint32_t* past,
                                       size_t rows, size_t heads, size_t capacity, size_t d, float scale,
                                       size_t split, float* out) {
  const size_t splits = (capacity + 1 + split - 1) / split;
  float* part = (float*)malloc(splits * (d + 2) * sizeof(float));
  float* sc = (float*)malloc(split * sizeof(float));
  for (size_t r = 0; r < rows; ++r) {
    const uint32_t p = past[r / heads];
    const int valid = p <= capacity;
    const size_t length = (size_t)p + 1;
    for (size_t part_i = 0; part_i < splits; ++part_i) {
      const size_t begin = part_i * split;
      const size_t end = valid ? (begin + split < length ? begin + split : length) : 0;
      float m = -3.402823466e38f;
      for (size_t t = 0; t < split; ++t) {
        const size_t at = begin + t;
        float s = -3.402823466e38f;
        if (at < end) {
          float dot = 0.0f;
          for (size_t i = 0; i < d; ++i) {
            const float kv = at == p ? sk[r * d + i]
                                     : round_bf16((float)(int8_t)k[(r * capacity + at) * d + i] * ks[r * capacity + at]);
            dot += q[r * d + i] * kv;
          }
          s = dot * scale;
        }
        sc[t] = s;
        m = fmaxf(m, s);
      }
      float z = 0.0f;
      for (size_t t = 0; t < split; ++t) {
        const float e = begin + t < end ? expf(sc[t] - m) : 0.0f;
        sc[t] = e;
        z += e;
      }
      float* rec = part + part_i * (d + 2);
      rec[0] = m;
      rec[1] = z;
      for (size_t i = 0; i < d; ++i) {
        float sum = 0.0f;
        for (size_t at = begin; at < end; ++at) {
          const float value = at == p ? sv[r * d + i]
                                      : round_bf16((float)(int8_t)v[(r * capacity + at) * d + i] * vs[r * capacity + at]);
          sum += sc[at - begin] * value;
        }
        rec[2 + i] = valid ? sum : NAN;
      }
    }
    float M = -3.402823466e38f;
    for (size_t s = 0; s < splits; ++s) M = fmaxf(M, part[s * (d + 2)]);
    for (size_t i = 0; i < d; ++i) {
      float z = 0.0f, y = 0.0f;
      for (size_t s = 0; s < splits; ++s) {
        const float w = expf(part[s * (d + 2)] - M);
        z += part[s * (d + 2) + 1] * w;
        y += part[s * (d + 2) + 2 + i] * w;
      }
      out[r * d + i] = z > 0.0f ? y / z : NAN;
    }
  }
  free(part);
  free(sc);
}

/*
 * Float-KV decode attention, the semantics of fused_attention::decode_attention
 * (app/src/model/fused_attention.rs:8-30) as computed by pp_attention_part and
 * pp_attention_merge (app/src/model/decode_attention.hip:9-66), in f64:
 *   row r, sequence b = r / heads; n = lengths ? lengths[b] : size
 *   (n counts every attended token; the current one is already in the cache)
 *   s_t = scale * <q_r, K_r[t]>, t < n;  out_r = sum_t e^{s_t - max} V_r[t] / sum_t e^{s_t - max}
 *   n == 0 or n > size yields NaN (decode_attention.hip:15,50).
 * K/V elements are bf16 (kv_bf16 = 1, raw 16-bit patterns) or f32; rows are
 * k_row_stride / v_row_stride elements apart, tokens d elements apart.
 */
void oracle_attention_float(const float* q, const void* k, const void* v, int kv_bf16, size_t k_row_stride,
                            size_t v_row_stride, const uint32_t* lengths, size_t rows, size_t heads, size_t size,
                            size_t d, float scale, double* out) {
  double* scores = (double*)malloc((size ? size : 1) * sizeof(double));
  for (size_t r = 0; r < rows; ++r) {
    const size_t n = lengths ? lengths[r / heads] : size;
    double* o = out + r * d;
    if (n == 0 || n > size) {
      for (size_t i = 0; i < d; ++i) o[i] = NAN;
      continue;
    }
    double mx = -INFINITY;
    for (size_t t = 0; t < n; ++t) {
      double acc = 0.0;
      for (size_t i = 0; i < d; ++i) {
        const size_t at = r * k_row_stride + t * d + i;
        float kv;
        if (kv_bf16) {
          const uint32_t bits = (uint32_t)((const uint16_t*)k)[at] << 16;
          memcpy(&kv, &bits, 4);
        } else {
          kv = ((const float*)k)[at];
        }
        acc += (double)q[r * d + i] * (double)kv;
      }
      scores[t] = acc * (double)scale;
      if (scores[t] > mx) mx = scores[t];
    }
    double z = 0.0;
    for (size_t t = 0; t < n; ++t) {
      scores[t] = exp(scores[t] - mx);
      z += scores[t];
    }
    for (size_t i = 0; i < d; ++i) o[i] = 0.0;
    for (size_t t = 0; t < n; ++t)
      for (size_t i = 0; i < d; ++i) {
        const size_t at = r * v_row_stride + t * d + i;
        float vv;
        if (kv_bf16) {
          const uint32_t bits = (uint32_t)((const uint16_t*)v)[at] << 16;
          memcpy(&vv, &bits, 4);
        } else {
          vv = ((const float*)v)[at];
        }
        o[i] += scores[t] * (double)vv;
      }
    for (size_t i = 0; i < d; ++i) o[i] /= z;
  }
  free(scores);
}

/*
 * CFG + Renyi effective-support sampler, restating the reference's host
 * validation oracle (app/src/inference/hip_sampling_reference.rs:12-141) of
 * the kernel pp_hip_renyi_sample (app/src/inference/renyi_sample.hip:23-204):
 *   value_c = guidance == 2 ? u_c + cfg * (c_c - u_c) : c_c   (every column checked finite)
 *   legal candidates [start, start + count); m = max; 256 strided partial sums
 *   of exp(v - m) and exp(alpha (v - m)) reduced by the kernel's tree;
 *   H = log Z + max(0, log Z - log Z_alpha) / (alpha - 1), clamped to [0, ln count];
 *   support = clamp((u32)(exp(H) + 0.5), 1, count); rank = min((u32)(uniform * support), support - 1);
 *   token = offset + the rank-th candidate by (value descending, index ascending).
 * Invalid rows give (fallback token, valid 0, support 1). cfg_fma = 0 is the
 * reference's form: a separately rounded product and sum, as its host oracle
 * computes it (hip_sampling_reference.rs:73) and as its kernel is compiled
 * (-ffp-contract=off, app/src/model/hip_kernel.rs:46). cfg_fma = 1 gives
 * fmaf(cfg, c - u, u), a contracted form no reference build produces; tests
 * use it only to show that a case tells the two forms apart.
 * margin[row] (optional) = distance of exp(H) + 0.5 from the nearest integer:
 * libm and device exp/log may round a row with a tiny margin differently.
 * Returns 0, or -1 for metadata the reference rejects.
 */
static int oracle_before(float a, uint32_t ai, float b, uint32_t bi) { return a > b || (a == b && ai < bi); }

static float* g_sort_values;
static int oracle_order_cmp(const void* x, const void* y) {
  const uint32_t a = *(const uint32_t*)x, b = *(const uint32_t*)y;
  if (oracle_before(g_sort_values[a], a, g_sort_values[b], b)) return -1;
  if (oracle_before(g_sort_values[b], b, g_sort_values[a], a)) return 1;
  return 0;
}

int oracle_renyi_sample(const float* raw, size_t physical_rows, size_t choices, const float* uniforms,
                        const uint32_t* bounds, float alpha, float cfg, size_t guidance, uint32_t offset,
                        int cfg_fma, uint32_t* token, uint32_t* valid, uint32_t* support, float* margin) {
  if (!(guidance == 1 || guidance == 2) || physical_rows == 0 || physical_rows % guidance != 0 || choices < 1 ||
      choices > 2048 || !isfinite(alpha) || alpha <= 1.f || !isfinite(cfg) || cfg < 0.f ||
      (guidance == 1 && cfg != 1.f) || (uint64_t)offset + (choices - 1) > 0xffffffffull)
    return -1;
  const size_t batch = physical_rows / guidance;
  float* logits = (float*)malloc(choices * sizeof(float));
  uint32_t* order = (uint32_t*)malloc(choices * sizeof(uint32_t));
  for (size_t row = 0; row < batch; ++row) {
    const uint32_t start = bounds[2 * row], count = bounds[2 * row + 1];
    const float uniform = uniforms[row];
    token[row] = offset + (start < choices ? start : 0);
    valid[row] = 0;
    support[row] = 1;
    if (margin) margin[row] = INFINITY;
    if (!isfinite(uniform) || !(uniform >= 0.f && uniform < 1.f) || count == 0 || start >= choices ||
        count > choices - start)
      continue;
    const float* c = raw + row * guidance * choices;
    int finite = 1;
    for (size_t col = 0; col < choices; ++col) {
      float value = c[col];
      if (guidance == 2) {
        const float u = c[choices + col];
        finite &= isfinite(u);
        value = cfg_fma ? fmaf(cfg, c[col] - u, u) : u + cfg * (c[col] - u);
      }
      finite &= isfinite(c[col]) && isfinite(value);
      logits[col] = value;
    }
    if (!finite) continue;
    float maximum = -INFINITY;
    for (uint32_t i = start; i < start + count; ++i) maximum = fmaxf(maximum, logits[i]);
    float sums[256] = {0}, sums_alpha[256] = {0};
    for (size_t t = 0; t < 256; ++t)
      for (size_t k = t; k < count; k += 256) {
        const float shifted = logits[start + k] - maximum;
        sums[t] += expf(shifted);
        sums_alpha[t] += expf(alpha * shifted);
      }
    for (size_t step = 128; step > 0; step >>= 1)
      for (size_t t = 0; t < step; ++t) {
        sums[t] += sums[t + step];
        sums_alpha[t] += sums_alpha[t + step];
      }
    const float log_z = logf(sums[0]);
    const float log_za = logf(sums_alpha[0]);
    const float excess = log_z - log_za;
    float entropy = log_z + (excess > 0.f ? excess : 0.f) / (alpha - 1.f);
    if (!isfinite(log_z) || !isfinite(log_za) || !isfinite(entropy)) continue;
    const float hmax = logf((float)count);
    if (entropy < 0.f) entropy = 0.f;
    if (entropy > hmax) entropy = hmax;
    const float rounded = expf(entropy) + 0.5f;
    if (margin) margin[row] = fabsf(rounded - nearbyintf(rounded));
    uint32_t s = rounded >= 4294967295.f ? 0xffffffffu : (uint32_t)rounded;
    if (s < 1) s = 1;
    if (s > count) s = count;
    const float scaled = uniform * (float)s;
    uint32_t rank = (uint32_t)scaled;
    if (rank > s - 1) rank = s - 1;
    for (uint32_t i = 0; i < count; ++i) order[i] = start + i;
    g_sort_values = logits;
    qsort(order, count, sizeof(uint32_t), oracle_order_cmp);
    token[row] = offset + order[rank];
    valid[row] = 1;
    support[row] = s;
  }
  free(logits);
  free(order);
  return 0;
}
