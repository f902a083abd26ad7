/*
 * CPU baselines timed by bench.py (not the oracle; test infrastructure):
 * the reference's Candle CPU decode, restated op for op in f32 and built
 * to run the way Candle's CPU backend does: the matrix products as SIMD
 * fused multiply-adds (Candle calls the `gemm` crate 0.19, which picks
 * AVX2/FMA kernels at run time: vendor/candle-core/src/cpu_backend/mod.rs:1380-1450),
 * the elementwise passes vectorised, rows shared out over every host core
 * by a pool of threads kept between calls (Candle's Rayon pool,
 * vendor/candle-core/src/utils.rs:327-346).
 *
 * The hot loops are written once and compiled twice, for AVX2 + FMA and for
 * the baseline x86-64 instruction set; the AVX2 form is taken when the CPU
 * has it (every EPYC host of an MI355X does). Dot products keep eight
 * independent partial sums (the vector lanes), so the compiler vectorises
 * them without reassociating anything itself.
 *
 * int8 history (cpu_baseline_decode; app/src/model/mod.rs:716-720,
 * batch.rs:211-222): per (b, h) row
 *   1. dequantize history K and V to dense f32 (int8_kv_ops.rs:33-35) and
 *      append the current token (cache.rs query_int8_prefill :133-141);
 *   2. scores = q . K^T (gemm);  3. scores *= 1/sqrt(d) (affine, cpu_backend/mod.rs:311-317);
 *   4. softmax_last_dim: max, exp(x - max), sum, divide (candle-nn 0.11);
 *   5. out = probs . V (gemm).
 * float history (cpu_baseline_float_decode; batch.rs:211-222): K, V
 * widened to f32 (to_dtype), then 2-5 over all `size` tokens of the row.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  const float* q;
  const uint8_t *k, *v;
  const float *ks, *vs, *sk, *sv;
  const uint32_t* past;
  size_t heads, capacity, d;
  float scale;
  float* out;
  size_t row_begin, row_end;
  int avx2;
} Int8Job;

typedef struct {
  const float* q;
  const void *k, *v;
  int kv_bf16;
  size_t size, d;
  float scale;
  float* out;
  size_t row_begin, row_end;
  int avx2;
} FloatJob;

/* ---- the vectorised steps, one body, two instruction sets -------------- */

#define DEQUANT_BODY                                                        \
  {                                                                         \
    for (size_t t = 0; t < n; ++t) {                                        \
      const float s = scales[t];                                            \
      const uint8_t* c = codes + t * d;                                     \
      float* o = out + t * d;                                               \
      for (size_t i = 0; i < d; ++i) o[i] = (float)(int8_t)c[i] * s;        \
    }                                                                       \
  }

#define WIDEN_BODY                                                          \
  {                                                                         \
    if (!bf16) {                                                            \
      memcpy(out, src, count * sizeof(float));                              \
    } else {                                                                \
      const uint16_t* h = (const uint16_t*)src;                             \
      uint32_t* o = (uint32_t*)out;                                         \
      for (size_t e = 0; e < count; ++e) o[e] = (uint32_t)h[e] << 16;       \
    }                                                                       \
  }

/* scores[t] = <q, K[t]> for t < n, eight partial sums per row of K. */
#define SCORES_BODY                                                         \
  {                                                                         \
    for (size_t t = 0; t < n; ++t) {                                        \
      const float* kr = kd + t * d;                                         \
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};                              \
      size_t i = 0;                                                         \
      for (; i + 8 <= d; i += 8)                                            \
        for (int l = 0; l < 8; ++l) acc[l] += q[i + l] * kr[i + l];         \
      float s = 0.0f;                                                       \
      for (; i < d; ++i) s += q[i] * kr[i];                                 \
      for (int l = 0; l < 8; ++l) s += acc[l];                              \
      sc[t] = s;                                                            \
    }                                                                       \
  }

/* affine, softmax_last_dim (max, exp, sum, divide) and probs . V. */
#define SOFTMAX_PV_BODY                                                     \
  {                                                                         \
    for (size_t t = 0; t < n; ++t) sc[t] = sc[t] * scale;                   \
    float mx = -INFINITY;                                                   \
    for (size_t t = 0; t < n; ++t) mx = sc[t] > mx ? sc[t] : mx;            \
    float z = 0.0f;                                                         \
    for (size_t t = 0; t < n; ++t) {                                        \
      sc[t] = expf(sc[t] - mx);                                             \
      z += sc[t];                                                           \
    }                                                                       \
    for (size_t t = 0; t < n; ++t) sc[t] = sc[t] / z;                       \
    for (size_t i = 0; i < d; ++i) o[i] = 0.0f;                             \
    for (size_t t = 0; t < n; ++t) {                                        \
      const float w = sc[t];                                                \
      const float* vr = vd + t * d;                                         \
      for (size_t i = 0; i < d; ++i) o[i] += w * vr[i];                     \
    }                                                                       \
  }

#define DEFINE_STEPS(SUFFIX, ATTR)                                                                      \
  ATTR static void dequant_##SUFFIX(const uint8_t* codes, const float* scales, size_t n, size_t d,   \
                                    float* out) DEQUANT_BODY                                         \
  ATTR static void widen_##SUFFIX(const void* src, int bf16, size_t count, float* out) WIDEN_BODY    \
  ATTR static void scores_##SUFFIX(const float* q, const float* kd, size_t n, size_t d, float* sc)     \
      SCORES_BODY                                                                                      \
  ATTR static void softmax_pv_##SUFFIX(float* sc, const float* vd, size_t n, size_t d, float scale,    \
                                       float* o) SOFTMAX_PV_BODY

DEFINE_STEPS(avx2, __attribute__((target("avx2,fma"))))
DEFINE_STEPS(plain, )

static int have_avx2(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* ---- a persistent worker pool (Rayon keeps its threads between calls) ----
   run_jobs(fn, jobs, size, n): job 0 and any job beyond the pool's workers
   run on the calling thread, job i (1 <= i <= workers) on worker i - 1;
   returns once every job has finished. Workers are created on first need
   and then wait for the next call. Calls are serialised by the pool. */

#define POOL_MAX 256
static pthread_mutex_t g_call = PTHREAD_MUTEX_INITIALIZER;  /* one call at a time */
static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t g_go = PTHREAD_COND_INITIALIZER;
static pthread_cond_t g_done = PTHREAD_COND_INITIALIZER;
static size_t g_workers = 0;
static unsigned long g_gen = 0;
static void* (*g_fn)(void*);
static char* g_jobs;
static size_t g_size, g_njobs, g_left;

static void* pool_worker(void* arg) {
  const size_t id = (size_t)(uintptr_t)arg; /* runs job id + 1 */
  unsigned long seen = 0;
  pthread_mutex_lock(&g_mu);
  for (;;) {
    while (g_gen == seen) pthread_cond_wait(&g_go, &g_mu);
    seen = g_gen;
    if (id + 1 < g_njobs) {
      void* (*fn)(void*) = g_fn;
      void* job = g_jobs + (id + 1) * g_size;
      pthread_mutex_unlock(&g_mu);
      fn(job);
      pthread_mutex_lock(&g_mu);
      if (--g_left == 0) pthread_cond_signal(&g_done);
    }
  }
  return NULL;
}

/* Returns 0, or -1 if a worker could not be started (its jobs then ran on the calling thread). */
static int run_jobs(void* (*fn)(void*), void* jobs, size_t size, size_t njobs) {
  int rc = 0;
  pthread_mutex_lock(&g_call);
  pthread_mutex_lock(&g_mu);
  while (g_workers + 1 < njobs && g_workers < POOL_MAX) {
    pthread_t t;
    if (pthread_create(&t, NULL, pool_worker, (void*)(uintptr_t)g_workers) != 0) {
      rc = -1;
      break;
    }
    pthread_detach(t);
    ++g_workers;
  }
  const size_t pooled = njobs - 1 < g_workers ? njobs - 1 : g_workers; /* jobs 1 .. pooled */
  g_fn = fn;
  g_jobs = (char*)jobs;
  g_size = size;
  g_njobs = pooled + 1;
  g_left = pooled;
  ++g_gen;
  pthread_cond_broadcast(&g_go);
  pthread_mutex_unlock(&g_mu);
  fn(jobs);
  for (size_t i = pooled + 1; i < njobs; ++i) fn((char*)jobs + i * size);
  pthread_mutex_lock(&g_mu);
  while (g_left > 0) pthread_cond_wait(&g_done, &g_mu);
  pthread_mutex_unlock(&g_mu);
  pthread_mutex_unlock(&g_call);
  return rc;
}

/* ---- int8 history --------------------------------------------------------- */

static void* int8_worker(void* arg) {
  const Int8Job* j = (const Int8Job*)arg;
  const size_t d = j->d;
  float *kd = NULL, *vd = NULL, *sc = NULL;
  size_t have = 0;
  for (size_t r = j->row_begin; r < j->row_end; ++r) {
    const uint32_t p = j->past[r / j->heads];
    float* o = j->out + r * d;
    if (p > j->capacity) {
      for (size_t i = 0; i < d; ++i) o[i] = NAN;
      continue;
    }
    const size_t n = (size_t)p + 1;
    if (have < n) {
      have = n;
      kd = (float*)realloc(kd, n * d * sizeof(float));
      vd = (float*)realloc(vd, n * d * sizeof(float));
      sc = (float*)realloc(sc, n * sizeof(float));
    }
    const uint8_t* kc = j->k + r * j->capacity * d;
    const uint8_t* vc = j->v + r * j->capacity * d;
    const float* ksr = j->ks + r * j->capacity;
    const float* vsr = j->vs + r * j->capacity;
    const float* qr = j->q + r * d;
    if (j->avx2) {
      dequant_avx2(kc, ksr, p, d, kd);
      dequant_avx2(vc, vsr, p, d, vd);
    } else {
      dequant_plain(kc, ksr, p, d, kd);
      dequant_plain(vc, vsr, p, d, vd);
    }
    memcpy(kd + (size_t)p * d, j->sk + r * d, d * sizeof(float));
    memcpy(vd + (size_t)p * d, j->sv + r * d, d * sizeof(float));
    if (j->avx2) {
      scores_avx2(qr, kd, n, d, sc);
      softmax_pv_avx2(sc, vd, n, d, j->scale, o);
    } else {
      scores_plain(qr, kd, n, d, sc);
      softmax_pv_plain(sc, vd, n, d, j->scale, o);
    }
  }
  free(kd);
  free(vd);
  free(sc);
  return NULL;
}

/* Runs the baseline over rows [0, rows) on `threads` threads (the caller's
   and threads - 1 pool workers), a contiguous range of rows each. Returns 0,
   or -1 if a worker could not start (its rows then ran on the calling thread). */
int cpu_baseline_decode(const float* q, const uint8_t* k, const uint8_t* v, const float* ks, const float* vs,
                        const float* sk, const float* sv, const uint32_t* past, size_t rows, size_t heads,
                        size_t capacity, size_t d, float scale, size_t threads, float* out) {
  if (threads < 1) threads = 1;
  if (threads > rows) threads = rows;
  const int avx2 = have_avx2();
  Int8Job* jobs = (Int8Job*)malloc(threads * sizeof(Int8Job));
  for (size_t t = 0; t < threads; ++t) {
    Int8Job jb = {q, k, v, ks, vs, sk, sv, past, heads, capacity, d, scale, out,
                  rows * t / threads, rows * (t + 1) / threads, avx2};
    jobs[t] = jb;
  }
  const int rc = run_jobs(int8_worker, jobs, sizeof(Int8Job), threads);
  free(jobs);
  return rc;
}

/* Which instruction set the baseline runs with on this host: 1 = AVX2 + FMA. */
int cpu_baseline_uses_avx2(void) { return have_avx2(); }

/* ---- float history -------------------------------------------------------- */

static void* float_worker(void* arg) {
  const FloatJob* j = (const FloatJob*)arg;
  const size_t n = j->size, d = j->d;
  const size_t eb = j->kv_bf16 ? 2 : 4;
  float* kd = (float*)malloc(n * d * sizeof(float));
  float* vd = (float*)malloc(n * d * sizeof(float));
  float* sc = (float*)malloc((n ? n : 1) * sizeof(float));
  for (size_t r = j->row_begin; r < j->row_end; ++r) {
    const char* kr = (const char*)j->k + r * n * d * eb;
    const char* vr = (const char*)j->v + r * n * d * eb;
    float* o = j->out + r * d;
    if (j->avx2) {
      widen_avx2(kr, j->kv_bf16, n * d, kd);
      widen_avx2(vr, j->kv_bf16, n * d, vd);
      scores_avx2(j->q + r * d, kd, n, d, sc);
      softmax_pv_avx2(sc, vd, n, d, j->scale, o);
    } else {
      widen_plain(kr, j->kv_bf16, n * d, kd);
      widen_plain(vr, j->kv_bf16, n * d, vd);
      scores_plain(j->q + r * d, kd, n, d, sc);
      softmax_pv_plain(sc, vd, n, d, j->scale, o);
    }
  }
  free(kd);
  free(vd);
  free(sc);
  return NULL;
}

int cpu_baseline_float_decode(const float* q, const void* k, const void* v, int kv_bf16, size_t rows, size_t size,
                              size_t d, float scale, size_t threads, float* out) {
  if (threads < 1) threads = 1;
  if (threads > rows) threads = rows;
  const int avx2 = have_avx2();
  FloatJob* jobs = (FloatJob*)malloc(threads * sizeof(FloatJob));
  for (size_t t = 0; t < threads; ++t) {
    FloatJob jb = {q, k, v, kv_bf16, size, d, scale, out, rows * t / threads, rows * (t + 1) / threads, avx2};
    jobs[t] = jb;
  }
  const int rc = run_jobs(float_worker, jobs, sizeof(FloatJob), threads);
  free(jobs);
  return rc;
}
