// gfx950 (CDNA4) kernels of the int8 KV-cache decode path, written for
// 64-wide wavefronts. Built ahead of time into a code object
// (hipcc --genco --offload-arch=gfx950) and launched by ppk_abi.cpp.
//
//   ppk_quantize_d{64,128,256}         quantize rows densely or append into arenas
//   ppk_dequantize                     codes * scales -> f32/bf16/f16
//   ppk_decode[_bf16h]_d{..}           decode attention (+ fused append, + in-block merge), up to 8 waves per
//                                      block
//   ppk_attn_merge_d{..}               cross-group merge + current token
//   ppk_decode_flat[_bf16h]_d{..}      decode attention over a balanced work list (ragged batches, + fused append)
//   ppk_attn_merge_flat_d{..}          merge of the balanced work list's records + current token
//   ppk_fdecode_{bf16,f32}_d{..}       decode attention over float (bf16/f32) K/V
//   ppk_fmerge_d{..}                   cross-group merge of the float path
//   ppk_fdecode_flat_{bf16,f32}_d{..}  float-path decode over a balanced work list (ragged batches)
//   ppk_fstep[_flat]_{bf16,f32}_d{..}  the float path's fused step: write the current token, then attend
//   ppk_fmerge_flat_d{..}              merge of the float balanced work list's records
//   ppk_renyi_sample                   CFG + Renyi effective-support sampler
//   ppk_kv_scatter_u{16,4,2}           float-store append of token records into arena slots
//   ppk_copy2d_batch                   batched rectangle copies + zero fill (arena joins, growth, copy-on-write)
//
// Semantics follow app/src/model/int8_kv_ops.rs:11-40 and
// app/src/model/int8_kv.cu:8-59; the design (wave-per-row quantize, one-wave
// split blocks streaming 1 KiB per load, scale folding) is this file's own.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "ppk_kernel_args.h"

namespace {

#ifdef PPK_WAVE_CLOCK
// Wave-clock diagnostics build (ppk_kernels_clock.hsaco, -DPPK_WAVE_CLOCK):
// the real-time clock at fixed points of a wave, kept in scalar registers and
// appended as one record at the wave's end (layout in ppk_kernel_args.h). A
// point "after x" first makes the wave wait for x (an empty asm that reads
// it), then reads the clock.
#define PPK_CLK_DECL uint64_t clk_[ppk::kWaveClockPoints] = {0, 0, 0, 0, 0, 0, 0, 0}
#define PPK_CLK(i) (clk_[i] = __builtin_amdgcn_s_memrealtime())
#define PPK_CLK_AFTER(i, dep)           \
  do {                                  \
    __asm__ volatile("" ::"v"(dep));    \
    PPK_CLK(i);                         \
  } while (0)
#define PPK_CLK_AT(var, dep)            \
  do {                                  \
    __asm__ volatile("" ::"v"(dep));    \
    (var) = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define PPK_CLK_RECORD(args, kind, block, wave) \
  clock_record(args.clock, args.clock_seq, args.clock_cap, kind, block, wave, clk_)
// The buffer's own capacity word is honoured only up to the capacity the host
// derived from the buffer's size, so a wrong word cannot send a record past it.
__device__ __forceinline__ void clock_record(uint64_t* clock, uint32_t seq, uint32_t cap, uint32_t kind,
                                             uint32_t block, uint32_t wave,
                                             const uint64_t (&t)[ppk::kWaveClockPoints]) {
  if (!clock || (threadIdx.x & 63) != 0) return;
  const uint64_t per = clock[0], local = uint64_t(block) * (blockDim.x >> 6) + wave;
  const uint64_t slot = (uint64_t(seq) * 2 + kind - 1) * per + local;
  if (local >= per || slot >= clock[1] || slot >= cap) return;
  uint64_t* r = clock + ppk::kWaveClockWords * (slot + 1);
  const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);    // HW_ID
  const uint32_t xcc = __builtin_amdgcn_s_getreg((15 << 11) | 20);  // XCC_ID
  r[0] = (uint64_t(kind) << 56) | (uint64_t(seq) << 32) | (uint64_t(block) << 8) | wave;
  r[1] = (uint64_t(xcc) << 32) | hw;
#pragma unroll
  for (int i = 0; i < ppk::kWaveClockPoints; ++i) r[2 + i] = t[i];
}
#else
#define PPK_CLK_DECL
#define PPK_CLK(i)
#define PPK_CLK_AFTER(i, dep)
#define PPK_CLK_AT(var, dep)
#define PPK_CLK_RECORD(args, kind, block, wave)
#endif

using u2 = uint32_t __attribute__((ext_vector_type(2)));
using u4 = uint32_t __attribute__((ext_vector_type(4)));
using f4 = float __attribute__((ext_vector_type(4)));

enum { kF32 = 0, kBF16 = 1, kF16 = 2 };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

__device__ __forceinline__ float load_elem(const void* p, size_t i, uint32_t dtype) {
  if (dtype == kF32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  return dtype == kBF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

// N consecutive elements starting at element i, widened to f32: one dtype
// branch, then N independent loads in flight together.
template <int N>
__device__ __forceinline__ void load_vec(const void* p, size_t i, uint32_t dtype, float (&out)[N]) {
  if (dtype == kF32) {
    const float* f = static_cast<const float*>(p) + i;
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = f[e];
  } else {
    const uint16_t* h = static_cast<const uint16_t*>(p) + i;
    uint16_t b[N];
#pragma unroll
    for (int e = 0; e < N; ++e) b[e] = h[e];
    if (dtype == kBF16) {
#pragma unroll
      for (int e = 0; e < N; ++e) out[e] = bf16_to_f32(b[e]);
    } else {
#pragma unroll
      for (int e = 0; e < N; ++e) out[e] = f16_to_f32(b[e]);
    }
  }
}

// Round-to-nearest-even to bfloat16, returned as the 16 stored bits. NaN stays
// a quiet NaN (the carry trick alone could turn some NaN payloads into Inf).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  if (x != x) return 0x7fc0u;
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
// The same rounding kept in fp32 (the value a bf16 tensor would hold).
__device__ __forceinline__ float round_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}
// Two values rounded to bfloat16 (nearest even) by one v_cvt_pk_bf16_f32 and
// widened back to fp32: for finite inputs the bits of round_bf16 on each.
__device__ __forceinline__ void round_bf16_pair(float a, float b, float& ra, float& rb) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
  ra = __uint_as_float(u << 16);
  rb = __uint_as_float(u & 0xffff0000u);
}
// f32 -> f16, round to nearest even, from a materialised f32 value: the empty
// asm keeps the backend from folding a producing multiply into one fused
// multiply-to-f16 (v_fma_mixlo_f16), which rounds once where the reference
// semantics (an f32 product, then a conversion) round twice.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  __asm__("" : "+v"(x));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

__device__ __forceinline__ void store_elem(void* p, size_t i, uint32_t dtype, float x) {
  if (dtype == kF32) static_cast<float*>(p)[i] = x;
  else static_cast<uint16_t*>(p)[i] = dtype == kBF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
}

// Signed byte k of a dword as float; hipcc folds the sign-extension into an
// SDWA operand of v_cvt_f32_i32 (one VALU op per byte).
__device__ __forceinline__ float sbyte(uint32_t w, int k) { return float(int(int8_t(w >> (8 * k)))); }

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_xor1(float x) { return dpp_f32<0xB1>(x); }  // quad_perm [1,0,3,2]
__device__ __forceinline__ float dpp_xor2(float x) { return dpp_f32<0x4E>(x); }  // quad_perm [2,3,0,1]
__device__ __forceinline__ float dpp_half_mirror(float x) { return dpp_f32<0x141>(x); }
__device__ __forceinline__ float dpp_mirror(float x) { return dpp_f32<0x140>(x); }

// Sum over the LPT consecutive lanes that hold one token (LPT in {4, 8, 16});
// every lane of the group receives the total. DPP adds, no LDS traffic.
template <int LPT>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp_xor1(x);
  x += dpp_xor2(x);
  if constexpr (LPT >= 8) x += dpp_half_mirror(x);
  if constexpr (LPT >= 16) x += dpp_mirror(x);
  return x;
}

// The same over ints (exact: no rounding at any step).
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int x) {
  return __builtin_amdgcn_mov_dpp(x, CTRL, 0xF, 0xF, true);
}
template <int LPT>
__device__ __forceinline__ int group_sum_i32(int x) {
  x += dpp_i32<0xB1>(x);
  x += dpp_i32<0x4E>(x);
  if constexpr (LPT >= 8) x += dpp_i32<0x141>(x);
  if constexpr (LPT >= 16) x += dpp_i32<0x140>(x);
  return x;
}

// Reductions over the whole wave, every lane receiving the result, without
// LDS: DPP within rows of 16 lanes (quad swaps, half-row and row mirrors),
// then gfx950's lane swaps across rows (v_permlane16_swap) and halves
// (v_permlane32_swap); each swap of a value with itself hands every lane its
// partner's value beside its own.
template <class Op>
__device__ __forceinline__ float wave_reduce(float x, Op op) {
  x = op(x, dpp_f32<0xB1>(x));   // quad_perm [1,0,3,2]
  x = op(x, dpp_f32<0x4E>(x));   // quad_perm [2,3,0,1]
  x = op(x, dpp_f32<0x141>(x));  // row_half_mirror
  x = op(x, dpp_f32<0x140>(x));  // row_mirror
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float wave_max(float x) {
  return wave_reduce(x, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_sum(float x) {
  return wave_reduce(x, [](float a, float b) { return a + b; });
}
// The same over a wave's token groups only (lanes that differ in the bits at
// and above log2(LPT)): each lane receives the reduction over the lanes of
// its position within a token.
template <int LPT, class Op>
__device__ __forceinline__ float groups_reduce(float x, Op op) {
  if constexpr (LPT <= 4) x = op(x, __shfl_xor(x, 4));
  if constexpr (LPT <= 8) x = op(x, dpp_f32<0x128>(x));  // row_ror:8, lane i ^ 8 of a row
  if constexpr (LPT <= 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  if constexpr (LPT <= 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  return x;
}
template <int LPT>
__device__ __forceinline__ float groups_max(float x) {
  return groups_reduce<LPT>(x, [](float a, float b) { return fmaxf(a, b); });
}

// Sum over a wave's token groups (lanes that differ in the bits at and above
// log2(LPT)) of each lane's N per-channel partial sums, scattered: one step
// per token-group bit, from bit 5 down, in which the two lanes that differ in
// that bit swap half of their values and add, so the values held halve each
// step and lane l ends with N >> steps totals, of its chunk's channels
// scatter_base<LPT, N>(l) + e, in acc[e]. Bits 5 and 4 use gfx950's lane
// swaps (v_permlane32_swap, v_permlane16_swap), bit 3 a DPP rotate by 8
// within a row, bit 2 one swizzle: VALU moves, where the butterfly over
// every value (__shfl_xor per value and bit) took one LDS permute each, 64
// per lane at D = 64 in every wave's epilogue.
template <int LPT, int N>
__device__ __forceinline__ int scatter_base(int lane) {
  int base = 0, n = N;
  if constexpr (LPT <= 32) { n >>= 1; base += ((lane >> 5) & 1) * n; }
  if constexpr (LPT <= 16) { n >>= 1; base += ((lane >> 4) & 1) * n; }
  if constexpr (LPT <= 8) { n >>= 1; base += ((lane >> 3) & 1) * n; }
  if constexpr (LPT <= 4) { n >>= 1; base += ((lane >> 2) & 1) * n; }
  return base;
}
template <int LPT, int N>
__device__ __forceinline__ void reduce_scatter_groups(float (&acc)[N], int lane) {
  if constexpr (LPT <= 32) {
    static_assert(N % 2 == 0, "a value per lane half");
    // Lanes 0-31 keep values [0, N/2), lanes 32-63 values [N/2, N).
#pragma unroll
    for (int k = 0; k < N / 2; ++k) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[k]), __float_as_uint(acc[N / 2 + k]),
                                                     false, false);
      acc[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  }
  if constexpr (LPT <= 16) {
    static_assert(N % 4 == 0, "a value per lane quarter");
    // Even rows of 16 lanes keep [0, N/4), odd rows [N/4, N/2).
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[k]), __float_as_uint(acc[N / 4 + k]),
                                                     false, false);
      acc[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  }
  if constexpr (LPT <= 8) {
    static_assert(N % 8 == 0, "a value per lane eighth");
    // Lanes i and i ^ 8 of a row: a rotate by 8 within the row pairs them.
    const bool hi = ((lane >> 3) & 1) != 0;
#pragma unroll
    for (int k = 0; k < N / 8; ++k) {
      const float keep = hi ? acc[N / 8 + k] : acc[k];
      const float give = hi ? acc[k] : acc[N / 8 + k];
      acc[k] = keep + dpp_f32<0x128>(give);  // row_ror:8
    }
  }
  if constexpr (LPT <= 4) {
    static_assert(N % 16 == 0, "a value per lane sixteenth");
    const bool hi = ((lane >> 2) & 1) != 0;
#pragma unroll
    for (int k = 0; k < N / 16; ++k) {
      const float keep = hi ? acc[N / 16 + k] : acc[k];
      const float give = hi ? acc[k] : acc[N / 16 + k];
      acc[k] = keep + __shfl_xor(give, 4);
    }
  }
}

// Largest |x| of a lane's values with f32::max / fmaxf semantics (NaNs of
// either kind skipped); the result is >= +0 and never NaN. Written on the bit
// patterns: the hardware float max quiets a signalling NaN and returns it,
// which would drop the max of the values before it.
template <int N>
__device__ __forceinline__ float lane_absmax(const float (&x)[N]) {
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const uint32_t a = __float_as_uint(x[k]) & 0x7fffffffu;
    m = max(m, a > 0x7f800000u ? 0u : a);
  }
  return __uint_as_float(m);
}

// ---------------------------------------------------------------------------
// Kernel 1: quantize (dense) / quantize-and-append (arena).
// One wave per (tensor, row); D/64 channels per lane.
// Bit-exact contract (int8_kv_ops.rs:17-18, int8_kv.cu:13,17):
//   s = max(absmax / 127, 1e-12); code = clamp(rne(x / s), -127, 127).
// NaN quotients become code 0 (as a float->int conversion of NaN does on
// the reference GPU path); the absmax ignores NaN like fmaxf / f32::max.
// ---------------------------------------------------------------------------
// Quantise one row of D values into codes[0..D) and *scale; the whole wave
// participates, lane l holding elements l*D/64 ... (l+1)*D/64 - 1 of the
// row. A non-finite value is reported through flags when given.
template <int D>
__device__ __forceinline__ void quantize_values(const float (&x)[D / ppk::kWave], uint8_t* codes, float* scale,
                                                uint32_t* flags, int lane) {
#pragma clang fp contract(off)
  constexpr int EPL = D / ppk::kWave;
  bool finite = true;
#pragma unroll
  for (int e = 0; e < EPL; ++e) finite = finite && __builtin_isfinite(x[e]);
  const float amax = wave_max(lane_absmax(x));
  const float s = fmaxf(amax / 127.0f, 1e-12f);
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float qf = rintf(x[e] / s);
    const int qi = (qf != qf) ? 0 : int(fminf(fmaxf(qf, -127.f), 127.f));
    packed |= (uint32_t(qi) & 0xffu) << (8 * e);
  }
  uint8_t* out = codes + size_t(lane) * EPL;
  if constexpr (EPL == 1) *out = uint8_t(packed);
  else if constexpr (EPL == 2) *reinterpret_cast<uint16_t*>(out) = uint16_t(packed);
  else *reinterpret_cast<uint32_t*>(out) = packed;
  if (lane == 0) *scale = s;
  if (flags) {
    const bool any_bad = __any(!finite);
    if (any_bad && lane == 0) atomicOr(flags, 1u);
  }
}

// The same for row src_row of src[rows, D] in dtype.
template <int D>
__device__ __forceinline__ void quantize_row(const void* src, size_t src_row, uint32_t dtype, uint8_t* codes,
                                             float* scale, uint32_t* flags, int lane) {
  constexpr int EPL = D / ppk::kWave;
  float x[EPL];
  load_vec<EPL>(src, src_row * D + size_t(lane) * EPL, dtype, x);
  quantize_values<D>(x, codes, scale, flags, lane);
}

template <int D>
__device__ __forceinline__ void quantize_body(const ppk::QuantizeArgs& a) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = uint64_t(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64;
  if (wave >= a.rows * a.ntensors) return;  // uniform per wave
  const uint32_t tensor = wave >= a.rows ? 1u : 0u;
  const uint64_t r = wave - (tensor ? a.rows : 0);
  const void* src = tensor ? a.src[1] : a.src[0];
  size_t dst = r;
  if (a.capacity) {
    const uint64_t bh = r / a.tokens;
    const uint32_t tok = uint32_t(r - bh * a.tokens);
    const uint64_t slot = uint64_t(a.past ? a.past[bh / a.heads] : a.uniform_past) + tok;
    if (slot >= a.capacity) {
      if (lane == 0 && a.flags) atomicOr(a.flags, 2u);
      return;
    }
    dst = bh * a.capacity + slot;
  }
  quantize_row<D>(src, r, a.src_dtype, (tensor ? a.codes[1] : a.codes[0]) + dst * D,
                  (tensor ? a.scales[1] : a.scales[0]) + dst, a.flags, lane);
}

// ---------------------------------------------------------------------------
// Dequantize: 16 codes per thread (one dwordx4), grid-stride.
// ---------------------------------------------------------------------------
// Dequantization in units of one 16-byte output chunk: E = 8 codes for a
// 16-bit output, 4 for f32. Lane l of a wave handles units i, i + stride, ...
// so every load instruction of a wave reads 64*E consecutive code bytes and
// every store instruction writes 1 KiB of consecutive output. Each lane keeps
// two batches of R units: the next batch's loads are issued before the
// current batch's stores, so a load never waits behind the previous batch's
// store acknowledgements (loads and stores share one in-order counter). The
// host sizes the grid for one batch per lane up to 128 blocks per CU (the
// measured optimum; the grid-stride loop covers larger inputs).
template <int E, uint32_t OUT, bool ROUND>
__device__ __forceinline__ void dequantize_units(const ppk::DequantizeArgs& a) {
#pragma clang fp contract(off)
  constexpr int R = 8;
  using Raw = typename std::conditional<E == 8, u2, uint32_t>::type;
  const uint64_t units = a.rows * (a.head_dim / E);
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  const uint32_t row_shift = __builtin_ctz(a.head_dim / E);  // units per token row: a power of two
  uint64_t base = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (base >= units) return;
  Raw cur[R], nxt[R];
  float cs[R], ns[R];
  auto load = [&](uint64_t b, Raw (&raw)[R], float (&sc)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint64_t u = min(b + r * stride, units - 1);  // clamp: always in bounds, extra units unused
      raw[r] = __builtin_nontemporal_load(reinterpret_cast<const Raw*>(a.codes) + u);
      sc[r] = a.scales[u >> row_shift];
    }
  };
  load(base, cur, cs);
  for (; base < units; base += R * stride) {
    const bool more = base + R * stride < units;
    if (more) load(base + R * stride, nxt, ns);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint64_t u = base + r * stride;
      if (u >= units) break;
      float f[E];
#pragma unroll
      for (int k = 0; k < E; ++k) {
        uint32_t w;
        if constexpr (E == 8) w = cur[r][k / 4];
        else w = cur[r];
        const float v = sbyte(w, k % 4) * cs[r];
        f[k] = ROUND ? round_bf16(v) : v;
      }
      if constexpr (E == 4) {
        __builtin_nontemporal_store(f4{f[0], f[1], f[2], f[3]}, static_cast<f4*>(a.out) + u);
      } else {
        uint32_t h[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint16_t lo = OUT == kBF16 ? f32_to_bf16_bits(f[2 * w]) : f32_to_f16_bits(f[2 * w]);
          const uint16_t hi = OUT == kBF16 ? f32_to_bf16_bits(f[2 * w + 1]) : f32_to_f16_bits(f[2 * w + 1]);
          h[w] = uint32_t(lo) | (uint32_t(hi) << 16);
        }
        __builtin_nontemporal_store(u4{h[0], h[1], h[2], h[3]}, static_cast<u4*>(a.out) + u);
      }
    }
    if (!more) break;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      cur[r] = nxt[r];
      cs[r] = ns[r];
    }
  }
}

// Output type and the bf16 pre-rounding are fixed per instantiation (a bf16
// output already rounds to bf16, so it needs no pre-rounding).
__device__ __forceinline__ void dequantize_body(const ppk::DequantizeArgs& a) {
  if (a.out_dtype == kF32) {
    if (a.round_bf16) dequantize_units<4, kF32, true>(a);
    else dequantize_units<4, kF32, false>(a);
  } else if (a.out_dtype == kBF16) {
    dequantize_units<8, kBF16, false>(a);
  } else {
    if (a.round_bf16) dequantize_units<8, kF16, true>(a);
    else dequantize_units<8, kF16, false>(a);
  }
}

// ---------------------------------------------------------------------------
// Kernel 2a: decode attention. A block of W waves covers W*S consecutive
// history tokens of one row (group g of the row); each wave streams its own S
// tokens, the block combines its waves through LDS. With one group per row
// the block also scores the current token and writes the final output, so a
// decode step is a single launch; otherwise it writes a partial (m, z, y)
// record for the merge kernel. Optionally the block first quantises the new
// K/V token of its row into slot past[b] (a slot attention never reads).
//
// Lane layout inside a wave: LPT = D/16 lanes share one token, each holding
// 16 channels, so one dwordx4 load per lane moves 1 KiB = TPL = 64/LPT whole
// tokens. The dot product is 16 FMAs per lane plus a DPP group sum; the
// per-token scale is applied once to the sum (default) instead of to every
// element. Phase K streams K codes and scales and leaves log2-domain scores
// in LDS; phase V streams V codes and scales and accumulates
// p_t * vscale_t * code_t per channel. The exact wave max is known before
// phase V, so no running rescale is needed. Each wave keeps two batches of
// loads in flight (the next batch is issued before the current is consumed).
// ---------------------------------------------------------------------------
struct WavePartial {
  float m;         // max log2-domain score (-inf if the wave had no tokens)
  float z;         // sum of 2^(s - m)
  float acc[16];   // sum of 2^(s - m) * v: while streaming over this lane's 16 channels; at the end the wave's
                   // totals of channels c * 16 + scatter_base<LPT, 16>(lane) + e in acc[e], e < D / 64
#ifdef PPK_WAVE_CLOCK
  uint64_t t_first = 0;  // the clock when the stream's first K data had arrived
#endif
};

// One batch = U load tiles = U*TPL consecutive tokens of this wave's range.
// Codes come as one dwordx4 per lane per tile; the batch's per-token scales
// come as one coalesced dword per lane (lane l holds token l of the batch)
// and reach each token's lane group through a cross-lane read.
template <int D, int U>
__device__ __forceinline__ void load_batch(const uint8_t* base, const float* scales, uint32_t t0, uint32_t n, int j,
                                           int lane, u4 (&raw)[U], float& scale) {
  constexpr int TPL = ppk::kWave / (D / 16);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t tc = min((t0 + u) * TPL + j, n - 1);  // clamp: always in bounds
    raw[u] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(base + size_t(tc) * D));
  }
  // Scales stay cacheable: a batch's 4*TPL scales need not start on a cache
  // line (capacity is arbitrary), and the next batch reuses the shared line.
  scale = scales[min(t0 * TPL + uint32_t(lane % (U * TPL)), n - 1)];
}

// q in exact integer form for the K-phase dot products: every lane's 16
// channels become q_int = rne(q / qmax * Q), Q = 127 * 2^21, split into four
// signed bytes hi*2^21 + m1*2^14 + m2*2^7 + lo (each in [-127, 127]) packed
// four channels per dword. <codes, part> is then an exact v_dot4_i32_i8 sum;
// the four partial sums pair up exactly in int32 (hi*2^7 + m1, m2*2^7 + lo),
// are summed over the token's lanes in int32 (exact), and meet in one fp32
// multiply-add, so q_int . codes carries fp32 rounding only. q_int keeps 29
// bits of q relative to the row's max |q|: with 22 bits (three slices) the
// rounding of q was the largest error on heavy-tailed history (max relative
// error 7.9e-3 at D = 64 against the f64 oracle, 1.2e-3 with 29 bits; the
// time per step the same).
struct QInt {
  int hi[4], m1[4], m2[4], lo[4];
  float unscale;  // qmax / Q (NaN if q held a non-finite value)
};

template <int LPT>
__device__ __forceinline__ float group_max(float x) {
  x = fmaxf(x, dpp_xor1(x));
  x = fmaxf(x, dpp_xor2(x));
  if constexpr (LPT >= 8) x = fmaxf(x, dpp_half_mirror(x));
  if constexpr (LPT >= 16) x = fmaxf(x, dpp_mirror(x));
  return x;
}

// Max over G consecutive lanes (G a power of two <= 64) of values that are
// >= +0 and never NaN: such floats order like their bit patterns, so the
// reduction runs as unsigned integer max (the DPP move folds into the max,
// and no NaN canonicalisation is needed).
template <int G>
__device__ __forceinline__ float group_max_nonneg(float x) {
  uint32_t b = __float_as_uint(x);
  auto step = [&](uint32_t o) { b = max(b, o); };
  step(uint32_t(__builtin_amdgcn_mov_dpp(int(b), 0xB1, 0xF, 0xF, true)));
  step(uint32_t(__builtin_amdgcn_mov_dpp(int(b), 0x4E, 0xF, 0xF, true)));
  if constexpr (G >= 8) step(uint32_t(__builtin_amdgcn_mov_dpp(int(b), 0x141, 0xF, 0xF, true)));
  if constexpr (G >= 16) step(uint32_t(__builtin_amdgcn_mov_dpp(int(b), 0x140, 0xF, 0xF, true)));
#pragma unroll
  for (int o = 16; o < G; o <<= 1) step(uint32_t(__shfl_xor(int(b), o)));
  return __uint_as_float(b);
}

// Quantization at streaming rates: dense (int8_kv_ops::quantize over [rows,
// D]) and quantize-and-append into arenas (rows of K and V written at slot
// past[b] + t). A row's D values are split over G = D / E lanes, 16 bytes (E
// values) per lane, so one wave-wide load covers 64 / G whole rows and the
// row's absmax is a G-lane reduction; each lane then forms its E codes with
// the same arithmetic as quantize_row (IEEE division, ties-to-even, clamp,
// NaN quotient -> 0). Lanes hold two batches of R units and issue the next
// batch's loads (and, for appends, the sequences' past entries) before the
// current batch's stores. Loop control is uniform per wave (rows never
// straddle waves: G divides 64), so the cross-lane reductions always run
// with every lane active; units past the end are clamped for loading and
// masked for storing. The host sends rows * ntensors < 2^32 here.
template <int D, int E, uint32_t DT, bool ARENA>
__device__ __forceinline__ void quantize_stream_units(const ppk::QuantizeArgs& a) {
#pragma clang fp contract(off)
  constexpr int G = D / E;
  constexpr int R = 4;
  static_assert(64 % G == 0, "a row's lanes stay inside one wave");
  using Code = typename std::conditional<E == 8, u2, uint32_t>::type;
  const int lane = threadIdx.x & 63;
  const uint32_t rows = uint32_t(a.rows);  // per tensor
  const uint64_t units = uint64_t(a.ntensors) * rows * G;
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  uint64_t wave_base = uint64_t(blockIdx.x) * blockDim.x + (threadIdx.x & ~63u);
  if (wave_base >= units) return;  // uniform per wave
  u4 cur[R], nxt[R];
  uint32_t pcur[R], pnxt[R];  // appends: past entry of the unit's sequence
  auto load = [&](uint64_t wb, u4 (&raw)[R], uint32_t (&pv)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint64_t u = min(wb + uint64_t(lane) + r * stride, units - 1);  // clamp: in bounds, masked later
      if constexpr (ARENA) {
        const uint32_t ri = uint32_t(u / G);
        const uint32_t t = ri >= rows ? 1u : 0u;
        const uint32_t row = ri - t * rows;
        const u4* src = static_cast<const u4*>(t ? a.src[1] : a.src[0]);
        raw[r] = __builtin_nontemporal_load(src + uint64_t(row) * G + uint32_t(u % G));
        pv[r] = a.past ? a.past[(row / a.tokens) / a.heads] : a.uniform_past;
      } else {
        raw[r] = __builtin_nontemporal_load(static_cast<const u4*>(a.src[0]) + u);
      }
    }
  };
  load(wave_base, cur, pcur);
  bool any_bad = false, any_over = false;
  for (; wave_base < units; wave_base += R * stride) {
    const bool more = wave_base + R * stride < units;  // uniform per wave
    if (more) load(wave_base + R * stride, nxt, pnxt);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint64_t u = wave_base + uint64_t(lane) + r * stride;
      const bool valid = u < units;
      float x[E];
      if constexpr (DT == kF32) {
#pragma unroll
        for (int k = 0; k < E; ++k) x[k] = __uint_as_float(cur[r][k]);
      } else {
#pragma unroll
        for (int k = 0; k < E; ++k) {
          const uint16_t h = uint16_t(cur[r][k / 2] >> (16 * (k % 2)));
          x[k] = DT == kBF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
      }
      // Fast row max: the float max chain is exact unless the lane holds a
      // NaN (a signalling one can drop the values before it); such a lane
      // then has a NaN product below, and the wave recomputes.
      float m = 0.f;
#pragma unroll
      for (int k = 0; k < E; ++k) m = fmaxf(m, fabsf(x[k]));
      float sc = fmaxf(group_max_nonneg<G>(m) / 127.0f, 1e-12f);
      // Rounded quotients from a product with the hardware reciprocal (at
      // most 1 ulp off 1/sc): for finite x, |x·r - RN(x/sc)| <= 2.7e-5 since
      // |x/sc| <= 127·(1 + 2^-24), so a product farther than 2^-14 from every
      // half-integer rounds to the same integer as the correctly rounded
      // quotient. A product within that band, or a non-finite one (x or sc
      // non-finite), marks its lane for the division. A product outside the
      // band is also below 127.5 in magnitude, so its rounded value needs no
      // clamp; the division path keeps the clamp.
      const float rcp = __builtin_amdgcn_rcpf(sc);
      int qi[E];
      bool near[E], any_near = false;
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const float p = x[k] * rcp;
        const float n = rintf(p);
        near[k] = !(fabsf(p - n) < 0.5f - 0x1p-14f);
        any_near = any_near || near[k];
        qi[k] = int(n);
      }
      auto exact = [&](int k) {
        const float t = rintf(x[k] / sc);
        qi[k] = t != t ? 0 : int(__builtin_amdgcn_fmed3f(t, -127.f, 127.f));  // NaN quotient -> code 0
      };
      bool finite = true;
      if (__any(any_near)) {  // wave-uniform
#pragma unroll
        for (int k = 0; k < E; ++k) finite = finite && __builtin_isfinite(x[k]);
        if (__any(!finite)) {
          // A non-finite input may have spoilt the fast max of its row: the
          // wave recomputes every row it holds with the NaN-skipping max and
          // the division (the reduction needs all lanes).
          sc = fmaxf(group_max_nonneg<G>(lane_absmax(x)) / 127.0f, 1e-12f);
#pragma unroll
          for (int k = 0; k < E; ++k) exact(k);
        } else {
          // Finite rows: the scale stands; only the flagged values divide.
#pragma unroll
          for (int k = 0; k < E; ++k)
            if (near[k]) exact(k);
        }
      }
      uint32_t packed[(E + 3) / 4];
#pragma unroll
      for (int w = 0; w < E / 4; ++w) {
        // v_perm: bytes 0 of (a, b) and of (c, d), then the two byte pairs.
        const uint32_t ab = __builtin_amdgcn_perm(uint32_t(qi[4 * w + 1]), uint32_t(qi[4 * w]), 0x0c0c0400u);
        const uint32_t cd = __builtin_amdgcn_perm(uint32_t(qi[4 * w + 3]), uint32_t(qi[4 * w + 2]), 0x0c0c0400u);
        packed[w] = __builtin_amdgcn_perm(cd, ab, 0x05040100u);
      }
      Code c;
      if constexpr (E == 8) c = u2{packed[0], packed[1]};
      else c = packed[0];
      bool in_arena = true;
      if constexpr (ARENA) {
        const uint32_t ri = uint32_t(min(u, units - 1) / G);
        const uint32_t t = ri >= rows ? 1u : 0u;
        const uint32_t row = ri - t * rows;
        const uint32_t bh = row / a.tokens;
        const uint64_t slot = uint64_t(pcur[r]) + (row - bh * a.tokens);
        in_arena = slot < a.capacity;
        const uint64_t dst = uint64_t(bh) * a.capacity + slot;
        if (valid && in_arena) {
          __builtin_nontemporal_store(c, reinterpret_cast<Code*>(a.codes[t] + dst * D) + uint32_t(u % G));
          if (lane % G == 0) a.scales[t][dst] = sc;
        }
      } else if (valid) {
        __builtin_nontemporal_store(c, reinterpret_cast<Code*>(a.codes[0]) + u);
        if (lane % G == 0) a.scales[0][u / G] = sc;
      }
      any_bad = any_bad || (valid && !finite);
      any_over = any_over || (valid && !in_arena);
    }
    if (!more) break;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      cur[r] = nxt[r];
      pcur[r] = pnxt[r];
    }
  }
  if (a.flags) {
    const bool bad = __any(any_bad), over = __any(any_over);
    if (lane == 0 && (bad || over)) atomicOr(a.flags, (bad ? 1u : 0u) | (over ? 2u : 0u));
  }
}

template <int D, bool ARENA>
__device__ __forceinline__ void quantize_stream_dtype(const ppk::QuantizeArgs& a) {
  if (a.src_dtype == kF32) quantize_stream_units<D, 4, kF32, ARENA>(a);
  else if (a.src_dtype == kBF16) quantize_stream_units<D, 8, kBF16, ARENA>(a);
  else quantize_stream_units<D, 8, kF16, ARENA>(a);
}


template <int LPT>
__device__ __forceinline__ QInt quantize_query(const float (&qr)[16]) {
  constexpr float Q = 266338304.0f;  // 127 * 2^21
  float amax = 0.f;
  bool finite = true;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    amax = fmaxf(amax, fabsf(qr[i]));
    finite = finite && __builtin_isfinite(qr[i]);
  }
  amax = group_max<LPT>(amax);  // every lane of a token group holds the whole row of q
  const float bad = group_max<LPT>(finite ? 0.f : 1.f);
  const float inv = amax > 0.f ? Q / amax : 0.f;
  QInt r;
  r.unscale = bad > 0.f ? __builtin_nanf("") : amax / Q;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t h = 0, a = 0, b = 0, l = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float x = fminf(fmaxf(rintf(qr[4 * w + k] * inv), -Q), Q);
      const int qi = finite ? int(x) : 0;
      const int hi = (qi + (1 << 20)) >> 21;  // [-127, 127]
      const int r1 = qi - hi * (1 << 21);     // [-2^20, 2^20)
      const int m1 = (r1 + 8192) >> 14;       // [-64, 64]
      const int r2 = r1 - m1 * 16384;         // [-8192, 8191]
      const int m2 = (r2 + 64) >> 7;          // [-64, 64]
      const int lo = r2 - m2 * 128;           // [-64, 63]
      h |= (uint32_t(hi) & 0xffu) << (8 * k);
      a |= (uint32_t(m1) & 0xffu) << (8 * k);
      b |= (uint32_t(m2) & 0xffu) << (8 * k);
      l |= (uint32_t(lo) & 0xffu) << (8 * k);
    }
    r.hi[w] = int(h);
    r.m1[w] = int(a);
    r.m2[w] = int(b);
    r.lo[w] = int(l);
  }
  return r;
}

// Phase K for one batch of U tiles: scores (log2 domain) into LDS, running max.
template <int D, bool BF16H, int U>
__device__ __forceinline__ float score_batch(const u4 (&raw)[U], float scale_lane, uint32_t t0, uint32_t n, int j,
                                             int c, const float (&qr)[16], const QInt& qi, float sl2, float* s_lds,
                                             float mloc) {
  constexpr int LPT = D / 16;
  constexpr int TPL = ppk::kWave / LPT;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t tok = (t0 + u) * TPL + j;
    const float kscale = __shfl(scale_lane, u * TPL + j);
    float sc;
    if constexpr (BF16H) {
      // pp_i8_load semantics: every element is bf16(code * scale) before the fp32 dot.
      float d = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          float e0, e1;
          round_bf16_pair(sbyte(raw[u][w], k) * kscale, sbyte(raw[u][w], k + 1) * kscale, e0, e1);
          d = fmaf(qr[4 * w + k], e0, d);
          d = fmaf(qr[4 * w + k + 1], e1, d);
        }
      sc = group_sum<LPT>(d) * sl2;
    } else {
      int sh = 0, s1 = 0, s2 = 0, sl = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        sh = __builtin_amdgcn_sdot4(int(raw[u][w]), qi.hi[w], sh, false);
        s1 = __builtin_amdgcn_sdot4(int(raw[u][w]), qi.m1[w], s1, false);
        s2 = __builtin_amdgcn_sdot4(int(raw[u][w]), qi.m2[w], s2, false);
        sl = __builtin_amdgcn_sdot4(int(raw[u][w]), qi.lo[w], sl, false);
      }
      const int hm = group_sum_i32<LPT>(sh * 128 + s1);
      const int lm = group_sum_i32<LPT>(s2 * 128 + sl);
      sc = fmaf(float(hm), 16384.f, float(lm)) * (kscale * sl2);
    }
    sc = tok < n ? sc : -INFINITY;
    mloc = fmaxf(mloc, sc);
    if (c == 0 && tok < n) s_lds[tok] = sc;
  }
  return mloc;
}

// Phase V for one batch: lane l owns token l of the batch (the layout of the
// scale load), turns its score into p = 2^(s - m) once, adds it to z and
// forms the weight p * vscale; each tile's token groups then fetch their
// token's weight with one cross-lane read and accumulate weight * code.
template <int D, bool BF16H, int U>
__device__ __forceinline__ void accumulate_batch(const u4 (&raw)[U], float scale_lane, uint32_t t0, uint32_t n, int j,
                                                 int lane, float m, const float* s_lds, float& z, float (&acc)[16]) {
  constexpr int LPT = D / 16;
  constexpr int TPL = ppk::kWave / LPT;
  constexpr int TPB = U * TPL;  // tokens per batch (<= 64)
  static_assert(TPB <= ppk::kWave, "one scale per lane per batch");
  const uint32_t tl = t0 * TPL + uint32_t(lane % TPB);
  const float e = __builtin_amdgcn_exp2f(s_lds[min(tl, n - 1)] - m);
  const float pr = (tl < n && lane < TPB) ? e : 0.f;
  z += pr;
  const float w_lane = BF16H ? pr : pr * scale_lane;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float wgt = __shfl(w_lane, u * TPL + j);
    if constexpr (BF16H) {
      const float vscale = __shfl(scale_lane, u * TPL + j);
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          float e0, e1;
          round_bf16_pair(sbyte(raw[u][w], k) * vscale, sbyte(raw[u][w], k + 1) * vscale, e0, e1);
          acc[4 * w + k] = fmaf(wgt, e0, acc[4 * w + k]);
          acc[4 * w + k + 1] = fmaf(wgt, e1, acc[4 * w + k + 1]);
        }
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[4 * w + k] = fmaf(wgt, sbyte(raw[u][w], k), acc[4 * w + k]);
    }
  }
}

// Log2-domain score of the current token (q . sk * scale), which comes from
// the scratch copy, not the arena: each lane dots its 16-channel chunk.
template <int D>
__device__ __forceinline__ float current_score(const ppk::DecodeArgs& a, const float (&kv)[16],
                                               const float (&qr)[16]) {
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) d = fmaf(qr[i], kv[i], d);
  return group_sum<D / 16>(d) * a.scale_log2;
}

// Streams this wave's n tokens (from `begin`) of one row: phase K scores,
// phase V accumulation. A ring of NB batches (rr[b], rs[b]) keeps NB - 1
// batches' loads in flight while one is consumed: batch i of the sequence
// K_0 .. K_{nb-1}, (padding to a whole ring), V_0 .. V_{nb-1} lives in slot
// i % NB, and each slot is refilled with batch i + NB as soon as batch i is
// used, so phase V's first batches are requested during phase K's last ones.
// Addresses past the end clamp to the last token and those tokens are masked
// out. With `pre` (nspec beyond the short window) the caller has already
// issued the first K batches into the ring, clamped to nspec instead of n
// (tokens at or past n are masked by their scores, so the wider clamp only
// reads other slots of the same arena row).
template <int D, bool BF16H, int NB>
__device__ __forceinline__ void wave_attention(const ppk::DecodeArgs& a, uint32_t row, uint32_t begin, uint32_t n,
                                               uint32_t nspec, const float (&qr)[16], float* s_lds, int lane,
                                               WavePartial& out, bool pre, u4 (&rr)[NB][4], float (&rs)[NB]) {
  static_assert(NB >= 2, "the short-stream path keeps its K batches in ring slots 0 and 1");
  constexpr int LPT = D / 16;
  constexpr int TPL = ppk::kWave / LPT;
  constexpr int U = 4;  // tiles per batch
  const int j = lane / LPT;  // token within a load tile
  const int c = lane % LPT;  // 16-channel chunk
  out.m = -INFINITY;
  out.z = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) out.acc[i] = 0.f;

  const size_t tok0 = size_t(row) * a.capacity + begin;
  const uint8_t* kb = a.k + tok0 * D + size_t(c) * 16;
  const uint8_t* vb = a.v + tok0 * D + size_t(c) * 16;
  const float* ksb = a.ks + tok0;
  const float* vsb = a.vs + tok0;
  if (nspec > 0 && nspec <= uint32_t(2 * U * TPL)) {
    // Short window (at most two batches per phase): K and V are requested
    // before the row's length is known, clamped to the window's slots inside
    // the arena (always in bounds); slots at or past the length n are masked
    // below and their scales zeroed, so stale or uninitialised arena memory
    // never reaches the result.
    const bool two = nspec > uint32_t(U * TPL);  // uniform per wave
    u4 ka[U], kb2[U], va[U], vb2[U];
    float ksa, ksb2, vsa, vsb2;
    load_batch<D, U>(kb, ksb, 0, nspec, j, lane, ka, ksa);
    load_batch<D, U>(vb, vsb, 0, nspec, j, lane, va, vsa);
    if (two) {
      load_batch<D, U>(kb, ksb, U, nspec, j, lane, kb2, ksb2);
      load_batch<D, U>(vb, vsb, U, nspec, j, lane, vb2, vsb2);
    }
    QInt qi{};
    float sl2 = a.scale_log2;
    if constexpr (!BF16H) {
      qi = quantize_query<LPT>(qr);
      sl2 *= qi.unscale;
    }
    if (n == 0) return;  // uniform per wave
    PPK_CLK_AT(out.t_first, ka[0][0]);
    const uint32_t tl = uint32_t(lane % (U * TPL));
    ksa = tl < n ? ksa : 0.f;
    vsa = tl < n ? vsa : 0.f;
    float mloc = -INFINITY;
    mloc = score_batch<D, BF16H, U>(ka, ksa, 0, n, j, c, qr, qi, sl2, s_lds, mloc);
    if (two) {
      ksb2 = U * TPL + tl < n ? ksb2 : 0.f;
      vsb2 = U * TPL + tl < n ? vsb2 : 0.f;
      mloc = score_batch<D, BF16H, U>(kb2, ksb2, U, n, j, c, qr, qi, sl2, s_lds, mloc);
    }
    float m = mloc, z = 0.f;
    m = groups_max<LPT>(m);
    __builtin_amdgcn_wave_barrier();
    accumulate_batch<D, BF16H, U>(va, vsa, 0, n, j, lane, m, s_lds, z, out.acc);
    if (two) accumulate_batch<D, BF16H, U>(vb2, vsb2, U, n, j, lane, m, s_lds, z, out.acc);
    z = wave_sum(z);
    reduce_scatter_groups<LPT, 16>(out.acc, lane);
    out.m = m;
    out.z = z;
    return;
  }
  if (n == 0) return;  // uniform per wave
  const uint32_t ntiles = (n + TPL - 1) / TPL;
  float mloc = -INFINITY;
  float m, z = 0.f;
  QInt qi{};
  float sl2 = a.scale_log2;
  if (ntiles <= 2 * U) {
    // Short stream (at most two batches per phase, e.g. many small splits of
    // short rows): K and V of the whole wave are requested together, so the
    // wave waits on one memory round trip instead of a K trip and a V trip.
    const bool two = ntiles > U;  // uniform per wave
    u4 va[U], vb2[U];
    float vsa, vsb2;
    if (!pre) load_batch<D, U>(kb, ksb, 0, n, j, lane, rr[0], rs[0]);
    load_batch<D, U>(vb, vsb, 0, n, j, lane, va, vsa);
    if (two) {
      if (!pre) load_batch<D, U>(kb, ksb, U, n, j, lane, rr[1], rs[1]);
      load_batch<D, U>(vb, vsb, U, n, j, lane, vb2, vsb2);
    }
    if constexpr (!BF16H) {
      qi = quantize_query<LPT>(qr);
      sl2 *= qi.unscale;
    }
    PPK_CLK_AT(out.t_first, rr[0][0][0]);
    mloc = score_batch<D, BF16H, U>(rr[0], rs[0], 0, n, j, c, qr, qi, sl2, s_lds, mloc);
    if (two) mloc = score_batch<D, BF16H, U>(rr[1], rs[1], U, n, j, c, qr, qi, sl2, s_lds, mloc);
    m = mloc;
    m = groups_max<LPT>(m);
    __builtin_amdgcn_wave_barrier();
    accumulate_batch<D, BF16H, U>(va, vsa, 0, n, j, lane, m, s_lds, z, out.acc);
    if (two) accumulate_batch<D, BF16H, U>(vb2, vsb2, U, n, j, lane, m, s_lds, z, out.acc);
  } else {
    // The first K batches do not depend on q: issue them before the query is
    // quantised, so the q load and its reductions overlap the first memory
    // round trip. Every ring load is issued unconditionally (batches past the
    // end clamp to the row's last token, a cached line) so that each wait is
    // for exactly the oldest batch: a conditional load leaves the compiler's
    // count of loads in flight unknown on one path, and it then waits for
    // all of them (vmcnt(0)), which drains the ring every batch. Only the
    // arithmetic of batches past the end is skipped (uniform branches).
    const uint32_t nb = (ntiles + U - 1) / U;       // K batches (and V batches)
    const uint32_t nbp = (nb + NB - 1) / NB * NB;   // rounded up to whole rings
    if (!pre) {
#pragma unroll
      for (int b = 0; b < NB; ++b) load_batch<D, U>(kb, ksb, uint32_t(b) * U, n, j, lane, rr[b], rs[b]);
    }
    if constexpr (!BF16H) {
      qi = quantize_query<LPT>(qr);
      sl2 *= qi.unscale;
    }
    PPK_CLK_AT(out.t_first, rr[0][0][0]);
    for (uint32_t k0 = 0; k0 < nbp; k0 += NB) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint32_t i = k0 + uint32_t(b);
        if (i < nb) mloc = score_batch<D, BF16H, U>(rr[b], rs[b], i * U, n, j, c, qr, qi, sl2, s_lds, mloc);
        // Refill slot b with item i + NB: K batch i + NB, or V batch i + NB - nbp.
        const bool isv = i + NB >= nbp;
        load_batch<D, U>(isv ? vb : kb, isv ? vsb : ksb, (isv ? i + NB - nbp : i + NB) * U, n, j, lane, rr[b],
                         rs[b]);
      }
    }
    m = mloc;
    m = groups_max<LPT>(m);
    __builtin_amdgcn_wave_barrier();
    for (uint32_t v0 = 0; v0 < nbp; v0 += NB) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint32_t i = v0 + uint32_t(b);
        if (i < nb) accumulate_batch<D, BF16H, U>(rr[b], rs[b], i * U, n, j, lane, m, s_lds, z, out.acc);
        load_batch<D, U>(vb, vsb, (i + NB) * U, n, j, lane, rr[b], rs[b]);  // past the end on the last ring
      }
    }
  }
  // Each token's p was added once, by its owning lane: sum over the wave.
  z = wave_sum(z);
  reduce_scatter_groups<LPT, 16>(out.acc, lane);
  out.m = m;
  out.z = z;
}

template <int D, bool BF16H, int NB>
__device__ __forceinline__ void decode_body(const ppk::DecodeArgs& a) {
  constexpr int LPT = D / 16;
  constexpr int EPL = D / ppk::kWave;
  PPK_CLK_DECL;
  PPK_CLK(0);
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  // The wave index is uniform: in a scalar register, every quantity derived
  // from it (the wave's range, its length, its batch counts) is too, and the
  // stream's loop and batch conditions become scalar branches.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int c = lane % LPT;
  // Blocks are numbered group-major: consecutive blocks belong to different
  // rows, so the empty tail groups of short rows (ragged batches) spread over
  // the CUs instead of leaving some CUs with only live blocks.
  const uint32_t row = blockIdx.x % a.rows;
  const uint32_t group = blockIdx.x / a.rows;
  const uint32_t S = a.split_tokens;
  const uint32_t p = a.past[row / a.heads];
  const uint64_t cover = uint64_t(a.ngroups) * W * S;
  const bool valid = p <= a.capacity && uint64_t(p) <= cover;

  // Everything the wave reads before its stream is requested first, in one
  // round trip: q, the current token (wave 0 of a block that covers its
  // row), the new K/V row of the fused commit (waves 0 and 1 of group 0) and
  // the stream's first two K batches, clamped to the arena (not to the
  // row's length, which arrives with them). The commit and the current
  // token's score then run while the K batches are in flight. Measured at
  // B=32 x 8192 tokens against committing first and loading the stream after
  // the length: D=64 94.8 -> 91.6 us, D=128 165.5 -> 165.0 us, bitwise the
  // same output. The slot the commit writes is past every wave's length, so
  // the speculative reads of it are masked. The host turns this off (a.speculate
  // = 0) when it knows many waves have no history (ragged host lengths, or
  // waves past the span): their speculative reads would be wasted bandwidth
  // (config 4: 9 % more HBM traffic than the history, 18.7 -> 18.3 us without).
  float qr[16];
  load_vec<16>(a.q, size_t(row) * D + size_t(c) * 16, a.q_dtype, qr);
  const bool final_out = a.ngroups == 1;
  float s_cur = -INFINITY;
  float sv[EPL], kv[16];
  if (final_out && wave == 0) {
    load_vec<16>(a.sk, size_t(row) * D + size_t(c) * 16, a.scratch_dtype, kv);
    load_vec<EPL>(a.sv, size_t(row) * D + size_t(lane) * EPL, a.scratch_dtype, sv);
  }
  const bool kw = a.append && group == 0 && wave == 0;
  const bool vw = a.append && group == 0 && wave == (W > 1 ? 1 : 0);
  float kx[EPL], vx[EPL];
  if (kw) load_vec<EPL>(a.k_new, size_t(row) * D + size_t(lane) * EPL, a.new_dtype, kx);
  if (vw) load_vec<EPL>(a.v_new, size_t(row) * D + size_t(lane) * EPL, a.new_dtype, vx);
  const uint32_t begin = (group * W + wave) * S;
  const uint32_t nspec = (a.speculate && begin < a.capacity) ? min(S, a.capacity - begin) : 0u;
  constexpr int TPL = ppk::kWave / LPT;
  const bool pre = nspec > uint32_t(8 * TPL);  // the wave takes a streamed (not short-window) path
  u4 rr[NB][4];
  float rs[NB];
  if (pre) {
    const size_t tok0 = size_t(row) * a.capacity + begin;
    const int j = lane / LPT;
#pragma unroll
    for (int b = 0; b < NB; ++b)
      load_batch<D, 4>(a.k + tok0 * D + size_t(c) * 16, a.ks + tok0, uint32_t(b) * 4, nspec, j, lane, rr[b], rs[b]);
  }
  PPK_CLK(1);
  // A length within the caller's span that the plan does not cover: the plan
  // was sized from a stale host copy of the lengths (the row gives NaN).
  if (kw && lane == 0 && a.flags && p <= a.capacity && p <= a.span && uint64_t(p) > cover) atomicOr(a.flags, 4u);
  if (kw || vw) {
    if (p >= a.capacity) {
      if (lane == 0 && a.flags) atomicOr(a.flags, 2u);
    } else {
      const size_t slot = size_t(row) * a.capacity + p;
      if (kw) quantize_values<D>(kx, a.k + slot * D, a.ks + slot, a.flags, lane);
      if (vw) quantize_values<D>(vx, a.v + slot * D, a.vs + slot, a.flags, lane);
    }
  }
  if (final_out && wave == 0) s_cur = current_score<D>(a, kv, qr);
  PPK_CLK_AFTER(2, p);
  const uint32_t n = (valid && begin < p) ? min(S, p - begin) : 0u;
  WavePartial part;
  wave_attention<D, BF16H, NB>(a, row, begin, n, nspec, qr, lds + size_t(wave) * S, lane, part, pre, rr, rs);
  PPK_CLK(4);
#ifdef PPK_WAVE_CLOCK
  clk_[3] = part.t_first;
#endif

  // Combine the block's waves through LDS (the staging area is reused).
  // Record of wave w at mrg + w * R: m, z, 2 pad floats, y[D] (16-byte aligned).
  constexpr int R = D + 4;
  __syncthreads();
  float* mrg = lds;
  {
    const int ch = c * 16 + scatter_base<LPT, 16>(lane);
#pragma unroll
    for (int e = 0; e < EPL; ++e) mrg[wave * R + 4 + ch + e] = part.acc[e];
  }
  if (lane == 0) {
    mrg[wave * R] = part.m;
    mrg[wave * R + 1] = part.z;
  }
  __syncthreads();
  PPK_CLK(5);
  if (wave != 0) {
    PPK_CLK_RECORD(a, ppk::kWaveClockDecode, blockIdx.x, uint32_t(wave));
    return;
  }

  float m = s_cur;
  for (int w = 0; w < W; ++w) m = fmaxf(m, mrg[w * R]);
  float y[EPL], zsum = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) y[e] = 0.f;
  for (int w = 0; w < W; ++w) {
    const float wt = mrg[w * R] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrg[w * R] - m);
    zsum = fmaf(wt, mrg[w * R + 1], zsum);
#pragma unroll
    for (int e = 0; e < EPL; ++e) y[e] = fmaf(wt, mrg[w * R + 4 + lane * EPL + e], y[e]);
  }
  if (final_out) {
    const float wc = __builtin_amdgcn_exp2f(s_cur - m);
    zsum += wc;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float o = valid ? fmaf(wc, sv[e], y[e]) / zsum : __builtin_nanf("");
      store_elem(a.out, size_t(row) * D + size_t(lane) * EPL + e, a.out_dtype, o);
    }
  } else {
    const size_t rec = size_t(row) * a.ngroups + group;
#pragma unroll
    for (int e = 0; e < EPL; ++e) a.part_y[rec * D + size_t(lane) * EPL + e] = y[e];
    if (lane == 0) {
      a.part_mz[rec * 2] = m;
      a.part_mz[rec * 2 + 1] = zsum;
    }
  }
  PPK_CLK(6);
  PPK_CLK_RECORD(a, ppk::kWaveClockDecode, blockIdx.x, 0u);
}

// ---------------------------------------------------------------------------
// Kernel 2b: merge. One wave per row: scores the current (unquantised) token,
// combines it with every split's (m, z, y) by log-sum-exp weights, divides.
// Rows with past > capacity (or beyond the launched coverage) give NaN.
// ---------------------------------------------------------------------------
// Log-sum-exp combine of one row's `nsplits` partial records, one wave: the
// combined max m (at least m0), the sum z of 2^(m_s - m) z_s, and y for this
// lane's D/64 channels, sum_s 2^(m_s - m) y_s, added in split order. Lane s
// loads record s's (m, z); the y rows load eight splits at a time with all
// eight loads issued before the first use, so the chain costs one memory
// round trip per eight splits instead of one per split.
template <int D, class CurrentScore>
__device__ __forceinline__ void combine_records(const float* mz, const float* py, uint32_t nsplits, int lane,
                                                CurrentScore current_score, float& m, float& z,
                                                float (&y)[D / ppk::kWave]) {
  constexpr int EPL = D / ppk::kWave;
  // Everything that does not depend on the max is requested first, in one
  // round trip: the y rows of the first sixteen splits, the (m, z) pairs of
  // the first 64 splits (kept in registers for the weights), and then
  // whatever current_score() loads before it returns the extra score that
  // joins the max (-inf for none).
  float first[16][EPL];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t si = min(uint32_t(k), nsplits - 1);  // clamp: always a loaded record
#pragma unroll
    for (int e = 0; e < EPL; ++e) first[k][e] = py[size_t(si) * D + size_t(lane) * EPL + e];
  }
  const uint32_t s_first = min(uint32_t(lane), nsplits - 1);
  const float m_first = uint32_t(lane) < nsplits ? mz[2 * s_first] : -INFINITY;
  const float z_first = uint32_t(lane) < nsplits ? mz[2 * s_first + 1] : 0.f;
  float mm = m_first;
  for (uint32_t s = lane + ppk::kWave; s < nsplits; s += ppk::kWave) mm = fmaxf(mm, mz[2 * s]);
  mm = fmaxf(mm, current_score());
  m = wave_max(mm);
  z = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) y[e] = 0.f;
  for (uint32_t s0 = 0; s0 < nsplits; s0 += ppk::kWave) {
    const uint32_t s = s0 + uint32_t(lane);
    float ms = m_first, zs = z_first;
    if (s0 != 0) {
      ms = s < nsplits ? mz[2 * s] : -INFINITY;
      zs = s < nsplits ? mz[2 * s + 1] : 0.f;
    }
    const float w = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - m);
    z = fmaf(w, zs, z);
    const uint32_t cnt = min(uint32_t(ppk::kWave), nsplits - s0);
    for (uint32_t i = 0; i < cnt; i += 8) {
      float v[8][EPL];
      if (s0 == 0 && i < 16) {
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
          for (int e = 0; e < EPL; ++e) v[k][e] = i == 0 ? first[k][e] : first[8 + k][e];
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t si = s0 + min(i + uint32_t(k), cnt - 1);  // clamp: always a loaded record
#pragma unroll
          for (int e = 0; e < EPL; ++e) v[k][e] = py[size_t(si) * D + size_t(lane) * EPL + e];
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // Record i + k's weight sits in that lane (a uniform index): one readlane, no LDS.
        const float wk = i + uint32_t(k) < cnt
                             ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), int(i) + k))
                             : 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) y[e] = fmaf(wk, v[k][e], y[e]);
      }
    }
  }
  z = wave_sum(z);
}

template <int D>
__device__ __forceinline__ void attn_merge_body(const ppk::MergeArgs& a) {
  constexpr int EPL = D / ppk::kWave;
  PPK_CLK_DECL;
  PPK_CLK(0);
  const int lane = threadIdx.x;
  const uint32_t row = blockIdx.x;

  float sv[EPL];
  float s_cur = -INFINITY;
  const size_t base = size_t(row) * D + size_t(lane) * EPL;
  // The current token (q . sk, and sv): loaded after the records are requested.
  auto current = [&]() {
    float qv[EPL], kv[EPL];
    load_vec<EPL>(a.q, base, a.q_dtype, qv);
    load_vec<EPL>(a.sk, base, a.scratch_dtype, kv);
    load_vec<EPL>(a.sv, base, a.scratch_dtype, sv);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) d = fmaf(qv[e], kv[e], d);
    s_cur = wave_sum(d) * a.scale_log2;
    return s_cur;
  };
  float m, zsum, y[EPL];
  combine_records<D>(a.part_mz + size_t(row) * a.nsplits * 2, a.part_y + size_t(row) * a.nsplits * D, a.nsplits,
                     lane, current, m, zsum, y);
  PPK_CLK_AFTER(1, y[0]);
  // The row's length is first needed here: read after the records went out
  // (deciding validity up front would hold every record load back by the
  // length's round trip).
  const uint32_t p = a.past[row / a.heads];
  const bool valid = p <= a.capacity && uint64_t(p) <= uint64_t(a.nsplits) * a.split_tokens;
  const float wc = __builtin_amdgcn_exp2f(s_cur - m);
  zsum += wc;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float o = valid ? fmaf(wc, sv[e], y[e]) / zsum : __builtin_nanf("");
    store_elem(a.out, base + e, a.out_dtype, o);
  }
  PPK_CLK(2);
  PPK_CLK_RECORD(a, ppk::kWaveClockMerge, blockIdx.x, 0u);
}

// ---------------------------------------------------------------------------
// Kernel 2c: decode attention over a balanced work list (ragged batches). The
// per-row plan above gives every row the same number of blocks, sized for
// the longest row, so in a ragged batch the CUs holding long rows run on
// while the others idle. Here the host, from its copy of the lengths, cuts
// the live history into units of at most Q tokens, each inside one row (row
// r of len_r tokens is max(1, ceil(len_r / Q)) units, Q = max(ceil(T /
// (waves - rows)), 64) for T live tokens in all, so the units fit the
// waves: sum <= T / Q + rows <= waves), and wave i takes unit i: no unit
// exceeds the mean share by more than waves / (waves - rows). The table
// travels in the kernel arguments, so every wave issues all of its loads at
// once, the device lengths among them (they are compared with the table
// before anything is written). A row of one unit is finished by its wave
// (current token included); the units of a longer row leave log-sum-exp
// records that the balanced merge kernel joins.
//
// A unit is streamed as (K, V) pairs of batches through a window of two
// pairs in registers with an online softmax (running max per token group,
// one rescale per batch). Measured against four pairs and one, and against
// the per-row kernel's two-phase stream inside the same assignment, on
// configs 3 and 4 and ragged batches of 16 to 64 sequences: two pairs and the
// two-phase stream tie, four pairs is 2-12 % slower.
// ---------------------------------------------------------------------------
// One (K, V) batch pair of a unit under the online softmax. Token group j
// (the LPT lanes holding one token of each tile) keeps its own running max m,
// sum z and 16-channel accumulator: the batch's four scores are formed, the
// state is rescaled once to the new max, then each tile's V codes are added
// with weight 2^(s - m) * vscale.
template <int D, bool BF16H>
__device__ __forceinline__ void online_pair(const u4 (&kraw)[4], const u4 (&vraw)[4], float ks_lane, float vs_lane,
                                            uint32_t t0, uint32_t n, int j, const float (&qr)[16], const QInt& qi,
                                            float sl2, float& m, float& z, float (&acc)[16]) {
  constexpr int LPT = D / 16;
  constexpr int TPL = ppk::kWave / LPT;
  float s[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t tok = (t0 + u) * TPL + j;
    const float kscale = __shfl(ks_lane, u * TPL + j);
    float sc;
    if constexpr (BF16H) {
      float d = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          float e0, e1;
          round_bf16_pair(sbyte(kraw[u][w], k) * kscale, sbyte(kraw[u][w], k + 1) * kscale, e0, e1);
          d = fmaf(qr[4 * w + k], e0, d);
          d = fmaf(qr[4 * w + k + 1], e1, d);
        }
      sc = group_sum<LPT>(d) * sl2;
    } else {
      int sh = 0, s1 = 0, s2 = 0, slo = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        sh = __builtin_amdgcn_sdot4(int(kraw[u][w]), qi.hi[w], sh, false);
        s1 = __builtin_amdgcn_sdot4(int(kraw[u][w]), qi.m1[w], s1, false);
        s2 = __builtin_amdgcn_sdot4(int(kraw[u][w]), qi.m2[w], s2, false);
        slo = __builtin_amdgcn_sdot4(int(kraw[u][w]), qi.lo[w], slo, false);
      }
      const int hm = group_sum_i32<LPT>(sh * 128 + s1);
      const int lm = group_sum_i32<LPT>(s2 * 128 + slo);
      sc = fmaf(float(hm), 16384.f, float(lm)) * (kscale * sl2);
    }
    s[u] = tok < n ? sc : -INFINITY;
  }
  const float mb = fmaxf(fmaxf(m, fmaxf(s[0], s[1])), fmaxf(s[2], s[3]));
  const float f = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mb);
  z *= f;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] *= f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float pr = s[u] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s[u] - mb);
    z += pr;
    const float vscale = __shfl(vs_lane, u * TPL + j);
    if constexpr (BF16H) {
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int k = 0; k < 4; k += 2) {
          float e0, e1;
          round_bf16_pair(sbyte(vraw[u][w], k) * vscale, sbyte(vraw[u][w], k + 1) * vscale, e0, e1);
          acc[4 * w + k] = fmaf(pr, e0, acc[4 * w + k]);
          acc[4 * w + k + 1] = fmaf(pr, e1, acc[4 * w + k + 1]);
        }
    } else {
      const float wgt = pr * vscale;
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[4 * w + k] = fmaf(wgt, sbyte(vraw[u][w], k), acc[4 * w + k]);
    }
  }
  m = mb;
}

// Streams tokens [begin, begin + n) of one row (n >= 1) through the window
// of two (K, V) pairs; returns the wave's partial (m, z in every lane, the
// 16-channel sums in lanes j == 0), as wave_attention does. early() runs
// once the window's first loads are in flight (work whose own loads were
// issued before, so that waiting for them does not hold the window back).
template <int D, bool BF16H, class Early>
__device__ __forceinline__ void wave_attention_window(const ppk::DecodeArgs& a, uint32_t row, uint32_t begin,
                                                      uint32_t n, const float (&qr)[16], int lane,
                                                      WavePartial& out, Early early) {
  constexpr int LPT = D / 16;
  constexpr int TPL = ppk::kWave / LPT;
  constexpr int U = 4, NP = 2;
  const int j = lane / LPT;
  const int c = lane % LPT;
  const size_t tok0 = size_t(row) * a.capacity + begin;
  const uint8_t* kb = a.k + tok0 * D + size_t(c) * 16;
  const uint8_t* vb = a.v + tok0 * D + size_t(c) * 16;
  const float* ksb = a.ks + tok0;
  const float* vsb = a.vs + tok0;
  const uint32_t nb = (n + U * TPL - 1) / (U * TPL);  // batches per phase
  u4 kr[NP][U], vr[NP][U];
  float ksl[NP], vsl[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    if (uint32_t(p) < nb) {  // uniform per wave
      load_batch<D, U>(kb, ksb, uint32_t(p) * U, n, j, lane, kr[p], ksl[p]);
      load_batch<D, U>(vb, vsb, uint32_t(p) * U, n, j, lane, vr[p], vsl[p]);
    }
  }
  QInt qi{};
  float sl2 = a.scale_log2;
  if constexpr (!BF16H) {
    qi = quantize_query<LPT>(qr);
    sl2 *= qi.unscale;
  }
  early();
  float m = -INFINITY, z = 0.f, acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  for (uint32_t b0 = 0; b0 < nb; b0 += NP) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const uint32_t bi = b0 + uint32_t(p);
      if (bi < nb) {  // uniform per wave
        // Scales of tokens at or past n are never used (their scores are -inf).
        online_pair<D, BF16H>(kr[p], vr[p], ksl[p], vsl[p], bi * U, n, j, qr, qi, sl2, m, z, acc);
        if (bi + NP < nb) {
          load_batch<D, U>(kb, ksb, (bi + NP) * U, n, j, lane, kr[p], ksl[p]);
          load_batch<D, U>(vb, vsb, (bi + NP) * U, n, j, lane, vr[p], vsl[p]);
        }
      }
    }
  }
  // Join the token groups: common max, then sums across groups.
  float mm = m;
  mm = groups_max<LPT>(mm);
  const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mm);
  z *= w;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] *= w;
  z = groups_reduce<LPT>(z, [](float a, float b) { return a + b; });
  reduce_scatter_groups<LPT, 16>(acc, lane);
  out.m = mm;
  out.z = z;
#pragma unroll
  for (int i = 0; i < 16; ++i) out.acc[i] = acc[i];
}

// The table's sequence holding unit `unit` (< units_total): the last b with
// first[b] <= unit. A uniform binary search over the kernel arguments.
__device__ __forceinline__ uint32_t flat_sequence(const ppk::FlatTable& t, uint32_t unit) {
  uint32_t lo = 0, hi = t.batch - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi + 1) / 2;
    if (t.first[mid] <= unit) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <int D, bool BF16H>
__device__ __forceinline__ void decode_flat_body(const ppk::DecodeFlatArgs& fa) {
  const ppk::DecodeArgs& a = fa.d;
  const ppk::FlatTable& t = fa.t;
  constexpr int LPT = D / 16;
  constexpr int EPL = D / ppk::kWave;
  const int lane = threadIdx.x & 63;
  const uint32_t W = blockDim.x >> 6;
  const uint32_t wid = blockIdx.x * W + (threadIdx.x >> 6);
  const int c = lane % LPT;

  // Append job (a decode step): wave q < 2 rows quantises tensor q & 1 of
  // row q >> 1 into slot past[b] (the device value) of the arenas. Its loads
  // are issued first, beside everything else this wave reads.
  const bool append = a.append && wid < 2 * a.rows;  // uniform per wave (the host keeps waves >= 2 rows)
  const uint32_t arow = wid >> 1;
  float ax[EPL];
  uint32_t ap = 0;
  if (append) {
    ap = a.past[arow / a.heads];
    load_vec<EPL>((wid & 1u) ? a.v_new : a.k_new, size_t(arow) * D + size_t(lane) * EPL, a.new_dtype, ax);
  }
  const bool work = wid < t.units_total;  // uniform per wave
  uint32_t b = 0, units = 1, len = 0, row = 0, slot = 0, t0 = 0, n = 0, pdev = 0;
  float qr[16], kv[16], sv[EPL];
  const int ch = c * 16 + scatter_base<LPT, 16>(lane);  // this lane's output channels: ch .. ch + EPL - 1
  if (work) {
    b = flat_sequence(t, wid);
    units = t.units[b];
    len = t.len[b];
    const uint32_t k = wid - t.first[b];
    const uint32_t h = k / units;
    slot = k - h * units;
    row = b * a.heads + h;
    t0 = slot * t.share;
    n = len > t0 ? min(t.share, len - t0) : 0u;
    pdev = a.past[b];
    if (n > 0) load_vec<16>(a.q, size_t(row) * D + size_t(c) * 16, a.q_dtype, qr);
    if (units == 1) {  // the whole row: its current token too
      if (n > 0) load_vec<16>(a.sk, size_t(row) * D + size_t(c) * 16, a.scratch_dtype, kv);
      load_vec<EPL>(a.sv, size_t(row) * D + size_t(ch), a.scratch_dtype, sv);
    }
  }
  auto commit = [&]() {
    if (!append) return;
    if (ap >= a.capacity) {
      if (lane == 0 && a.flags) atomicOr(a.flags, 2u);
    } else {
      const size_t dst = size_t(arow) * a.capacity + ap;
      if (wid & 1u) quantize_values<D>(ax, a.v + dst * D, a.vs + dst, a.flags, lane);
      else quantize_values<D>(ax, a.k + dst * D, a.ks + dst, a.flags, lane);
    }
  };
  if (!work) {
    commit();
    return;
  }
  // The row is valid when the host's length is in range and the device agrees.
  const uint32_t phost = t.past[b];
  const bool host_ok = phost <= a.capacity && phost <= a.span;
  WavePartial part;
  part.m = -INFINITY;
  part.z = 0.f;
  float s_cur = -INFINITY;
  if (n > 0) {
    auto early = [&]() {  // with the unit's first loads in flight
      commit();
      if (units == 1) s_cur = current_score<D>(a, kv, qr);
    };
    wave_attention_window<D, BF16H>(a, row, t0, n, qr, lane, part, early);
  } else {
    commit();
  }
  const bool fresh = pdev == phost;
  if (!fresh && lane == 0 && a.flags) atomicOr(a.flags, 4u);
  if (units == 1) {
    const bool valid = fresh && host_ok;
    const float m = fmaxf(part.m, s_cur);
    const float wp = n > 0 ? __builtin_amdgcn_exp2f(part.m - m) : 0.f;
    const float wc = n > 0 ? __builtin_amdgcn_exp2f(s_cur - m) : 1.f;
    const float zsum = n > 0 ? fmaf(wp, part.z, wc) : 1.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float o = valid ? fmaf(wc, sv[e], n > 0 ? wp * part.acc[e] : 0.f) / zsum : __builtin_nanf("");
      store_elem(a.out, size_t(row) * D + size_t(ch + e), a.out_dtype, o);
    }
  } else if (slot < a.ngroups) {  // always, by the host's count of slots
    const size_t rec = size_t(row) * a.ngroups + slot;
#pragma unroll
    for (int e = 0; e < EPL; ++e) a.part_y[rec * D + size_t(ch + e)] = part.acc[e];
    if (lane == 0) {
      a.part_mz[rec * 2] = part.m;
      a.part_mz[rec * 2 + 1] = part.z;
    }
  }
}

// Balanced merge: one wave per row of two or more units (the others were
// written by the decode launch): joins the row's records and the current
// token, or gives NaN when the row is invalid or the device length differs
// from the table's.
template <int D>
__device__ __forceinline__ void attn_merge_flat_body(const ppk::MergeFlatArgs& fa) {
  const ppk::MergeArgs& a = fa.m;
  const ppk::FlatTable& t = fa.t;
  constexpr int EPL = D / ppk::kWave;
  const int lane = threadIdx.x;
  const uint32_t row = blockIdx.x;
  const uint32_t b = row / a.heads;
  const uint32_t units = t.units[b];
  if (units < 2) return;  // uniform per wave
  const uint32_t phost = t.past[b];
  const uint32_t pdev = a.past[b];
  const size_t base = size_t(row) * D + size_t(lane) * EPL;
  float sv[EPL];
  float s_cur = -INFINITY;
  auto current = [&]() {
    float qv[EPL], kv[EPL];
    load_vec<EPL>(a.q, base, a.q_dtype, qv);
    load_vec<EPL>(a.sk, base, a.scratch_dtype, kv);
    load_vec<EPL>(a.sv, base, a.scratch_dtype, sv);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) d = fmaf(qv[e], kv[e], d);
    s_cur = wave_sum(d) * a.scale_log2;
    return s_cur;
  };
  float m, zsum, y[EPL];
  combine_records<D>(a.part_mz + size_t(row) * a.nsplits * 2, a.part_y + size_t(row) * a.nsplits * D,
                     min(units, a.nsplits), lane, current, m, zsum, y);
  const bool valid = pdev == phost && phost <= a.capacity && phost <= a.span;
  const float wc = __builtin_amdgcn_exp2f(s_cur - m);
  zsum += wc;
#pragma unroll
  for (int e = 0; e < EPL; ++e)
    store_elem(a.out, base + e, a.out_dtype, valid ? fmaf(wc, sv[e], y[e]) / zsum : __builtin_nanf(""));
}

// ---------------------------------------------------------------------------
// Float-KV decode attention: the reference's non-int8 decode path
// (app/src/model/decode_attention.hip:9-66, fused_attention.rs:8-30) on the
// block geometry of the int8 kernel. K/V are stored bf16 or f32; row r attends
// its first n = lengths ? lengths[r / heads] : size tokens (the current token
// is already in the store) and gives NaN if n == 0 or n > span (max_length,
// or size).
//
// Lane layout: a lane holds one 16-byte chunk of a token, EPC = 8 (bf16) or 4
// (f32) channels; LPT = D / EPC lanes share a token and a wave-wide dwordx4
// load moves TPL = 64 / LPT whole tokens (1 KiB). Scores go to LDS in the
// log2 domain, exactly as in the int8 kernel, and phase V weights each token's
// chunk by p = 2^(s - m) broadcast from the lane that owns the token.
// ---------------------------------------------------------------------------
template <int LPT>
__device__ __forceinline__ float token_sum(float x) {
  if constexpr (LPT <= 16) {
    return group_sum<LPT>(x);
  } else {
    x = group_sum<16>(x);
    x += __shfl_xor(x, 16);
    if constexpr (LPT >= 64) x += __shfl_xor(x, 32);
    return x;
  }
}

template <bool BF16KV>
__device__ __forceinline__ void unpack_chunk(const u4& r, float (&x)[BF16KV ? 8 : 4]) {
  if constexpr (BF16KV) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      x[2 * w] = __uint_as_float(r[w] << 16);
      x[2 * w + 1] = __uint_as_float(r[w] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) x[w] = __uint_as_float(r[w]);
  }
}

template <int D, bool BF16KV>
struct FloatGeom {
  static constexpr int kElemBytes = BF16KV ? 2 : 4;
  static constexpr int kEpc = ppk::kLaneBytes / kElemBytes;  // channels per lane
  static constexpr int kLpt = D / kEpc;                       // lanes per token
  static constexpr int kTpl = ppk::kWave / kLpt;              // tokens per wave load
  static constexpr int kTokenBytes = D * kElemBytes;
  static_assert(kLpt >= 4 && kLpt <= ppk::kWave, "token must span 4..64 lanes");
};

template <int D, bool BF16KV, int U>
__device__ __forceinline__ void load_fbatch(const char* base, uint32_t t0, uint32_t n, int j, u4 (&raw)[U]) {
  using G = FloatGeom<D, BF16KV>;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t tc = min((t0 + u) * G::kTpl + j, n - 1);  // clamp: always in bounds
    raw[u] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(base + size_t(tc) * G::kTokenBytes));
  }
}

template <int D, bool BF16KV, int U>
__device__ __forceinline__ float fscore_batch(const u4 (&raw)[U], uint32_t t0, uint32_t n, int j, int c,
                                              const float (&qr)[FloatGeom<D, BF16KV>::kEpc], float sl2,
                                              float* s_lds, float mloc) {
  using G = FloatGeom<D, BF16KV>;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t tok = (t0 + u) * G::kTpl + j;
    float x[G::kEpc];
    unpack_chunk<BF16KV>(raw[u], x);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < G::kEpc; ++e) d = fmaf(qr[e], x[e], d);
    float sc = token_sum<G::kLpt>(d) * sl2;
    sc = tok < n ? sc : -INFINITY;
    mloc = fmaxf(mloc, sc);
    if (c == 0 && tok < n) s_lds[tok] = sc;
  }
  return mloc;
}

template <int D, bool BF16KV, int U>
__device__ __forceinline__ void faccumulate_batch(const u4 (&raw)[U], uint32_t t0, uint32_t n, int j, int lane,
                                                  float m, const float* s_lds, float& z,
                                                  float (&acc)[FloatGeom<D, BF16KV>::kEpc]) {
  using G = FloatGeom<D, BF16KV>;
  constexpr int TPB = U * G::kTpl;  // tokens per batch (<= 64)
  static_assert(TPB <= ppk::kWave, "one token per lane per batch");
  const uint32_t tl = t0 * G::kTpl + uint32_t(lane % TPB);
  const float e = __builtin_amdgcn_exp2f(s_lds[min(tl, n - 1)] - m);
  const float pr = (tl < n && lane < TPB) ? e : 0.f;
  z += pr;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float wgt = __shfl(pr, u * G::kTpl + j);
    float x[G::kEpc];
    unpack_chunk<BF16KV>(raw[u], x);
#pragma unroll
    for (int e = 0; e < G::kEpc; ++e) acc[e] = fmaf(wgt, x[e], acc[e]);
  }
}

template <int D, bool BF16KV>
struct FloatWavePartial {
  float m, z;
  // While streaming: this lane's chunk; at the end the wave's totals of channels
  // c * kEpc + scatter_base<kLpt, kEpc>(lane) + e in acc[e], e < D / 64.
  float acc[FloatGeom<D, BF16KV>::kEpc];
};

// One wave streams n tokens of a row from `begin`: phase K scores into LDS,
// phase V accumulation; A/B batches ping-pong, and the last phase-K
// iteration already fetches the first V batch.
template <int D, bool BF16KV>
__device__ __forceinline__ void fwave_attention(const ppk::FloatDecodeArgs& a, uint32_t row, uint32_t begin,
                                                uint32_t n, const float (&qr)[FloatGeom<D, BF16KV>::kEpc],
                                                float* s_lds, int lane, FloatWavePartial<D, BF16KV>& out) {
  using G = FloatGeom<D, BF16KV>;
  constexpr int U = 4;
  const int j = lane / G::kLpt;
  const int c = lane % G::kLpt;
  out.m = -INFINITY;
  out.z = 0.f;
#pragma unroll
  for (int i = 0; i < G::kEpc; ++i) out.acc[i] = 0.f;
  if (n == 0) return;  // uniform per wave

  const char* kb = static_cast<const char*>(a.k) +
                   (size_t(row) * a.k_stride + size_t(begin) * D) * G::kElemBytes + size_t(c) * ppk::kLaneBytes;
  const char* vb = static_cast<const char*>(a.v) +
                   (size_t(row) * a.v_stride + size_t(begin) * D) * G::kElemBytes + size_t(c) * ppk::kLaneBytes;
  const uint32_t ntiles = (n + G::kTpl - 1) / G::kTpl;
  const float sl2 = a.scale_log2;
  // Each wave takes its batches in a rotated order: it starts at batch rot of
  // its nb batches and wraps, and phase V follows the same order. Waves that
  // start at the same offset of rows a power of two apart (a store of 4096 or
  // 8192 tokens) otherwise move through the same HBM channels in step. rot is
  // a multiplicative hash of the wave's global index scaled into [0, nb) (no
  // division), uniform per wave, so the remapping is scalar work. Scores land
  // in LDS by token and phase V reads them by token, so only the order of
  // phase V's fp32 sums changes. Logical batches past nb (the padding to
  // whole ping-pong pairs) keep their place past the end, where loads clamp
  // and tokens are masked. Measured with bf16 stores of exactly the sequence
  // length (power-of-two strides): B=8 x 4096 D=64 30.0 -> 21.7 us, B=4 x
  // 4096 D=128 26.3 -> 21.7 us, B=16 x 1024 D=128 23.3 -> 20.1 us; B=32 x
  // 8192 D=128 310.5 -> 309.0 us. It costs where a few long rows stream one
  // wave per CU: 4 x 8192 + 28 x 512 tokens on the per-row plan 112.2 ->
  // 115.7 us (the balanced plan, which host lengths select, does not rotate).
  const uint32_t nb = (ntiles + U - 1) / U;
  const uint32_t wave_id = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
  const uint32_t rot = ((wave_id * 0x9E37u & 0xFFFFu) * nb) >> 16;
  auto ph = [&](uint32_t t) {  // logical first tile of a batch -> the tile it reads
    const uint32_t b = t / U;
    return b < nb ? (b + rot >= nb ? b + rot - nb : b + rot) * U : t;
  };

  u4 ra[U], rb[U];
  float mloc = -INFINITY;
  load_fbatch<D, BF16KV, U>(kb, ph(0), n, j, ra);
  for (uint32_t t0 = 0; t0 < ntiles; t0 += 2 * U) {
    load_fbatch<D, BF16KV, U>(kb, ph(t0 + U), n, j, rb);
    mloc = fscore_batch<D, BF16KV, U>(ra, ph(t0), n, j, c, qr, sl2, s_lds, mloc);
    const bool last = t0 + 2 * U >= ntiles;
    load_fbatch<D, BF16KV, U>(last ? vb : kb, last ? ph(0) : ph(t0 + 2 * U), n, j, ra);
    mloc = fscore_batch<D, BF16KV, U>(rb, ph(t0 + U), n, j, c, qr, sl2, s_lds, mloc);
  }
  float m = mloc;
  m = groups_max<G::kLpt>(m);
  __builtin_amdgcn_wave_barrier();

  float z = 0.f;
  for (uint32_t t0 = 0; t0 < ntiles; t0 += 2 * U) {
    load_fbatch<D, BF16KV, U>(vb, ph(t0 + U), n, j, rb);
    faccumulate_batch<D, BF16KV, U>(ra, ph(t0), n, j, lane, m, s_lds, z, out.acc);
    load_fbatch<D, BF16KV, U>(vb, ph(t0 + 2 * U), n, j, ra);
    faccumulate_batch<D, BF16KV, U>(rb, ph(t0 + U), n, j, lane, m, s_lds, z, out.acc);
  }
  z = wave_sum(z);
  reduce_scatter_groups<G::kLpt, G::kEpc>(out.acc, lane);
  out.m = m;
  out.z = z;
}

__device__ __forceinline__ uint32_t float_row_length(const uint32_t* lengths, uint32_t row, uint32_t heads,
                                                     uint32_t size) {
  return lengths ? lengths[row / heads] : size;
}

// The fused step's current token of row `row`, channels lane * EPL .. + EPL,
// rounded to the store's dtype (the value a stored token would hold).
template <int EPL, bool BF16KV>
__device__ __forceinline__ void load_current(const void* src, uint32_t row, uint32_t dtype, int lane,
                                             float (&x)[EPL]) {
  load_vec<EPL>(src, size_t(row) * (EPL * ppk::kWave) + size_t(lane) * EPL, dtype, x);
  if constexpr (BF16KV) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) x[e] = bf16_to_f32(f32_to_bf16_bits(x[e]));
  }
}

// The fused step's write of one current-token tensor of `row` at slot p of
// the store (or the overflow flag when the slot is past the store).
template <int EPL, bool BF16KV>
__device__ __forceinline__ void write_current(void* store, uint64_t stride, uint32_t row, uint32_t p, uint32_t size,
                                              const float (&x)[EPL], uint32_t* flags, int lane) {
  if (p >= size) {
    if (lane == 0 && flags) atomicOr(flags, 2u);
    return;
  }
  const size_t base = size_t(row) * stride + size_t(p) * (EPL * ppk::kWave) + size_t(lane) * EPL;
#pragma unroll
  for (int e = 0; e < EPL; ++e) store_elem(store, base + e, BF16KV ? kBF16 : kF32, x[e]);
}

template <int D, bool BF16KV, bool STEP>
__device__ __forceinline__ void fdecode_body(const ppk::FloatDecodeArgs& a) {
  using G = FloatGeom<D, BF16KV>;
  constexpr int EPL = D / ppk::kWave;
  extern __shared__ float lds[];
  const int lane = threadIdx.x & 63;
  // Uniform: the wave's range, length and loop bounds stay in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int c = lane % G::kLpt;
  // Blocks are numbered group-major: consecutive blocks belong to different
  // rows, so the empty tail groups of short rows (ragged batches) spread over
  // the CUs instead of leaving some CUs with only live blocks.
  const uint32_t row = blockIdx.x % a.rows;
  const uint32_t group = blockIdx.x / a.rows;
  const uint32_t S = a.split_tokens;
  // The stored tokens a row streams: lengths[b] (the step's current token
  // comes from k_new / v_new instead).
  const uint32_t len = float_row_length(a.lengths, row, a.heads, a.size);
  bool valid;
  if constexpr (STEP)
    valid = len < a.size && len + 1 <= a.span && uint64_t(len) <= uint64_t(a.ngroups) * W * S;
  else
    valid = len > 0 && len <= a.span && len <= a.size && uint64_t(len) <= uint64_t(a.ngroups) * W * S;

  float qr[G::kEpc];
  load_vec<G::kEpc>(a.q, size_t(row) * a.q_stride + size_t(c) * G::kEpc, a.q_dtype, qr);
  // The step: group 0's waves 0 and 1 write the current key and value at slot
  // len (never read here: every stream stops before it); wave 0 of a block
  // that finishes its row also folds the current token into the result.
  const bool final_out = a.ngroups == 1;
  const bool kw = STEP && group == 0 && wave == 0;
  const bool vw = STEP && group == 0 && wave == (W > 1 ? 1 : 0);
  const bool cur = STEP && final_out && wave == 0;
  float kcur[EPL], vcur[EPL], qcur[EPL];
  if (kw || cur) load_current<EPL, BF16KV>(a.k_new, row, a.new_dtype, lane, kcur);
  if (vw || cur) load_current<EPL, BF16KV>(a.v_new, row, a.new_dtype, lane, vcur);
  if (cur) load_vec<EPL>(a.q, size_t(row) * a.q_stride + size_t(lane) * EPL, a.q_dtype, qcur);
  // A stored length within the span that the plan does not cover: the plan
  // was sized from a stale host copy of the lengths (the row gives NaN).
  if (kw && lane == 0 && a.flags && len < a.size && len + 1 <= a.span && uint64_t(len) > uint64_t(a.ngroups) * W * S)
    atomicOr(a.flags, 4u);
  if (kw) write_current<EPL, BF16KV>(const_cast<void*>(a.k), a.k_stride, row, len, a.size, kcur, a.flags, lane);
  if (vw) write_current<EPL, BF16KV>(const_cast<void*>(a.v), a.v_stride, row, len, a.size, vcur, a.flags, lane);
  const uint32_t begin = (group * W + wave) * S;
  const uint32_t n = (valid && begin < len) ? min(S, len - begin) : 0u;
  FloatWavePartial<D, BF16KV> part;
  fwave_attention<D, BF16KV>(a, row, begin, n, qr, lds + size_t(wave) * S, lane, part);

  // Combine the block's waves through LDS: record of wave w at mrg + w * R
  // holds m, z, 2 pad floats, y[D] (16-byte aligned).
  constexpr int R = D + 4;
  __syncthreads();
  float* mrg = lds;
  {
    const int ch = c * G::kEpc + scatter_base<G::kLpt, G::kEpc>(lane);
#pragma unroll
    for (int e = 0; e < EPL; ++e) mrg[wave * R + 4 + ch + e] = part.acc[e];
  }
  if (lane == 0) {
    mrg[wave * R] = part.m;
    mrg[wave * R + 1] = part.z;
  }
  __syncthreads();
  if (wave != 0) return;

  float m = -INFINITY;
  for (int w = 0; w < W; ++w) m = fmaxf(m, mrg[w * R]);
  float s_cur = -INFINITY;
  if (cur) {
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) d = fmaf(qcur[e], kcur[e], d);
    s_cur = wave_sum(d) * a.scale_log2;
    m = fmaxf(m, s_cur);
  }
  float y[EPL], zsum = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) y[e] = 0.f;
  for (int w = 0; w < W; ++w) {
    const float wt = mrg[w * R] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mrg[w * R] - m);
    zsum = fmaf(wt, mrg[w * R + 1], zsum);
#pragma unroll
    for (int e = 0; e < EPL; ++e) y[e] = fmaf(wt, mrg[w * R + 4 + lane * EPL + e], y[e]);
  }
  if (cur) {
    const float wc = __builtin_amdgcn_exp2f(s_cur - m);
    zsum += wc;
#pragma unroll
    for (int e = 0; e < EPL; ++e) y[e] = fmaf(wc, vcur[e], y[e]);
  }
  if (a.ngroups == 1) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float o = (valid && zsum > 0.f) ? y[e] / zsum : __builtin_nanf("");
      store_elem(a.out, size_t(row) * D + size_t(lane) * EPL + e, a.out_dtype, o);
    }
  } else {
    const size_t rec = size_t(row) * a.ngroups + group;
#pragma unroll
    for (int e = 0; e < EPL; ++e) a.part_y[rec * D + size_t(lane) * EPL + e] = y[e];
    if (lane == 0) {
      a.part_mz[rec * 2] = m;
      a.part_mz[rec * 2 + 1] = zsum;
    }
  }
}

// Cross-group merge of the float path (pp_attention_merge,
// decode_attention.hip:55-66): one wave per row, log-sum-exp weights, NaN for
// invalid rows or a non-positive total weight.
// The fused step's current token in a merge: q . k_new (rounded to the
// store's dtype) as a log2-domain score, with v_new kept for the fold.
template <int D>
__device__ __forceinline__ float merge_current(const ppk::FloatMergeArgs& a, uint32_t row, int lane,
                                               float (&vcur)[D / ppk::kWave]) {
  constexpr int EPL = D / ppk::kWave;
  float qv[EPL], kv[EPL];
  load_vec<EPL>(a.q, size_t(row) * a.q_stride + size_t(lane) * EPL, a.q_dtype, qv);
  load_vec<EPL>(a.k_new, size_t(row) * D + size_t(lane) * EPL, a.new_dtype, kv);
  load_vec<EPL>(a.v_new, size_t(row) * D + size_t(lane) * EPL, a.new_dtype, vcur);
  if (a.kv_bf16) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      kv[e] = bf16_to_f32(f32_to_bf16_bits(kv[e]));
      vcur[e] = bf16_to_f32(f32_to_bf16_bits(vcur[e]));
    }
  }
  float d = 0.f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) d = fmaf(qv[e], kv[e], d);
  return wave_sum(d) * a.scale_log2;
}

template <int D>
__device__ __forceinline__ void fmerge_body(const ppk::FloatMergeArgs& a) {
  constexpr int EPL = D / ppk::kWave;
  const int lane = threadIdx.x;
  const uint32_t row = blockIdx.x;
  float m, zsum, y[EPL], vcur[EPL];
  float s_cur = -INFINITY;
  auto current = [&]() {
    if (a.step) s_cur = merge_current<D>(a, row, lane, vcur);
    return s_cur;
  };
  combine_records<D>(a.part_mz + size_t(row) * a.nsplits * 2, a.part_y + size_t(row) * a.nsplits * D, a.nsplits,
                     lane, current, m, zsum, y);
  // The row's length is first needed here: read after the records went out
  // (deciding validity up front would hold every record load back by the
  // length's round trip).
  const uint32_t len = float_row_length(a.lengths, row, a.heads, a.size);
  const bool cover = uint64_t(len) <= uint64_t(a.nsplits) * a.split_tokens;
  const bool valid = a.step ? (len < a.size && len + 1 <= a.span && cover)
                            : (len > 0 && len <= a.span && len <= a.size && cover);
  if (a.step) {
    const float wc = __builtin_amdgcn_exp2f(s_cur - m);
    zsum += wc;
#pragma unroll
    for (int e = 0; e < EPL; ++e) y[e] = fmaf(wc, vcur[e], y[e]);
  }
  const size_t base = size_t(row) * D + size_t(lane) * EPL;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float o = (valid && zsum > 0.f) ? y[e] / zsum : __builtin_nanf("");
    store_elem(a.out, base + e, a.out_dtype, o);
  }
}

// ---------------------------------------------------------------------------
// Float-KV decode over the balanced work list (ragged batches with the host's
// copy of the lengths): the int8 path's table (units of at most Q tokens of
// one row, one unit per wave), each unit streamed as (K, V) batch
// pairs through a window of two pairs with an online softmax. A row of one
// unit is finished in the decode launch; longer rows leave one record per
// unit for ppk_fmerge_flat_d*. A row whose host length lies outside
// (0, min(size, max_length)], or whose device lengths[b] differs from the
// table's, gives NaN.
// ---------------------------------------------------------------------------
// One (K, V) batch pair under the online softmax: token group j (the lanes
// of one token of each tile) keeps its running max m, sum z and channel
// accumulators; the batch's four scores, one rescale, then the V rows.
template <int D, bool BF16KV>
__device__ __forceinline__ void fonline_pair(const u4 (&kraw)[4], const u4 (&vraw)[4], uint32_t t0, uint32_t n, int j,
                                             const float (&qr)[FloatGeom<D, BF16KV>::kEpc], float sl2, float& m,
                                             float& z, float (&acc)[FloatGeom<D, BF16KV>::kEpc]) {
  using G = FloatGeom<D, BF16KV>;
  float s[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t tok = (t0 + u) * G::kTpl + j;
    float x[G::kEpc];
    unpack_chunk<BF16KV>(kraw[u], x);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < G::kEpc; ++e) d = fmaf(qr[e], x[e], d);
    const float sc = token_sum<G::kLpt>(d) * sl2;
    s[u] = tok < n ? sc : -INFINITY;
  }
  const float mb = fmaxf(fmaxf(m, fmaxf(s[0], s[1])), fmaxf(s[2], s[3]));
  const float f = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mb);
  z *= f;
#pragma unroll
  for (int e = 0; e < G::kEpc; ++e) acc[e] *= f;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float pr = s[u] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s[u] - mb);
    z += pr;
    float x[G::kEpc];
    unpack_chunk<BF16KV>(vraw[u], x);
#pragma unroll
    for (int e = 0; e < G::kEpc; ++e) acc[e] = fmaf(pr, x[e], acc[e]);
  }
  m = mb;
}

// Streams tokens [begin, begin + n) of one row (n >= 1) through the window
// of two (K, V) pairs; the partial (m, z in every lane, the channel sums in
// lanes j == 0), as fwave_attention returns it.
template <int D, bool BF16KV>
__device__ __forceinline__ void fwave_attention_window(const ppk::FloatDecodeArgs& a, uint32_t row, uint32_t begin,
                                                       uint32_t n, const float (&qr)[FloatGeom<D, BF16KV>::kEpc],
                                                       int lane, FloatWavePartial<D, BF16KV>& out) {
  using G = FloatGeom<D, BF16KV>;
  constexpr int U = 4, NP = 2;
  const int j = lane / G::kLpt;
  const int c = lane % G::kLpt;
  const char* kb = static_cast<const char*>(a.k) +
                   (size_t(row) * a.k_stride + size_t(begin) * D) * G::kElemBytes + size_t(c) * ppk::kLaneBytes;
  const char* vb = static_cast<const char*>(a.v) +
                   (size_t(row) * a.v_stride + size_t(begin) * D) * G::kElemBytes + size_t(c) * ppk::kLaneBytes;
  const uint32_t nb = (n + U * G::kTpl - 1) / (U * G::kTpl);  // batches per phase
  u4 kr[NP][U], vr[NP][U];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    if (uint32_t(p) < nb) {  // uniform per wave
      load_fbatch<D, BF16KV, U>(kb, uint32_t(p) * U, n, j, kr[p]);
      load_fbatch<D, BF16KV, U>(vb, uint32_t(p) * U, n, j, vr[p]);
    }
  }
  float m = -INFINITY, z = 0.f, acc[G::kEpc];
#pragma unroll
  for (int e = 0; e < G::kEpc; ++e) acc[e] = 0.f;
  for (uint32_t b0 = 0; b0 < nb; b0 += NP) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const uint32_t bi = b0 + uint32_t(p);
      if (bi < nb) {  // uniform per wave
        fonline_pair<D, BF16KV>(kr[p], vr[p], bi * U, n, j, qr, a.scale_log2, m, z, acc);
        if (bi + NP < nb) {
          load_fbatch<D, BF16KV, U>(kb, (bi + NP) * U, n, j, kr[p]);
          load_fbatch<D, BF16KV, U>(vb, (bi + NP) * U, n, j, vr[p]);
        }
      }
    }
  }
  float mm = m;
  mm = groups_max<G::kLpt>(mm);
  const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mm);
  z *= w;
#pragma unroll
  for (int e = 0; e < G::kEpc; ++e) acc[e] *= w;
  z = groups_reduce<G::kLpt>(z, [](float a, float b) { return a + b; });
  reduce_scatter_groups<G::kLpt, G::kEpc>(acc, lane);
  out.m = mm;
  out.z = z;
#pragma unroll
  for (int e = 0; e < G::kEpc; ++e) out.acc[e] = acc[e];
}

template <int D, bool BF16KV, bool STEP>
__device__ __forceinline__ void fdecode_flat_body(const ppk::FloatDecodeFlatArgs& fa) {
  const ppk::FloatDecodeArgs& a = fa.d;
  const ppk::FlatTable& t = fa.t;
  using G = FloatGeom<D, BF16KV>;
  const int lane = threadIdx.x & 63;
  // Wave w of block x takes unit w * blocks + x: the waves that share a CU
  // take units far apart in the list (rows of different lengths, idle waves
  // spread over the CUs), which evens the bytes each CU streams. Measured on
  // MI355X (H = 16, bf16, D = 128, against unit 4x + w): 8 sequences of 4096
  // tokens beside 24 of 1024, 87.5 -> 78.1 us; 4 of 8192 beside 28 of 512,
  // 68.9 -> 67.0 us; f32 1 of 8192 beside 31 of 256, 52.5 -> 48.0 us;
  // within 2 % elsewhere. (The int8 kernel keeps consecutive units per
  // block: this mapping did not help it.)
  const uint32_t wid = (threadIdx.x >> 6) * gridDim.x + blockIdx.x;
  if constexpr (STEP) {
    // The step's writes: wave q < 2 rows writes tensor q & 1 of row q >> 1 at
    // slot lengths[b] (the device value; every stream stops before it).
    if (wid < 2 * a.rows) {  // uniform per wave (the host keeps waves >= 2 rows)
      constexpr int EPL = D / ppk::kWave;
      const uint32_t arow = wid >> 1;
      const bool value = (wid & 1u) != 0;
      float x[EPL];
      load_current<EPL, BF16KV>(value ? a.v_new : a.k_new, arow, a.new_dtype, lane, x);
      write_current<EPL, BF16KV>(const_cast<void*>(value ? a.v : a.k), value ? a.v_stride : a.k_stride, arow,
                                 a.lengths[arow / a.heads], a.size, x, a.flags, lane);
    }
  }
  if (wid >= t.units_total) return;  // uniform per wave
  constexpr int EPL = D / ppk::kWave;
  const int c = lane % G::kLpt;
  const int ch = c * G::kEpc + scatter_base<G::kLpt, G::kEpc>(lane);  // this lane's output channels
  const uint32_t b = flat_sequence(t, wid);
  const uint32_t units = t.units[b];
  const uint32_t len = t.len[b];
  const uint32_t k = wid - t.first[b];
  const uint32_t h = k / units;
  const uint32_t slot = k - h * units;
  const uint32_t row = b * a.heads + h;
  const uint32_t t0 = slot * t.share;
  const uint32_t n = len > t0 ? min(t.share, len - t0) : 0u;
  const uint32_t ldev = a.lengths[b];
  // The step's current token, folded by the wave of a one-unit row (longer
  // rows: by the merge), in this kernel's lane layout and token arithmetic.
  const bool cur = STEP && units == 1;
  float qr[G::kEpc], kx[G::kEpc], vx[EPL];
  if (n > 0 || cur) load_vec<G::kEpc>(a.q, size_t(row) * a.q_stride + size_t(c) * G::kEpc, a.q_dtype, qr);
  if (cur) {
    load_vec<G::kEpc>(a.k_new, size_t(row) * D + size_t(c) * G::kEpc, a.new_dtype, kx);
    load_vec<EPL>(a.v_new, size_t(row) * D + size_t(ch), a.new_dtype, vx);
    if constexpr (BF16KV) {
#pragma unroll
      for (int e = 0; e < G::kEpc; ++e) kx[e] = bf16_to_f32(f32_to_bf16_bits(kx[e]));
#pragma unroll
      for (int e = 0; e < EPL; ++e) vx[e] = bf16_to_f32(f32_to_bf16_bits(vx[e]));
    }
  }
  FloatWavePartial<D, BF16KV> part;
  part.m = -INFINITY;
  part.z = 0.f;
#pragma unroll
  for (int e = 0; e < G::kEpc; ++e) part.acc[e] = 0.f;
  if (n > 0) fwave_attention_window<D, BF16KV>(a, row, t0, n, qr, lane, part);
  bool valid;
  if constexpr (STEP) {
    valid = ldev == t.past[b] && t.past[b] < a.size && t.past[b] + 1 <= a.span;
    // A device length that differs from the host copy the table was built
    // from: the row gives NaN, and a decode step says why in its flags.
    if (ldev != t.past[b] && lane == 0 && a.flags) atomicOr(a.flags, 4u);
  } else {
    valid = len > 0 && ldev == t.past[b];
  }
  if (cur) {
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < G::kEpc; ++e) d = fmaf(qr[e], kx[e], d);
    const float s_cur = token_sum<G::kLpt>(d) * a.scale_log2;
    const float m2 = fmaxf(part.m, s_cur);
    const float w1 = part.m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(part.m - m2);
    const float wc = __builtin_amdgcn_exp2f(s_cur - m2);
    part.z = fmaf(part.z, w1, wc);
#pragma unroll
    for (int e = 0; e < EPL; ++e) part.acc[e] = fmaf(part.acc[e], w1, wc * vx[e]);
  }
  if (units == 1) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float o = (valid && part.z > 0.f) ? part.acc[e] / part.z : __builtin_nanf("");
      store_elem(a.out, size_t(row) * D + size_t(ch + e), a.out_dtype, o);
    }
  } else if (slot < a.ngroups) {  // always, by the host's count of slots
    const size_t rec = size_t(row) * a.ngroups + slot;
#pragma unroll
    for (int e = 0; e < EPL; ++e) a.part_y[rec * D + size_t(ch + e)] = part.acc[e];
    if (lane == 0) {
      a.part_mz[rec * 2] = part.m;
      a.part_mz[rec * 2 + 1] = part.z;
    }
  }
}

// Merge of the float balanced work list: one wave per row of two or more
// units (the others were written by the decode launch).
template <int D>
__device__ __forceinline__ void fmerge_flat_body(const ppk::FloatMergeFlatArgs& fa) {
  const ppk::FloatMergeArgs& a = fa.m;
  const ppk::FlatTable& t = fa.t;
  constexpr int EPL = D / ppk::kWave;
  const int lane = threadIdx.x;
  const uint32_t row = blockIdx.x;
  const uint32_t b = row / a.heads;
  const uint32_t units = t.units[b];
  if (units < 2) return;  // uniform per wave
  const uint32_t ldev = a.lengths[b];
  float m, zsum, y[EPL], vcur[EPL];
  float s_cur = -INFINITY;
  auto current = [&]() {
    if (a.step) s_cur = merge_current<D>(a, row, lane, vcur);
    return s_cur;
  };
  combine_records<D>(a.part_mz + size_t(row) * a.nsplits * 2, a.part_y + size_t(row) * a.nsplits * D,
                     min(units, a.nsplits), lane, current, m, zsum, y);
  if (a.step) {
    const float wc = __builtin_amdgcn_exp2f(s_cur - m);
    zsum += wc;
#pragma unroll
    for (int e = 0; e < EPL; ++e) y[e] = fmaf(wc, vcur[e], y[e]);
  }
  const bool valid = a.step ? (ldev == t.past[b] && t.past[b] < a.size && t.past[b] + 1 <= a.span)
                            : (t.len[b] > 0 && ldev == t.past[b]);
  const size_t base = size_t(row) * D + size_t(lane) * EPL;
#pragma unroll
  for (int e = 0; e < EPL; ++e)
    store_elem(a.out, base + e, a.out_dtype, (valid && zsum > 0.f) ? y[e] / zsum : __builtin_nanf(""));
}

// ---------------------------------------------------------------------------
// CFG + Renyi effective-support sampler (app/src/inference/renyi_sample.hip:23-204,
// hip_sampling.rs:89-105). Per logical row: v = u + cfg (c - u) over the whole
// head (every column must be finite), legal candidates [start, start + count),
// H = log Z + max(0, log Z - log Z_alpha) / (alpha - 1) clamped to [0, ln count],
// support = clamp((u32)(exp(H) + 0.5), 1, count), rank = min((u32)(uniform *
// support), support - 1), token = the rank-th candidate by (value descending,
// index ascending).
//
// The arithmetic that decides support keeps the reference's order: 256
// strided partial sums of exp(v - m) and exp(alpha (v - m)) in candidate
// order, then the halving tree (steps 128, 64 through LDS, 32..1 by
// shuffles within one wave: the same pairs added in the same order), with
// the device expf/logf. The candidate selection is this file's own: the
// reference sorts the whole legal range (a bitonic network of ~66 barrier
// phases at 2048 candidates); here a 4-pass radix select over a 32-bit
// order-preserving key of the value finds the selected value and a ballot
// count orders equal values by index, which names the same candidate.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool finite_bits(float x) { return (__float_as_uint(x) & 0x7fffffffu) < 0x7f800000u; }
__device__ __forceinline__ bool sample_before(float a, uint32_t ai, float b, uint32_t bi) {
  return a > b || (a == b && ai < bi);
}
// Ascending key order = descending value order; -0 and +0 share a key (they
// compare equal, so their order is by index).
__device__ __forceinline__ uint32_t descending_key(float v) {
  const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
  const uint32_t ascending = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ~ascending;
}

__device__ __forceinline__ void write_sample(const ppk::RenyiArgs& a, uint32_t row, uint32_t token, uint32_t valid,
                                             uint32_t support) {
  a.out[row] = token;
  a.out[size_t(a.batch) + row] = valid;
  a.out[2 * size_t(a.batch) + row] = support;
}

__device__ __forceinline__ void renyi_sample_body(const ppk::RenyiArgs& a) {
  // Every float operation rounds on its own, as the reference kernel is built
  // (-ffp-contract=off, app/src/model/hip_kernel.rs:46) and as its host oracle
  // evaluates (app/src/inference/hip_sampling_reference.rs:73): the CFG value
  // u + cfg * (c - u) is a rounded product and then a rounded sum, never one
  // fused multiply-add, whose 1-ulp differences can reorder candidates.
#pragma clang fp contract(off)
  constexpr int T = ppk::kSamplerThreads;
  constexpr int PER = ppk::kSamplerMaxChoices / T;  // candidates per thread
  __shared__ float s_vals[ppk::kSamplerMaxChoices];
  __shared__ float s_sum[T], s_sum_a[T];
  __shared__ float s_wmax[T / 64];
  __shared__ uint32_t s_wid[T / 64], s_wbad[T / 64];
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_wtotal[T / 64];
  __shared__ uint64_t s_ballot[PER][T / 64];
  __shared__ uint32_t s_state[4];  // support, rank, invalid, selected bin / below

  const uint32_t row = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  // The whole head is requested first, beside the row's metadata: each
  // thread's columns (at most PER of each head, inside the row's raw logits
  // whatever the metadata say) before any is used, so the pass costs one
  // memory round trip instead of one or two per column.
  const float* c_row = a.raw + size_t(row) * a.guidance * a.choices;
  const bool guided = a.guidance == 2;
  float cv[PER], uv[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t col = uint32_t(t) + uint32_t(k) * T;
    cv[k] = col < a.choices ? c_row[col] : 0.f;
    uv[k] = guided && col < a.choices ? c_row[a.choices + col] : 0.f;
  }
  const uint32_t start = a.bounds[2 * row];
  const uint32_t count = a.bounds[2 * row + 1];
  const float uniform = a.uniforms[row];
  // Every thread evaluates the same metadata, so these exits are uniform.
  if (!finite_bits(uniform) || uniform < 0.f || uniform >= 1.f || start >= a.choices || count == 0 ||
      count > a.choices - start) {
    if (t == 0) write_sample(a, row, a.token_offset + (start < a.choices ? start : 0u), 0, 1);
    return;
  }

  // Whole head, in column order: CFG combine and finiteness; legal values to
  // LDS; arg-max.
  float lmax = -INFINITY;
  uint32_t lid = 0xffffffffu, lbad = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t col = uint32_t(t) + uint32_t(k) * T;
    if (col >= a.choices) continue;
    const float c = cv[k];
    float value = c;
    bool finite = finite_bits(c);
    if (guided) {
      const float u = uv[k];
      finite = finite && finite_bits(u);
      value = u + a.cfg * (c - u);
    }
    finite = finite && finite_bits(value);
    lbad |= finite ? 0u : 1u;
    if (!finite) value = 0.f;
    if (col >= start && col - start < count) {
      s_vals[col - start] = value;
      if (sample_before(value, col, lmax, lid)) {
        lmax = value;
        lid = col;
      }
    }
  }
#pragma unroll
  for (int o = 32; o; o >>= 1) {
    const float ov = __shfl_xor(lmax, o);
    const uint32_t oi = __shfl_xor(lid, o);
    if (sample_before(ov, oi, lmax, lid)) {
      lmax = ov;
      lid = oi;
    }
    lbad |= __shfl_xor(lbad, o);
  }
  if (lane == 0) {
    s_wmax[wave] = lmax;
    s_wid[wave] = lid;
    s_wbad[wave] = lbad;
  }
  __syncthreads();
  float maximum = s_wmax[0];
  uint32_t maximum_id = s_wid[0], bad = s_wbad[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) {
    if (sample_before(s_wmax[w], s_wid[w], maximum, maximum_id)) {
      maximum = s_wmax[w];
      maximum_id = s_wid[w];
    }
    bad |= s_wbad[w];
  }
  if (bad) {
    if (t == 0) write_sample(a, row, a.token_offset + start, 0, 1);
    return;
  }

  // Strided partial sums in candidate order, then the halving tree.
  float vals[PER];
  float sum = 0.f, sum_a = 0.f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t ci = uint32_t(t) + uint32_t(k) * T;
    vals[k] = ci < count ? s_vals[ci] : 0.f;
    if (ci < count) {
      const float shifted = vals[k] - maximum;
      sum += expf(shifted);
      sum_a += expf(a.alpha * shifted);
    }
  }
  s_sum[t] = sum;
  s_sum_a[t] = sum_a;
  __syncthreads();
  if (t < 128) {
    s_sum[t] += s_sum[t + 128];
    s_sum_a[t] += s_sum_a[t + 128];
  }
  __syncthreads();
  if (wave == 0) {
    float z = s_sum[lane] + s_sum[lane + 64];
    float za = s_sum_a[lane] + s_sum_a[lane + 64];
#pragma unroll
    for (int o = 32; o; o >>= 1) {
      z += __shfl_down(z, o);
      za += __shfl_down(za, o);
    }
    if (lane == 0) {
      const float log_z = logf(z);
      const float log_za = logf(za);
      float correction = log_z - log_za;
      if (correction < 0.0f) correction = 0.0f;
      float entropy = log_z + correction / (a.alpha - 1.0f);
      uint32_t invalid = !finite_bits(log_z) || !finite_bits(log_za) || !finite_bits(entropy);
      uint32_t support = 1, rank = 0;
      if (!invalid) {
        const float maximum_entropy = logf((float)count);
        if (entropy < 0.0f) entropy = 0.0f;
        if (entropy > maximum_entropy) entropy = maximum_entropy;
        const float rounded = expf(entropy) + 0.5f;
        support = (uint32_t)rounded;
        if (support < 1) support = 1;
        if (support > count) support = count;
        rank = (uint32_t)(uniform * (float)support);
        if (rank >= support) rank = support - 1;
      }
      s_state[0] = support;
      s_state[1] = rank;
      s_state[2] = invalid;
    }
  }
  __syncthreads();
  const uint32_t support = s_state[0];
  uint32_t r = s_state[1];
  if (s_state[2]) {
    if (t == 0) write_sample(a, row, a.token_offset + start, 0, 1);
    return;
  }
  if (r == 0) {
    if (t == 0) write_sample(a, row, a.token_offset + maximum_id, 1, support);
    return;
  }

  // Radix select, 8 key bits per pass from the top: after four passes the
  // prefix is the selected value's key and r its rank among equal values.
  uint32_t keys[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) keys[k] = descending_key(vals[k]);
  uint32_t prefix = 0, pmask = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    s_hist[t] = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const uint32_t ci = uint32_t(t) + uint32_t(k) * T;
      if (ci < count && (keys[k] & pmask) == prefix) atomicAdd(&s_hist[(keys[k] >> shift) & 255u], 1u);
    }
    __syncthreads();
    const uint32_t h = s_hist[t];
    uint32_t incl = h;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) s_wtotal[wave] = incl;
    __syncthreads();
    uint32_t below = incl - h;
    for (int w = 0; w < wave; ++w) below += s_wtotal[w];
    if (h > 0 && below <= r && r < below + h) {
      s_state[3] = uint32_t(t);
      s_hist[0] = below;  // every thread has read its own bin already
    }
    __syncthreads();
    const uint32_t bin = s_state[3];
    r -= s_hist[0];
    prefix |= bin << shift;
    pmask |= 255u << shift;
    __syncthreads();
  }

  // Among candidates with the selected key, the r-th by ascending index.
  // Candidate ci = t + 256 k: index order is (k, wave, lane) order. The
  // selection always names one candidate (r stays below the count of keys
  // matching the prefix); the record written first only keeps the row's
  // output defined should it not.
  if (t == 0) write_sample(a, row, a.token_offset + start, 0, 1);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t ci = uint32_t(t) + uint32_t(k) * T;
    const uint64_t b = __ballot(ci < count && keys[k] == prefix);
    if (lane == 0) s_ballot[k][wave] = b;
  }
  __syncthreads();
  uint32_t before_k = 0;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t ci = uint32_t(t) + uint32_t(k) * T;
    if (ci < count && keys[k] == prefix) {
      uint32_t pos = before_k + uint32_t(__popcll(s_ballot[k][wave] & ((uint64_t(1) << lane) - 1)));
      for (int w = 0; w < wave; ++w) pos += uint32_t(__popcll(s_ballot[k][w]));
      if (pos == r) write_sample(a, row, a.token_offset + start + ci, 1, support);
    }
#pragma unroll
    for (int w = 0; w < T / 64; ++w) before_k += uint32_t(__popcll(s_ballot[k][w]));
  }
}

// ---------------------------------------------------------------------------
// Float-store append (the in-place slice_set / scatter_set of
// app/src/model/cache.rs:271-276,437-469): token records of K and V to their
// arena slots, UNIT bytes per thread and step, grid-stride. Slots at or past
// capacity are skipped (the host never plans them).
// ---------------------------------------------------------------------------
template <int UNIT>
struct UnitType;
template <>
struct UnitType<16> {
  using T = u4;
};
template <>
struct UnitType<4> {
  using T = uint32_t;
};
template <>
struct UnitType<2> {
  using T = uint16_t;
};

template <int UNIT>
__device__ __forceinline__ void scatter_body(const ppk::ScatterArgs& a) {
  using T = typename UnitType<UNIT>::T;
  const uint64_t per_tensor = a.rows * a.tokens * a.row_units;
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < 2 * per_tensor; i += stride) {
    const uint32_t tensor = i >= per_tensor ? 1u : 0u;
    const uint64_t j = i - (tensor ? per_tensor : 0);
    const uint64_t rt = j / a.row_units;
    const uint32_t u = uint32_t(j - rt * a.row_units);
    const uint64_t r = rt / a.tokens;
    const uint32_t t = uint32_t(rt - r * a.tokens);
    const uint64_t slot = uint64_t(a.past ? a.past[r / a.heads] : a.uniform_past) + t;
    if (slot >= a.capacity) continue;
    const T* src = reinterpret_cast<const T*>(a.src[tensor]);
    T* dst = reinterpret_cast<T*>(a.dst[tensor]);
    dst[(r * a.capacity + slot) * a.row_units + u] = src[rt * a.row_units + u];
  }
}

// ---------------------------------------------------------------------------
// Batched rectangle copy with zero fill (arena joins, growth and
// copy-on-write: every row of a new arena receives its committed prefix and
// zeros up to its capacity in one launch, instead of a memset of the whole
// arena plus one runtime copy per plane and sequence). Blocks stride over
// tiles of one row each, eight units in flight per thread.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void copy_rect(const ppk::Copy2D& c, uint32_t unit_bytes) {
  constexpr uint32_t ILP = 8;
  const uint32_t per_row = c.fill / unit_bytes;
  const uint32_t copy_cols = c.width / unit_bytes;
  if (per_row == 0) return;
  // Tiles of up to ILP * blockDim.x units of one row: a block finds its tile's
  // row and first column with one (block-uniform) division, and each lane's
  // columns follow by addition, so no unit pays an integer division.
  const uint32_t tile = min(per_row, ILP * blockDim.x);
  const uint32_t tiles_per_row = (per_row + tile - 1) / tile;
  const uint64_t tiles = uint64_t(c.height) * tiles_per_row;
  for (uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const uint64_t row = t / tiles_per_row;
    const uint32_t col0 = uint32_t(t - row * tiles_per_row) * tile;
    const uint32_t end = min(col0 + tile, per_row);
    const T* src = reinterpret_cast<const T*>(c.src + row * c.spitch);
    T* dst = reinterpret_cast<T*>(c.dst + row * c.dpitch);
    T val[ILP];
#pragma unroll
    for (uint32_t k = 0; k < ILP; ++k) {
      const uint32_t col = col0 + k * blockDim.x + threadIdx.x;
      val[k] = T{};
      if (col < end && col < copy_cols) val[k] = __builtin_nontemporal_load(src + col);
    }
#pragma unroll
    for (uint32_t k = 0; k < ILP; ++k) {
      const uint32_t col = col0 + k * blockDim.x + threadIdx.x;
      if (col < end) dst[col] = val[k];
    }
  }
}

__device__ __forceinline__ void copy_batch_body(const ppk::CopyBatchArgs& a) {
  if (blockIdx.y >= a.n) return;
  const ppk::Copy2D& c = a.c[blockIdx.y];
  switch (c.unit) {  // uniform per block
    case 16: copy_rect<u4>(c, 16); break;
    case 4: copy_rect<uint32_t>(c, 4); break;
    case 2: copy_rect<uint16_t>(c, 2); break;
    default: copy_rect<uint8_t>(c, 1); break;
  }
}

}  // namespace

#define PPK_QUANTIZE(D)                                                                \
  extern "C" __global__ __launch_bounds__(256) void ppk_quantize_d##D(ppk::QuantizeArgs a) { \
    quantize_body<D>(a);                                                               \
  }
PPK_QUANTIZE(64)
PPK_QUANTIZE(128)
PPK_QUANTIZE(256)

extern "C" __global__ __launch_bounds__(256) void ppk_dequantize(ppk::DequantizeArgs a) { dequantize_body(a); }
// Streaming quantize: dense [rows, D] (ppk_quantize) and appends into arenas
// (ppk_quantize_append, KV arena writes), separate kernels so the dense path
// keeps its smaller register footprint.
#define PPK_QSTREAM(D)                                                                              \
  extern "C" __global__ __launch_bounds__(256) void ppk_quantize_dense_d##D(ppk::QuantizeArgs a) {  \
    quantize_stream_dtype<D, false>(a);                                                             \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(256) void ppk_quantize_append_d##D(ppk::QuantizeArgs a) { \
    quantize_stream_dtype<D, true>(a);                                                              \
  }
PPK_QSTREAM(64)
PPK_QSTREAM(128)
PPK_QSTREAM(256)
#undef PPK_QSTREAM

// Blocks of up to 8 waves (the plan never makes larger int8 blocks): two
// waves per SIMD, up to 256 VGPRs each, a ring of kRing batches in flight.
constexpr int kRing = 3;
#define PPK_ATTN(D)                                                                          \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))    \
  void ppk_decode_d##D(ppk::DecodeArgs a) {                                                  \
    decode_body<D, false, kRing>(a);                                                         \
  }                                                                                          \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))    \
  void ppk_decode_bf16h_d##D(ppk::DecodeArgs a) {                                            \
    decode_body<D, true, kRing>(a);                                                          \
  }                                                                                          \
  extern "C" __global__ __launch_bounds__(64) void ppk_attn_merge_d##D(ppk::MergeArgs a) {   \
    attn_merge_body<D>(a);                                                                   \
  }
PPK_ATTN(64)
PPK_ATTN(128)
PPK_ATTN(256)

// Flat work list kernels: up to 256 VGPRs, i.e. 8 resident waves per CU (the host launches 8).
#define PPK_ATTN_FLAT(D)                                                                                \
  extern "C" __global__ __launch_bounds__(512) void ppk_decode_flat_d##D(ppk::DecodeFlatArgs a) {      \
    decode_flat_body<D, false>(a);                                                                      \
  }                                                                                                     \
  extern "C" __global__ __launch_bounds__(512) void ppk_decode_flat_bf16h_d##D(ppk::DecodeFlatArgs a) { \
    decode_flat_body<D, true>(a);                                                                       \
  }                                                                                                     \
  extern "C" __global__ __launch_bounds__(64) void ppk_attn_merge_flat_d##D(ppk::MergeFlatArgs a) {   \
    attn_merge_flat_body<D>(a);                                                                         \
  }
PPK_ATTN_FLAT(64)
PPK_ATTN_FLAT(128)
PPK_ATTN_FLAT(256)
#undef PPK_ATTN_FLAT

#define PPK_FLOAT_ATTN(D)                                                                        \
  extern "C" __global__ __launch_bounds__(1024) void ppk_fdecode_bf16_d##D(ppk::FloatDecodeArgs a) { \
    fdecode_body<D, true, false>(a);                                                             \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(1024) void ppk_fdecode_f32_d##D(ppk::FloatDecodeArgs a) {  \
    fdecode_body<D, false, false>(a);                                                            \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(1024) void ppk_fstep_bf16_d##D(ppk::FloatDecodeArgs a) {   \
    fdecode_body<D, true, true>(a);                                                              \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(1024) void ppk_fstep_f32_d##D(ppk::FloatDecodeArgs a) {    \
    fdecode_body<D, false, true>(a);                                                             \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(64) void ppk_fmerge_d##D(ppk::FloatMergeArgs a) {      \
    fmerge_body<D>(a);                                                                           \
  }
PPK_FLOAT_ATTN(64)
PPK_FLOAT_ATTN(128)
PPK_FLOAT_ATTN(256)

#define PPK_FLOAT_ATTN_FLAT(D)                                                                                 \
  extern "C" __global__ __launch_bounds__(512) void ppk_fdecode_flat_bf16_d##D(ppk::FloatDecodeFlatArgs a) { \
    fdecode_flat_body<D, true, false>(a);                                                                      \
  }                                                                                                            \
  extern "C" __global__ __launch_bounds__(512) void ppk_fdecode_flat_f32_d##D(ppk::FloatDecodeFlatArgs a) {  \
    fdecode_flat_body<D, false, false>(a);                                                                     \
  }                                                                                                            \
  extern "C" __global__ __launch_bounds__(512) void ppk_fstep_flat_bf16_d##D(ppk::FloatDecodeFlatArgs a) {   \
    fdecode_flat_body<D, true, true>(a);                                                                       \
  }                                                                                                            \
  extern "C" __global__ __launch_bounds__(512) void ppk_fstep_flat_f32_d##D(ppk::FloatDecodeFlatArgs a) {    \
    fdecode_flat_body<D, false, true>(a);                                                                      \
  }                                                                                                            \
  extern "C" __global__ __launch_bounds__(64) void ppk_fmerge_flat_d##D(ppk::FloatMergeFlatArgs a) {          \
    fmerge_flat_body<D>(a);                                                                                    \
  }
PPK_FLOAT_ATTN_FLAT(64)
PPK_FLOAT_ATTN_FLAT(128)
PPK_FLOAT_ATTN_FLAT(256)
#undef PPK_FLOAT_ATTN_FLAT

extern "C" __global__ __launch_bounds__(256) void ppk_renyi_sample(ppk::RenyiArgs a) { renyi_sample_body(a); }

extern "C" __global__ __launch_bounds__(256) void ppk_kv_scatter_u16(ppk::ScatterArgs a) { scatter_body<16>(a); }
extern "C" __global__ __launch_bounds__(256) void ppk_kv_scatter_u4(ppk::ScatterArgs a) { scatter_body<4>(a); }
extern "C" __global__ __launch_bounds__(256) void ppk_kv_scatter_u2(ppk::ScatterArgs a) { scatter_body<2>(a); }
extern "C" __global__ __launch_bounds__(256) void ppk_copy2d_batch(ppk::CopyBatchArgs a) { copy_batch_body(a); }
