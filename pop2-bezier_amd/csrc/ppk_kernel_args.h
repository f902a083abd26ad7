// Kernel argument blocks shared by the gfx950 code object (ppk_kernels.hip)
// and the host shim (ppk_abi.cpp). Each kernel takes one of these by value,
// so hipModuleLaunchKernel passes a single pointer to it.
#pragma once
#include <stdint.h>

namespace ppk {

// Wave64 lanes; every kernel here is written for 64-wide wavefronts.
constexpr int kWave = 64;
// Bytes one lane moves per global load in the attention kernels (dwordx4).
constexpr int kLaneBytes = 16;

// Quantize one (row, token) of D channels per wave, either densely
// (dst index = src index) or into an arena slot past[b] + token.
struct QuantizeArgs {
  const void* src[2];       // K and V sources ([rows_per_tensor, D]); src[1] unused if ntensors == 1
  uint8_t* codes[2];        // dense [rows, D] or arena [bh, capacity, D]
  float* scales[2];         // dense [rows] or arena [bh, capacity]
  const uint32_t* past;     // append mode: slot of token 0 of sequence b = past[b]
  uint32_t* flags;          // optional
  uint64_t rows;            // (bh * tokens) rows per tensor
  uint32_t heads;           // append mode: sequence b = bh / heads
  uint32_t tokens;          // append mode: tokens per bh row
  uint32_t capacity;        // 0 = dense mode; > 0 = append mode
  uint32_t src_dtype;       // PPK_F32 / PPK_BF16 / PPK_F16
  uint32_t ntensors;        // 1 or 2
  uint32_t uniform_past;    // append mode with past == nullptr: slot of token 0 for every row
};

// Float-store append: copy [rows, tokens, row_bytes] token records of K and V
// into [rows, capacity, row_bytes] arenas at slot past[row / heads] + t (or
// uniform_past + t when past is null), in units of the kernel's UNIT bytes.
struct ScatterArgs {
  const uint8_t* src[2];
  uint8_t* dst[2];
  const uint32_t* past;
  uint64_t rows;
  uint32_t heads, tokens, capacity, uniform_past;
  uint32_t row_units;       // units per token record
  uint32_t pad;
};

struct DequantizeArgs {
  const uint8_t* codes;     // [rows, D]
  const float* scales;      // [rows]
  void* out;                // [rows, D]
  uint64_t rows;
  uint32_t head_dim;
  uint32_t out_dtype;
  uint32_t round_bf16;
  uint32_t pad;
};

// Wave-clock diagnostics (code objects built with PPK_WAVE_CLOCK; the
// library's own code object never reads these fields): when `clock` is set,
// every wave of the int8 per-row decode and merge kernels writes one record
// of kWaveClockWords u64 at a slot of its own: word 0 of the buffer holds
// the slots per launch and kernel kind (at least blocks x waves per block),
// word 1 the most records the buffer takes; wave w of block x of the launch
// with sequence number s writes record (2 s + kind - 1) * word0 + x * waves +
// w, records from word kWaveClockWords (no atomics: a shared counter would
// serialise every wave's end). Record: [0] kind << 56 | launch sequence <<
// 32 | block << 8 | wave (0 for a slot never written), [1] XCC id << 32 |
// HW_ID register, [2 + i] the wave's real-time clock (100 MHz) at point i of
// its kind (kWaveClockPoints).
constexpr int kWaveClockWords = 16;
constexpr int kWaveClockPoints = 8;
constexpr uint32_t kWaveClockDecode = 1;  // 0 entry, 1 first loads issued, 2 past[b] here, 3 first K data here,
                                          // 4 stream done, 5 block joined, 6 output / record stored
constexpr uint32_t kWaveClockMerge = 2;   // 0 entry, 1 records combined, 2 output stored

// Decode attention: block (group g, row r), blockIdx.x = g * rows + r, of
// W = blockDim.x / 64 waves covers history tokens [g*W*S, (g+1)*W*S) of row r,
// S = split_tokens per wave.
// ngroups == 1: the block writes the final output row (current token included).
// ngroups > 1: it writes a partial record for the merge kernel:
//   y[D] floats at part_y + (row * ngroups + g) * D
//   (m, z) at part_mz + (row * ngroups + g) * 2, m in log2 units.
// append != 0: group 0 of each row first quantises k_new/v_new[row] into
// slot past[b] of the arenas k/v/ks/vs (never read by this launch).
struct DecodeArgs {
  const void* q;            // [rows, D]
  uint8_t* k;               // [rows, capacity, D]
  uint8_t* v;
  float* ks;                // [rows, capacity]
  float* vs;
  const void* sk;           // [rows, D] current key (unquantised)
  const void* sv;
  const uint32_t* past;     // [rows / heads]
  float* part_y;
  float* part_mz;
  void* out;                // [rows, D]
  const void* k_new;        // [rows, D] token to append (append != 0)
  const void* v_new;
  uint32_t* flags;          // optional
  uint32_t rows, heads, capacity, split_tokens, ngroups;
  uint32_t q_dtype, scratch_dtype, out_dtype, new_dtype, append;
  float scale_log2;         // softmax_scale * log2(e)
  uint32_t span;            // max_past or capacity: balanced plan, rows with past[b] > span give NaN; per-row
                            // plan, a past[b] <= span past the plan's coverage flags stale host lengths
  uint32_t speculate;       // per-row plan: request each wave's first K batches before past[] arrives
  uint32_t clock_seq;       // wave-clock builds only: the launch's sequence number in the records
  uint32_t clock_cap;       // wave-clock builds only: records the buffer holds (from its size on the host)
  uint64_t* clock;          // wave-clock builds only (kWaveClock*): record buffer, or null
};

struct MergeArgs {
  const void* q;            // [rows, D]
  const void* sk;           // [rows, D]
  const void* sv;           // [rows, D]
  const uint32_t* past;
  const float* part_y;
  const float* part_mz;
  void* out;                // [rows, D]
  uint32_t rows, heads, capacity, split_tokens, nsplits;
  uint32_t q_dtype, scratch_dtype, out_dtype;
  float scale_log2;
  uint32_t span;            // rows with past[b] > span give NaN (balanced plan)
  uint32_t clock_seq;       // wave-clock builds only, as in DecodeArgs
  uint32_t clock_cap;
  uint64_t* clock;
};

// Balanced work list of a ragged batch (the ppk_decode_flat kernels), built
// on the host from the caller's host copy of the lengths: the live history
// of row r = b * heads + h is len[b] tokens (past[b] when it is at most
// min(capacity, span), else none), cut into units[b] = max(1, ceil(len[b] /
// share)) units of at most `share` tokens inside the row; units are numbered
// row after row from first[b] (first[] is nondecreasing and holds
// 0xffffffff past the batch). Wave i takes unit i. A row of one unit is
// finished by its wave; unit s of a longer row leaves the record at slot s
// of the row's ngroups slots (y at part_y + (row * ngroups + s) * D, (m, z)
// at part_mz + (row * ngroups + s) * 2) for the balanced merge kernel.
// past[] is compared with the device's past: a sequence whose values differ
// gives NaN rows.
constexpr int kFlatMaxBatch = 64;
struct FlatTable {
  uint32_t batch;                  // sequences
  uint32_t share;                  // most tokens of a unit
  uint32_t units_total;            // units over all rows
  uint32_t pad;
  uint32_t past[kFlatMaxBatch];    // the host's past[b]
  uint32_t len[kFlatMaxBatch];     // live history tokens of each row of sequence b
  uint32_t units[kFlatMaxBatch];   // units per row of sequence b
  uint32_t first[kFlatMaxBatch];   // index of sequence b's first unit
};
struct DecodeFlatArgs {
  DecodeArgs d;             // ngroups = record slots per row
  FlatTable t;
};
struct MergeFlatArgs {
  MergeArgs m;              // nsplits = record slots per row
  FlatTable t;
};

// Float-KV decode attention: the same block geometry over unquantised bf16 or
// f32 K/V. Row r attends its first n = lengths ? lengths[r / heads] : size
// tokens (the current token is already stored); no separate current token.
// n == 0 or n > span (= max_length, or size) gives NaN. ngroups > 1 leaves
// partial records for the float merge kernel, laid out as for DecodeArgs.
struct FloatDecodeArgs {
  const void* q;            // row r at q + r * q_stride elements
  const void* k;            // row r at k + r * k_stride elements, tokens D apart
  const void* v;
  const uint32_t* lengths;  // [rows / heads], or nullptr
  float* part_y;
  float* part_mz;
  void* out;                // [rows, D]
  // The fused step (ppk_fstep_* kernels): lengths[b] = p tokens are stored;
  // row r's current token k_new/v_new[r] (new_dtype, rounded to the store's
  // dtype) is written at slot p when p < size (else PPK_FLAG_OVERFLOW in
  // *flags) and the row attends the p stored tokens plus that token: NaN
  // unless p < size and p + 1 <= span.
  const void* k_new;
  const void* v_new;
  uint32_t* flags;
  uint64_t q_stride, k_stride, v_stride;
  uint32_t rows, heads, size, split_tokens, ngroups;
  uint32_t q_dtype, out_dtype;
  float scale_log2;         // softmax_scale * log2(e)
  uint32_t span;            // most tokens a row may attend (<= size)
  uint32_t new_dtype;
};

struct FloatMergeArgs {
  const uint32_t* lengths;  // [rows / heads], or nullptr
  const float* part_y;
  const float* part_mz;
  void* out;                // [rows, D]
  // The fused step (step != 0): the current token joins the records as in
  // the int8 merge; q, k_new and v_new as in FloatDecodeArgs.
  const void* q;
  const void* k_new;
  const void* v_new;
  uint64_t q_stride;
  uint32_t rows, heads, size, split_tokens, nsplits, out_dtype, span;
  uint32_t step, q_dtype, new_dtype, kv_bf16;
  float scale_log2;
};

// Float-KV decode over the balanced work list: the table as for the int8
// path, with past[b] the host's lengths[b] and len[b] its live tokens (0 for
// a length outside (0, min(size, max_length)], whose rows give NaN).
struct FloatDecodeFlatArgs {
  FloatDecodeArgs d;
  FlatTable t;
};
struct FloatMergeFlatArgs {
  FloatMergeArgs m;
  FlatTable t;
};

// Batched rectangle copies: block (x, y) serves rectangle y. Each of its
// `height` destination rows receives `width` bytes copied from the source row
// followed by zeros up to `fill` bytes (src may be null when width is 0).
// `unit` bytes (16, 4, 2 or 1) per thread and step, chosen on the host so
// that width, fill, both pitches and both base addresses are multiples of it.
struct Copy2D {
  const uint8_t* src;
  uint8_t* dst;
  uint64_t spitch, dpitch;
  uint32_t width, fill, height, unit;
};
constexpr int kMaxCopies = 32;
struct CopyBatchArgs {
  uint32_t n, pad;
  Copy2D c[kMaxCopies];
};

// CFG + Renyi effective-support sampler: one 256-thread block per logical row.
struct RenyiArgs {
  const float* raw;         // [batch * guidance, choices]; guided rows interleave (conditional, unconditional)
  const float* uniforms;    // [batch]
  const uint32_t* bounds;   // [batch, 2] = (start, count) of the legal range
  uint32_t* out;            // [3, batch]: token, valid, support
  uint32_t batch, choices, guidance, token_offset;
  float alpha, cfg;
};

// Threads per sampler block: the partial-sum layout (256 strided partials and
// their tree) is part of the sampler's arithmetic contract.
constexpr int kSamplerThreads = 256;
constexpr int kSamplerMaxChoices = 2048;

}  // namespace ppk
