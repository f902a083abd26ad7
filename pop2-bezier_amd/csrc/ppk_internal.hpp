// Host-side internals shared by the C-ABI shim (ppk_abi.cpp) and the
// int8_kv_ops host mirror (int8_kv_ops.cpp). Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/ppk_int8_kv.h"
#include "ppk_kernel_args.h"

namespace ppk {

// Error classes map onto the ABI status codes; the message prefixes are the
// ones the reference's failure classifier keys on
// (app/src/model/hip_kernel.rs:79-81,162-170; app/src/inference.rs:84-92).
struct PreconditionError : std::runtime_error {
  explicit PreconditionError(const std::string& m) : std::runtime_error("HIP_PREPARATION: " + m) {}
};
struct UncertainError : std::runtime_error {
  explicit UncertainError(const std::string& m) : std::runtime_error("HIP_EXECUTION_UNCERTAIN: " + m) {}
};
struct InvalidOutputError : std::runtime_error {
  explicit InvalidOutputError(const std::string& m) : std::runtime_error("INVALID_OUTPUT: " + m) {}
};

// Checks on the launch path run hundreds of times per call (per row, per
// pair of rows): a literal message is only turned into a string on failure.
inline void require(bool ok, const char* message) {
  if (!ok) throw PreconditionError(message);
}
inline void require(bool ok, const std::string& message) {
  if (!ok) throw PreconditionError(message);
}

enum Fn : int {
  kQuantize64, kQuantize128, kQuantize256, kDequantize,
  kDecode64, kDecode128, kDecode256,
  kDecodeBf16h64, kDecodeBf16h128, kDecodeBf16h256,
  kMerge64, kMerge128, kMerge256,
  kFDecodeBf16_64, kFDecodeBf16_128, kFDecodeBf16_256,
  kFDecodeF32_64, kFDecodeF32_128, kFDecodeF32_256,
  kFMerge64, kFMerge128, kFMerge256,
  kRenyiSample,
  kScatter16, kScatter4, kScatter2,
  kCopyBatch,
  kQuantizeDense64, kQuantizeDense128, kQuantizeDense256,
  kQuantizeAppend64, kQuantizeAppend128, kQuantizeAppend256,
  kDecodeFlat64, kDecodeFlat128, kDecodeFlat256,
  kDecodeFlatBf16h64, kDecodeFlatBf16h128, kDecodeFlatBf16h256,
  kMergeFlat64, kMergeFlat128, kMergeFlat256,
  kFDecodeFlatBf16_64, kFDecodeFlatBf16_128, kFDecodeFlatBf16_256,
  kFDecodeFlatF32_64, kFDecodeFlatF32_128, kFDecodeFlatF32_256,
  kFMergeFlat64, kFMergeFlat128, kFMergeFlat256,
  kFStepBf16_64, kFStepBf16_128, kFStepBf16_256,
  kFStepF32_64, kFStepF32_128, kFStepF32_256,
  kFStepFlatBf16_64, kFStepFlatBf16_128, kFStepFlatBf16_256,
  kFStepFlatF32_64, kFStepFlatF32_128, kFStepFlatF32_256,
  kFnCount
};

struct EventPair {
  hipEvent_t start = nullptr, stop = nullptr;
};

// Bytes of the per-GPU device array behind ppk_decode_step_noalloc (ppk_scratch.hip).
constexpr size_t kScratchBytes = PPK_NOALLOC_SCRATCH_BYTES;
// Waves per CU of the balanced plan's launch (all resident: the decode_flat
// kernels hold at most 256 VGPRs).
constexpr uint32_t kFlatWavesPerCu = 8;
// int8 decode waves resident per CU: its kernels run two waves per SIMD
// (amdgpu_waves_per_eu(2, 2)), so blocks of 1, 2, 4 or 8 waves fill a CU.
constexpr uint32_t kInt8WavesPerCu = 8;

}  // namespace ppk

struct ppk_context {
  int device = -1;
  int cu_count = 0;
  hipModule_t module = nullptr;
  hipFunction_t fn[ppk::kFnCount] = {};
  std::string code_object;

  std::mutex prepare_mutex;
  bool int8_ready = false;  // ppk_prepare_int8_kv's self-check passed on this context

  // Device address of this GPU's copy of the no-alloc scratch array, looked up
  // at context creation (nullptr with the reason in scratch_error if that failed).
  void* scratch = nullptr;
  std::string scratch_error;

  // Device vectors of released write plans, recycled by the next plan created
  // on the same stream (stream order puts its upload after the old plan's
  // readers; the event recorded at release also orders it when a new stream
  // reuses the handle of a destroyed one); an allocation per plan costs ~9 us
  // of host time.
  struct PlanBuffer {
    uint32_t* dev = nullptr;
    size_t bytes = 0;
    hipStream_t stream = nullptr;
    hipEvent_t released = nullptr;  // recorded on `stream` when the plan was released
  };
  std::mutex plan_mutex;
  std::vector<PlanBuffer> plan_pool;

  // Stream-ordered pool for what the library allocates (arenas, plan
  // vectors, aliased-source copies), apart from the runtime's default pool.
  // Released at ppk_context_release.
  hipMemPool_t mem_pool = nullptr;

  // Arena blocks whose caches were released, kept for the next arena of the
  // same size: an event recorded on the stream that last used a block is
  // waited for by the stream that reuses it, so the new writes follow the old
  // readers on any stream. The runtime pool hands freed memory back at every
  // stream synchronisation whatever its release threshold, and a 24-layer
  // join of B = 32 that took its batch arenas from the runtime spent
  // 160-210 ms allocating; with released blocks kept here it takes 2-3 ms
  // (1.8 ms of it the copy kernel). Bounded by block_cache_limit (32 GiB, or
  // an eighth of the device's memory if that is less): a release that would
  // pass it first frees the oldest idle blocks. An allocation that fails while
  // blocks are kept frees them all and tries once more. Freed at release.
  struct CachedBlock {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t released = nullptr;  // recorded after the block's last use
  };
  static constexpr size_t kBlockCacheBytes = size_t(32) << 30;
  size_t block_cache_limit = kBlockCacheBytes;
  std::mutex block_mutex;
  std::vector<CachedBlock> block_cache;  // oldest first
  size_t block_cache_bytes = 0;
  std::vector<hipEvent_t> spare_events;  // events of reused blocks, recorded again by later releases

  std::mutex prof_mutex;
  bool profiling = false;
  uint64_t* wave_clock = nullptr;   // ppk_context_set_wave_clock
  uint32_t wave_clock_seq = 0;
  uint32_t wave_clock_cap = 0;      // records after the header the buffer holds
  std::vector<ppk::EventPair> pending[PPK_KERNEL_COUNT];
  std::vector<ppk::EventPair> pool;
  uint64_t launches[PPK_KERNEL_COUNT] = {};
  double total_ms[PPK_KERNEL_COUNT] = {};
};

namespace ppk {

// Restores the caller's current HIP device on scope exit.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device);
  ~DeviceGuard();
  DeviceGuard(const DeviceGuard&) = delete;
  DeviceGuard& operator=(const DeviceGuard&) = delete;

 private:
  int previous_ = -1;
  bool changed_ = false;
};

// Validated launch plans. Validation throws PreconditionError before any
// enqueue; launch throws UncertainError once a launch has been attempted.
struct AttentionPlan {
  uint32_t head_dim = 0;
  uint32_t split = 0;    // history tokens per wave (flat: most tokens a wave streams per piece)
  uint32_t waves = 0;    // waves per block
  uint32_t ngroups = 0;  // blocks per row; 1 = final output in the same launch (flat: record slots per row)
  uint32_t lds_bytes = 0;
  uint64_t y_bytes = 0, mz_bytes = 0, workspace_bytes = 0;
  // Balanced work list (attention over a ragged batch whose host lengths
  // are known, see FlatTable); ngroups = record slots per row, 1 when every
  // row is a single unit (then no merge launch).
  bool flat = false;
  // Per-row plan: whether each wave requests its first K batches before the
  // row's length arrives (off when 1/16 or more of the waves are known to
  // have no history).
  bool speculate = true;
  uint32_t blocks = 0;   // flat: blocks launched
  uint32_t span = 0;     // flat: rows with past beyond it give NaN
  FlatTable table{};
};
// Split policy shared by both attention paths: span history tokens per row,
// tpl tokens per wave-wide load, token_bytes of K+V (+scales) per token.
// min_split > 0: in the few-long-rows case, waves' shares may be halved down to
// min_split tokens so that blocks get four waves (0: never; int8: one batch,
// float: one batch and at least 16 KiB per wave). block_waves: the
// most waves of one block (int8: 8, float: 16).
AttentionPlan plan_rows(const ppk_context* ctx, uint32_t rows, uint64_t span, uint32_t explicit_split,
                        uint32_t tpl, uint64_t token_bytes, uint32_t head_dim, uint32_t min_split,
                        uint32_t block_waves);
AttentionPlan plan_attention(const ppk_context* ctx, const PpkAttentionArgs& a);
// The balanced plan of `rows` rows, `heads` per sequence, from the host
// lengths host[0 .. rows / heads) (at most 64 sequences); a length above
// `limit` has no live history. Needs 2 * rows <= the plan's waves.
AttentionPlan plan_flat(const ppk_context* ctx, uint32_t rows, uint32_t heads, const uint32_t* host, uint64_t limit,
                        uint32_t head_dim);
// Whether the balanced plan pays for these host lengths: the longest live
// row beyond 1.1 x the mean, at most 64 sequences, 2 * rows within its waves.
bool flat_pays(const ppk_context* ctx, uint32_t rows, uint32_t heads, const uint32_t* host, uint64_t limit);
// Whether a batch fits the balanced plan (at most 64 sequences, 2 * rows
// within its waves); require_balanced throws PreconditionError, naming what
// is missing, for a caller that asked for the balanced plan.
bool flat_fits(const ppk_context* ctx, uint32_t rows, uint32_t heads);
void require_balanced(const ppk_context* ctx, uint32_t rows, uint32_t heads, const uint32_t* host,
                      uint32_t split_tokens);
// The PPK_ATTN_PLAN_* bits.
constexpr uint32_t kPlanFlags = PPK_ATTN_PLAN_PER_ROW | PPK_ATTN_PLAN_BALANCED;
// The most live tokens of any of `batch` sequences (a length above limit has none).
uint64_t longest_live(const uint32_t* host, uint32_t batch, uint64_t limit);
// The history the per-row plan covers with host lengths: the longest live
// row, at least one token.
uint64_t row_cover(const uint32_t* host, uint32_t batch, uint64_t limit);
// The most live history tokens one CU streams under a per-row plan p or a
// balanced plan (block i on CU i mod cus, as an all-resident launch is
// placed).
uint64_t per_row_cu_peak(const AttentionPlan& p, uint32_t rows, uint32_t heads, const uint32_t* host,
                         uint64_t limit, uint32_t cus);
uint64_t flat_cu_peak(const AttentionPlan& p, uint32_t heads, uint32_t cus);
// Whether the balanced plan `flat` beats the per-row plan of an int8 attention
// call over the host lengths (token_bytes of history per token and row).
// Whether the per-row plan p should speculate (AttentionPlan::speculate):
// fewer than 1/16 of its waves lie wholly past their row's live history (the
// host lengths, or every row at `span` without them).
bool per_row_speculates(const AttentionPlan& p, uint32_t rows, uint32_t heads, const uint32_t* host, uint64_t span,
                        uint64_t limit);
bool balanced_pays(const ppk_context* ctx, const AttentionPlan& per_row, const AttentionPlan& flat, uint32_t rows,
                   uint32_t heads, const uint32_t* host, uint64_t limit, uint64_t token_bytes);
// Whether the per-row plan's waves of `split` tokens are uneven: the most
// tokens one streams beyond 1.1 x the mean over those that stream any.
bool per_row_waves_uneven(uint32_t batch, const uint32_t* host, uint64_t limit, uint32_t split);
AttentionPlan plan_float_attention(const ppk_context* ctx, const PpkFloatAttentionArgs& a);

void run_quantize(ppk_context* ctx, hipStream_t stream, const PpkQuantizeArgs& a);
void run_append(ppk_context* ctx, hipStream_t stream, const PpkAppendArgs& a);
void run_dequantize(ppk_context* ctx, hipStream_t stream, const PpkDequantizeArgs& a);
// step == nullptr: attention only; otherwise the fused decode step.
// scratch != nullptr: the partial records go to that device buffer of
// scratch_bytes (the no-alloc entry point) instead of a.workspace, which is
// then ignored, and no launch is traced (tracing creates events).
void run_attention(ppk_context* ctx, hipStream_t stream, const PpkAttentionArgs& a,
                   const PpkDecodeStepArgs* step = nullptr, void* scratch = nullptr, uint64_t scratch_bytes = 0);

// Device address of the current process's no-alloc scratch array on `device`
// (ppk_scratch.hip): looked up once per device with that device current,
// then served from a per-device table. Throws PreconditionError if the
// lookup failed.
void* scratch_lookup(int device);
// step == nullptr: attention only; otherwise the fused float decode step.
void run_float_attention(ppk_context* ctx, hipStream_t stream, const PpkFloatAttentionArgs& a,
                         const PpkFloatDecodeStepArgs* step = nullptr);
void run_renyi_sample(ppk_context* ctx, hipStream_t stream, const PpkRenyiSampleArgs& a);

// Arena writes for the KV cache manager (kv_arena.cpp). Rows of `heads`
// per sequence; token t of sequence b lands at slot (past ? past[b] :
// uniform_past) + t of [rows, capacity, head_dim] storage. The caller has
// validated every shape; these only build the kernel arguments and launch.
struct ArenaWrite {
  const void* k_src = nullptr;
  const void* v_src = nullptr;
  uint32_t src_dtype = 0;     // PPK_F32 / PPK_BF16 / PPK_F16
  uint8_t* k = nullptr;       // codes (int8) or float records
  uint8_t* v = nullptr;
  float* ks = nullptr;        // int8 only
  float* vs = nullptr;
  const uint32_t* past = nullptr;
  uint32_t uniform_past = 0;
  uint64_t sequences = 0;
  uint32_t heads = 0, tokens = 0, capacity = 0, head_dim = 0;
  uint32_t elem_bytes = 0;    // 0 = int8 (quantise); else bytes per float element
};
void run_arena_write(ppk_context* ctx, hipStream_t stream, const ArenaWrite& w);

// Batched strided copies (one launch per up to kMaxCopies rectangles): each of
// `height` dst rows (dpitch apart) gets `width` bytes of its src row (spitch
// apart; src may be null when width is 0), then zeros up to `fill` bytes.
struct CopyDesc {
  const void* src = nullptr;
  void* dst = nullptr;
  uint64_t spitch = 0, dpitch = 0, width = 0, fill = 0;
  uint32_t height = 0;
};
void run_copy_batch(ppk_context* ctx, hipStream_t stream, const std::vector<CopyDesc>& copies);

// KV cache manager (kv_arena.cpp).
namespace kv {
ppk_kv_cache* create(ppk_context* ctx, const PpkKvConfig& cfg);
void info(const ppk_kv_cache& c, PpkKvInfo* out);
void view(const ppk_kv_cache& c, PpkKvView* out);
void truncate(ppk_kv_cache& c, uint32_t new_len);
ppk_kv_cache* adopt(ppk_context* ctx, const PpkKvConfig& cfg, void* k, void* v, uint32_t capacity,
                    uint32_t committed_len);
void advance(ppk_kv_cache& c, uint32_t previous, uint32_t next);
void query(ppk_context* ctx, hipStream_t stream, ppk_kv_cache& c, uint32_t past, const PpkKvWrite& w,
           PpkKvView* out);
ppk_write_plan* plan_create(ppk_context* ctx, hipStream_t stream, const uint32_t* past_lens, uint32_t batch,
                            uint32_t heads, uint32_t head_dim);
// Frees every kept arena block once the work that last used it has finished,
// then returns the pool's unused memory to the device; the bytes freed.
uint64_t drain_blocks(ppk_context* ctx);
// hipMallocFromPoolAsync from the context's pool; when it runs out of memory
// while released blocks are kept (reused only at an equal size), drains them
// and tries once more.
hipError_t pool_alloc(ppk_context* ctx, void** ptr, size_t bytes, hipStream_t stream);
void query_batch(ppk_context* ctx, hipStream_t stream, ppk_kv_cache* const* caches, uint32_t batch,
                 const uint32_t* past_lens, const PpkKvWrite& w, const ppk_write_plan* plan, PpkKvView* out);
ppk_kv_cache* clone(const ppk_kv_cache& c);
void release(ppk_kv_cache* c);
void plan_release(ppk_write_plan* p);
}  // namespace kv

// int8_kv_ops::prepare known-answer checks (int8_kv_ops.cpp).
void prepare_self_check(ppk_context* ctx);
// hip_attention::validate_split_k known-answer checks (fused_attention.cpp).
void float_attention_self_check(ppk_context* ctx);

}  // namespace ppk
