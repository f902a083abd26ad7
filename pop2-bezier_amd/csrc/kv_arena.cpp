// KV arenas: per-(sequence, layer) caches over shared device arenas with
// copy-on-write snapshots, slot reuse and shared write plans.
//
// Rules follow LayerCache (app/src/model/cache.rs:40-531), the commit path of
// Int8LayerCache (app/src/model/int8_cache.rs:292-359) and BatchWritePlan
// (app/src/model/write_plan.rs:12-102). The storage design is this file's
// own: an arena is one stream-ordered device allocation holding K and V (and
// for int8 the two scale planes) of `batch` sequences x `heads` rows x
// `capacity` slots; a cache owns a Backing = (arena, slot); a write plan is a
// device vector of per-sequence offsets (plus offsets + 1, the attended
// lengths), which the append and attention kernels read directly instead of
// the reference's per-element [B*H, 1, D] index tensor.
#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "ppk_internal.hpp"

namespace {

using ppk::PreconditionError;
using ppk::require;
using ppk::UncertainError;

void check_exec(hipError_t st, const char* what) {
  if (st != hipSuccess) throw UncertainError(std::string(what) + ": " + hipGetErrorString(st));
}

size_t elem_bytes(uint32_t kind) { return kind == PPK_KV_INT8 ? 1 : kind == PPK_KV_F32 ? 4 : 2; }
uint32_t storage_dtype(uint32_t kind) {
  return kind == PPK_KV_F32 ? PPK_F32 : kind == PPK_KV_BF16 ? PPK_BF16 : PPK_F16;
}
size_t align256(size_t n) { return (n + 255) / 256 * 256; }

struct Backing;

// One device allocation: K | V [| K scales | V scales] | offsets (grouped).
struct Arena {
  ppk_context* ctx = nullptr;
  uint32_t kind = 0, heads = 0, head_dim = 0, capacity = 0, batch = 0;
  bool grouped = false;
  bool external = false;  // K and V are caller-owned (an adopted graph view): never freed here
  void* base = nullptr;
  size_t bytes = 0;
  uint8_t* k = nullptr;
  uint8_t* v = nullptr;
  float* ks = nullptr;
  float* vs = nullptr;
  uint32_t* offsets = nullptr;  // grouped: past[batch] then lengths[batch]
  hipStream_t last_stream = nullptr;

  std::mutex mu;
  std::vector<std::weak_ptr<Backing>> owners;  // grouped: one registration per sequence slot
  std::vector<uint32_t> cached_offsets;        // host copy of the uploaded offsets (writes without a plan)
  std::vector<uint32_t> staged;                // upload source, kept alive after the copy is queued
  uint64_t copied_rows = 0, offset_uploads = 0;

  size_t row_bytes() const { return size_t(capacity) * head_dim * elem_bytes(kind); }
  size_t scale_row_bytes() const { return size_t(capacity) * 4; }
  uint8_t* k_rows(uint32_t slot) const { return k + size_t(slot) * heads * row_bytes(); }
  uint8_t* v_rows(uint32_t slot) const { return v + size_t(slot) * heads * row_bytes(); }
  float* ks_rows(uint32_t slot) const { return ks ? ks + size_t(slot) * heads * capacity : nullptr; }
  float* vs_rows(uint32_t slot) const { return vs ? vs + size_t(slot) * heads * capacity : nullptr; }
  size_t slot_bytes() const {
    return 2 * size_t(heads) * (row_bytes() + (kind == PPK_KV_INT8 ? scale_row_bytes() : 0));
  }
  size_t plane_bytes() const { return size_t(batch) * heads * row_bytes(); }
  // Whether [p, p + n) overlaps the arena's storage: the whole allocation,
  // or for an external arena its K and V planes.
  bool contains(const void* p, size_t n) const {
    auto hit = [&](const void* lo, size_t len) {
      const auto a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(lo);
      return len > 0 && n > 0 && a < b + len && b < a + n;
    };
    return external ? hit(k, plane_bytes()) || hit(v, plane_bytes()) : hit(base, bytes);
  }
  bool overlaps(const Arena& o) const {
    return o.external ? contains(o.k, o.plane_bytes()) || contains(o.v, o.plane_bytes()) : contains(o.base, o.bytes);
  }

  ~Arena() {
    if (!base) return;
    ppk::DeviceGuard guard(ctx->device);
    std::vector<ppk_context::CachedBlock> evicted;
    bool kept = false;
    {
      std::lock_guard<std::mutex> lock(ctx->block_mutex);
      // Room for this block: the oldest kept blocks go first (sizes that no
      // later arena asked for age out). They are freed below, after the lock.
      auto& cache = ctx->block_cache;
      while (!cache.empty() && bytes <= ctx->block_cache_limit &&
             ctx->block_cache_bytes + bytes > ctx->block_cache_limit) {
        evicted.push_back(cache.front());
        ctx->block_cache_bytes -= cache.front().bytes;
        cache.erase(cache.begin());
      }
      hipEvent_t ev = nullptr;
      if (ctx->block_cache_bytes + bytes <= ctx->block_cache_limit) {
        if (!ctx->spare_events.empty()) {
          ev = ctx->spare_events.back();
          ctx->spare_events.pop_back();
        } else if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
          ev = nullptr;
        }
      }
      if (ev) {
        if (hipEventRecord(ev, last_stream) == hipSuccess) {
          ctx->block_cache.push_back({base, bytes, ev});
          ctx->block_cache_bytes += bytes;
          kept = true;
        } else {
          (void)hipEventDestroy(ev);
        }
      }
    }
    // Evicted blocks are freed in stream order behind their last use (this
    // stream waits for the event recorded at their release), so neither the
    // host nor other arena calls wait here; the host waits only if the
    // runtime refuses the stream wait.
    for (const auto& b : evicted) {
      if (hipStreamWaitEvent(last_stream, b.released, 0) != hipSuccess) (void)hipEventSynchronize(b.released);
      (void)hipFreeAsync(b.ptr, last_stream);
    }
    if (!evicted.empty()) {
      std::lock_guard<std::mutex> lock(ctx->block_mutex);
      for (const auto& b : evicted) ctx->spare_events.push_back(b.released);
    }
    if (!kept) (void)hipFreeAsync(base, last_stream);
  }
};

struct Backing {
  std::shared_ptr<Arena> arena;
  uint32_t slot = 0;
};

// Allocates and zeroes an arena on `stream` (the reference's Tensor::zeros).
std::shared_ptr<Arena> make_arena(ppk_context* ctx, hipStream_t stream, const PpkKvConfig& cfg, uint32_t capacity,
                                  uint32_t batch, bool grouped) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) == hipSuccess && capture != hipStreamCaptureStatusNone)
    throw PreconditionError("KV arena allocation requested during HIP graph capture");
  auto a = std::make_shared<Arena>();
  a->ctx = ctx;
  a->kind = cfg.kind;
  a->heads = cfg.heads;
  a->head_dim = cfg.head_dim;
  a->capacity = capacity;
  a->batch = batch;
  a->grouped = grouped;
  const size_t plane = align256(size_t(batch) * cfg.heads * a->row_bytes());
  const size_t splane = cfg.kind == PPK_KV_INT8 ? align256(size_t(batch) * cfg.heads * capacity * 4) : 0;
  const size_t offs = grouped ? align256(size_t(batch) * 2 * 4) : 0;
  a->bytes = 2 * plane + 2 * splane + offs;
  ppk::DeviceGuard guard(ctx->device);
  {
    // A released arena of the same size; this stream first waits for the
    // block's last use.
    std::lock_guard<std::mutex> lock(ctx->block_mutex);
    auto& cache = ctx->block_cache;
    for (size_t i = cache.size(); i-- > 0;)
      if (cache[i].bytes == a->bytes) {
        if (hipStreamWaitEvent(stream, cache[i].released, 0) != hipSuccess) break;  // allocate instead
        ctx->spare_events.push_back(cache[i].released);
        a->base = cache[i].ptr;
        ctx->block_cache_bytes -= cache[i].bytes;
        cache.erase(cache.begin() + std::ptrdiff_t(i));
        break;
      }
  }
  if (!a->base) {
    const hipError_t st = ppk::kv::pool_alloc(ctx, &a->base, a->bytes, stream);
    if (st != hipSuccess) {
      a->base = nullptr;
      throw PreconditionError(std::string("KV arena allocation of ") + std::to_string(a->bytes) +
                              " bytes failed: " + hipGetErrorString(st));
    }
  }
  a->last_stream = stream;
  uint8_t* p = static_cast<uint8_t*>(a->base);
  a->k = p;
  a->v = p + plane;
  if (splane) {
    a->ks = reinterpret_cast<float*>(p + 2 * plane);
    a->vs = reinterpret_cast<float*>(p + 2 * plane + splane);
  }
  if (offs) a->offsets = reinterpret_cast<uint32_t*>(p + 2 * plane + 2 * splane);
  if (grouped) a->owners.resize(batch);
  // No memset: the caller fills every row of every slot it hands out (copied
  // prefix + zeros, add_prefix) before the first read, as the reference's
  // zero-initialised storage would read.
  return a;
}

// Initialises slot dst_slot of a new arena: each row receives the first
// `tokens` slots of the matching row of (src, src_slot) (committed history
// only, never the reserve) and zeros up to its capacity; with src null or
// tokens 0 the rows are zeroed. Executed later, all at once, by run_copy_batch.
void add_prefix(std::vector<ppk::CopyDesc>& out, const Arena* src, uint32_t src_slot, const Arena& dst,
                uint32_t dst_slot, uint32_t tokens) {
  if (!src) tokens = 0;
  const uint64_t width = uint64_t(tokens) * dst.head_dim * elem_bytes(dst.kind);
  auto rect = [&](const void* s, uint64_t spitch, void* d, uint64_t dpitch, uint64_t w) {
    ppk::CopyDesc c;
    c.src = tokens ? s : nullptr;
    c.dst = d;
    c.spitch = tokens ? spitch : 0;
    c.dpitch = dpitch;
    c.width = w;
    c.fill = dpitch;
    c.height = dst.heads;
    out.push_back(c);
  };
  rect(src ? src->k_rows(src_slot) : nullptr, src ? src->row_bytes() : 0, dst.k_rows(dst_slot), dst.row_bytes(),
       width);
  rect(src ? src->v_rows(src_slot) : nullptr, src ? src->row_bytes() : 0, dst.v_rows(dst_slot), dst.row_bytes(),
       width);
  if (dst.kind == PPK_KV_INT8) {
    rect(src ? src->ks_rows(src_slot) : nullptr, src ? src->scale_row_bytes() : 0, dst.ks_rows(dst_slot),
         dst.scale_row_bytes(), tokens * 4ull);
    rect(src ? src->vs_rows(src_slot) : nullptr, src ? src->scale_row_bytes() : 0, dst.vs_rows(dst_slot),
         dst.scale_row_bytes(), tokens * 4ull);
  }
}

// A source that lies inside the arena about to be written is copied out
// first (cache.rs:399-416: an input view can alias the arena).
struct SourceSnapshot {
  const void* k;
  const void* v;
  void* tmp = nullptr;
  hipStream_t stream = nullptr;
  SourceSnapshot(const void* k_src, const void* v_src, size_t n, const Arena& dst, hipStream_t s)
      : k(k_src), v(v_src), stream(s) {
    if (!dst.contains(k_src, n) && !dst.contains(v_src, n)) return;
    check_exec(ppk::kv::pool_alloc(dst.ctx, &tmp, 2 * align256(n), s), "hipMallocFromPoolAsync (aliased source)");
    uint8_t* t = static_cast<uint8_t*>(tmp);
    check_exec(hipMemcpyAsync(t, k_src, n, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync (aliased K)");
    check_exec(hipMemcpyAsync(t + align256(n), v_src, n, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync (aliased V)");
    k = t;
    v = t + align256(n);
  }
  ~SourceSnapshot() {
    if (tmp) (void)hipFreeAsync(tmp, stream);
  }
};

void fill_view(PpkKvView* out, const Arena& a, uint32_t slot, uint32_t rows, uint32_t length, uint32_t batch,
               const uint32_t* past, const uint32_t* lengths) {
  if (!out) return;
  require(out->struct_size >= sizeof(PpkKvView), "PpkKvView.struct_size too small");
  const uint32_t size = out->struct_size;
  std::memset(out, 0, sizeof(PpkKvView));
  out->struct_size = size;
  out->kind = a.kind;
  out->rows = rows;
  out->capacity = a.capacity;
  out->head_dim = a.head_dim;
  out->length = length;
  out->batch = batch;
  out->k = a.k_rows(slot);
  out->v = a.v_rows(slot);
  out->k_scales = a.ks_rows(slot);
  out->v_scales = a.vs_rows(slot);
  out->past = past;
  out->lengths = lengths;
}

bool same_config(const PpkKvConfig& a, const PpkKvConfig& b) {
  return a.kind == b.kind && a.heads == b.heads && a.head_dim == b.head_dim && a.max_context == b.max_context &&
         a.min_capacity == b.min_capacity;
}

// A batch write with both sources NULL reserves slot past[b] of every row of
// an int8, bf16 or f32 cache (all of the write's bookkeeping, no data): the
// caller's fused decode step (int8, or the float path's) fills it on the same
// stream. F16 caches have no float decode step (the float attention reads
// bf16 and f32 stores).
bool reserves(const PpkKvWrite& w) { return w.k == nullptr && w.v == nullptr; }

void check_write(const PpkKvConfig& cfg, const PpkKvWrite& w, bool reserve_allowed) {
  require(w.struct_size >= sizeof(PpkKvWrite), "PpkKvWrite.struct_size too small");
  if (reserve_allowed && reserves(w)) {
    require(cfg.kind == PPK_KV_INT8 || cfg.kind == PPK_KV_BF16 || cfg.kind == PPK_KV_F32,
            "a reserving KV write (NULL sources) needs an int8, bf16 or f32 cache");
    return;
  }
  require(w.k && w.v, "KV query null source");
  if (cfg.kind == PPK_KV_INT8)
    require(w.src_dtype == PPK_F32 || w.src_dtype == PPK_BF16 || w.src_dtype == PPK_F16,
            "INT8 KV source dtype must be f32, bf16 or f16");
  else
    require(w.src_dtype == storage_dtype(cfg.kind), "K/V query dtype differs from the cache storage dtype");
  const size_t eb = w.src_dtype == PPK_F32 ? 4 : 2;
  require(reinterpret_cast<uintptr_t>(w.k) % eb == 0 && reinterpret_cast<uintptr_t>(w.v) % eb == 0,
          "KV query source misaligned");
}

uint32_t grown_capacity(const PpkKvConfig& cfg, uint32_t current, uint64_t end) {
  uint64_t c = std::max<uint64_t>(current, std::min(cfg.min_capacity, cfg.max_context));
  while (c < end) c = std::min<uint64_t>(c * 2, cfg.max_context);
  return uint32_t(c);
}

}  // namespace

struct ppk_kv_cache {
  ppk_context* ctx = nullptr;
  PpkKvConfig cfg{};
  std::shared_ptr<Backing> backing;
  uint32_t committed = 0;
};

struct ppk_write_plan {
  ppk_context* ctx = nullptr;
  std::vector<uint32_t> offsets;
  std::vector<uint32_t> staged;  // past then lengths, the upload source
  uint32_t heads = 0, head_dim = 0;
  uint32_t* dev = nullptr;
  size_t bytes = 0;
  hipStream_t stream = nullptr;
  hipEvent_t released = nullptr;  // the vector's event, carried from buffer to buffer
  // The device vector goes back to the context's pool (up to 8 kept) for the
  // next plan on the same stream, with an event recorded here that the next
  // plan's stream waits for; beyond that it is freed in stream order.
  ~ppk_write_plan() {
    if (!dev) return;
    ppk::DeviceGuard guard(ctx->device);
    if (!released && hipEventCreateWithFlags(&released, hipEventDisableTiming) != hipSuccess) released = nullptr;
    if (released && hipEventRecord(released, stream) == hipSuccess) {
      std::lock_guard<std::mutex> lock(ctx->plan_mutex);
      if (ctx->plan_pool.size() < 8) {
        ctx->plan_pool.push_back({dev, bytes, stream, released});
        return;
      }
    }
    if (released) (void)hipEventDestroy(released);
    (void)hipFreeAsync(dev, stream);
  }
};

namespace ppk::kv {

uint64_t drain_blocks(ppk_context* ctx) {
  DeviceGuard guard(ctx->device);
  std::vector<ppk_context::CachedBlock> blocks;
  {
    std::lock_guard<std::mutex> lock(ctx->block_mutex);
    blocks.swap(ctx->block_cache);
    ctx->block_cache_bytes = 0;
  }
  uint64_t freed = 0;
  for (auto& b : blocks) {
    (void)hipEventSynchronize(b.released);  // the block's last use has finished
    (void)hipFree(b.ptr);
    freed += b.bytes;
    std::lock_guard<std::mutex> lock(ctx->block_mutex);
    ctx->spare_events.push_back(b.released);
  }
  if (ctx->mem_pool) (void)hipMemPoolTrimTo(ctx->mem_pool, 0);
  return freed;
}

hipError_t pool_alloc(ppk_context* ctx, void** ptr, size_t bytes, hipStream_t stream) {
  hipError_t st = hipMallocFromPoolAsync(ptr, bytes, ctx->mem_pool, stream);
  if (st == hipSuccess) return st;
  // The failure is reported through this library's status; leave no HIP
  // error behind for the caller's next launch check to pick up.
  (void)hipGetLastError();
  *ptr = nullptr;
  bool kept = false;
  {
    std::lock_guard<std::mutex> lock(ctx->block_mutex);
    kept = !ctx->block_cache.empty();
  }
  if (st != hipErrorOutOfMemory || !kept) return st;
  drain_blocks(ctx);
  st = hipMallocFromPoolAsync(ptr, bytes, ctx->mem_pool, stream);
  if (st != hipSuccess) {
    (void)hipGetLastError();
    *ptr = nullptr;
  }
  return st;
}

ppk_kv_cache* create(ppk_context* ctx, const PpkKvConfig& in) {
  require(ctx != nullptr, "KV cache needs a context");
  require(in.struct_size >= sizeof(PpkKvConfig), "PpkKvConfig.struct_size too small");
  PpkKvConfig cfg = in;
  cfg.struct_size = sizeof(PpkKvConfig);
  if (cfg.max_context == 0) cfg.max_context = 1024;
  if (cfg.min_capacity == 0) cfg.min_capacity = 64;
  require(cfg.kind <= PPK_KV_F32, "unknown KV cache kind");
  require(cfg.heads > 0 && cfg.head_dim > 0, "KV cache heads and head_dim must be nonzero");
  if (cfg.kind == PPK_KV_INT8)
    require(cfg.head_dim == 64 || cfg.head_dim == 128 || cfg.head_dim == 256,
            "INT8 KV cache head_dim must be 64, 128 or 256");
  require(cfg.max_context <= (1u << 24), "KV cache max_context too large");
  require(uint64_t(cfg.heads) * cfg.max_context * cfg.head_dim * 4 <= (uint64_t(1) << 40),
          "KV cache dimensions overflow");
  auto* c = new ppk_kv_cache();
  c->ctx = ctx;
  c->cfg = cfg;
  return c;
}

void info(const ppk_kv_cache& c, PpkKvInfo* out) {
  require(out && out->struct_size >= sizeof(PpkKvInfo), "PpkKvInfo missing or struct_size too small");
  const uint32_t size = out->struct_size;
  std::memset(out, 0, sizeof(PpkKvInfo));
  out->struct_size = size;
  out->length = c.committed;
  if (!c.backing) return;
  const Arena& a = *c.backing->arena;
  out->capacity = a.capacity;
  out->grouped = a.grouped ? 1 : 0;
  out->slot = c.backing->slot;
  out->shared = c.backing.use_count() > 1 ? 1 : 0;
  out->reserved_bytes = a.slot_bytes();
  out->scale_bytes = a.kind == PPK_KV_INT8 ? 2 * uint64_t(a.heads) * a.scale_row_bytes() : 0;
  out->storage_id = reinterpret_cast<uintptr_t>(c.backing.get());
  out->arena_id = reinterpret_cast<uintptr_t>(&a);
  std::lock_guard<std::mutex> lock(c.backing->arena->mu);
  out->arena_copied_rows = a.copied_rows;
  out->arena_offset_uploads = a.offset_uploads;
}

void view(const ppk_kv_cache& c, PpkKvView* out) {
  require(out && out->struct_size >= sizeof(PpkKvView), "PpkKvView missing or struct_size too small");
  if (!c.backing) {
    const uint32_t size = out->struct_size;
    std::memset(out, 0, sizeof(PpkKvView));
    out->struct_size = size;
    out->kind = c.cfg.kind;
    out->head_dim = c.cfg.head_dim;
    out->rows = c.cfg.heads;
    return;
  }
  fill_view(out, *c.backing->arena, c.backing->slot, c.cfg.heads, c.committed, 0, nullptr, nullptr);
}

void truncate(ppk_kv_cache& c, uint32_t new_len) {
  require(new_len <= c.committed, "KV metadata truncation cannot extend committed history");
  c.committed = new_len;
}

// LayerCache::adopt_graph_view (cache.rs:55-64): caller-owned f32 K and V of
// [heads, capacity, head_dim] become the storage of a new cache holding
// committed_len tokens. Writes that fit go into that memory in place; growth
// or copy-on-write moves the cache into storage of its own, as for any cache.
ppk_kv_cache* adopt(ppk_context* ctx, const PpkKvConfig& in, void* k, void* v, uint32_t capacity,
                    uint32_t committed_len) {
  require(in.struct_size >= sizeof(PpkKvConfig), "PpkKvConfig.struct_size too small");
  require(in.kind == PPK_KV_F32 && in.heads > 0 && in.head_dim > 0, "invalid graph KV view");
  std::unique_ptr<ppk_kv_cache> c(create(ctx, in));
  const PpkKvConfig& cfg = c->cfg;
  const size_t plane = size_t(cfg.heads) * capacity * cfg.head_dim * 4;
  const auto kp = reinterpret_cast<uintptr_t>(k), vp = reinterpret_cast<uintptr_t>(v);
  require(k && v && kp % 4 == 0 && vp % 4 == 0 && committed_len <= capacity && capacity <= cfg.max_context &&
              (plane == 0 || kp + plane <= vp || vp + plane <= kp),
          "invalid graph KV view");
  auto a = std::make_shared<Arena>();
  a->ctx = ctx;
  a->kind = cfg.kind;
  a->heads = cfg.heads;
  a->head_dim = cfg.head_dim;
  a->capacity = capacity;
  a->batch = 1;
  a->external = true;
  a->k = static_cast<uint8_t*>(k);
  a->v = static_cast<uint8_t*>(v);
  auto backing = std::make_shared<Backing>();
  backing->arena = std::move(a);
  c->backing = std::move(backing);
  c->committed = committed_len;
  return c.release();
}

// LayerCache::advance_graph_length (cache.rs:66-73): the graph wrote slot
// `previous`; the committed length moves by exactly one, metadata only.
void advance(ppk_kv_cache& c, uint32_t previous, uint32_t next) {
  require(c.committed == previous && uint64_t(next) == uint64_t(previous) + 1 && c.backing &&
              next <= c.backing->arena->capacity,
          "graph KV commit length differs from validated host state");
  c.committed = next;
}

// LayerCache::query (cache.rs:194-283), Int8LayerCache::query (int8_cache.rs:313-323).
void query(ppk_context* ctx, hipStream_t stream, ppk_kv_cache& c, uint32_t past, const PpkKvWrite& w,
           PpkKvView* out) {
  require(ctx == c.ctx, "KV cache belongs to another context");
  check_write(c.cfg, w, false);
  if (past != c.committed)
    throw PreconditionError("KV past_len " + std::to_string(past) + " differs from the committed length " +
                            std::to_string(c.committed));
  require(w.tokens > 0, "KV query dimensions must be nonzero");
  const uint64_t end = uint64_t(past) + w.tokens;
  if (end > c.cfg.max_context)
    throw PreconditionError("KV capacity is " + std::to_string(c.cfg.max_context) + ", the query needs " +
                            std::to_string(end) + "; rebuild the context first");
  if (out) require(out->struct_size >= sizeof(PpkKvView), "PpkKvView.struct_size too small");
  const uint32_t current = c.backing ? c.backing->arena->capacity : 0;
  const uint32_t capacity = grown_capacity(c.cfg, current, end);
  // Validation done; device work from here on.
  DeviceGuard guard(ctx->device);
  // Shared with a snapshot (Arc::strong_count > 1, cache.rs:249-251): counted
  // before `target` takes its own reference.
  const bool shared = c.backing && c.backing.use_count() > 1;
  std::shared_ptr<Backing> target = c.backing;
  if (!target || capacity > current || shared) {
    auto arena = make_arena(ctx, stream, c.cfg, capacity, 1, false);
    auto fresh = std::make_shared<Backing>();
    fresh->arena = arena;
    fresh->slot = 0;
    std::vector<CopyDesc> copies;
    add_prefix(copies, target ? target->arena.get() : nullptr, target ? target->slot : 0, *arena, 0, c.committed);
    run_copy_batch(ctx, stream, copies);
    if (target) target->arena->last_stream = stream;  // its free must follow the copy
    target = fresh;
  }
  Arena& a = *target->arena;
  const size_t src_bytes = size_t(c.cfg.heads) * w.tokens * c.cfg.head_dim *
                           (c.cfg.kind == PPK_KV_INT8 ? (w.src_dtype == PPK_F32 ? 4 : 2) : elem_bytes(c.cfg.kind));
  SourceSnapshot src(w.k, w.v, src_bytes, a, stream);
  ArenaWrite aw;
  aw.k_src = src.k;
  aw.v_src = src.v;
  aw.src_dtype = w.src_dtype;
  aw.k = a.k_rows(target->slot);
  aw.v = a.v_rows(target->slot);
  aw.ks = a.ks_rows(target->slot);
  aw.vs = a.vs_rows(target->slot);
  aw.uniform_past = past;
  aw.sequences = 1;
  aw.heads = c.cfg.heads;
  aw.tokens = w.tokens;
  aw.capacity = a.capacity;
  aw.head_dim = c.cfg.head_dim;
  aw.elem_bytes = c.cfg.kind == PPK_KV_INT8 ? 0 : uint32_t(elem_bytes(c.cfg.kind));
  run_arena_write(ctx, stream, aw);
  a.last_stream = stream;
  c.backing = target;
  if (w.commit) c.committed = uint32_t(end);
  fill_view(out, a, target->slot, c.cfg.heads, uint32_t(end), 0, nullptr, nullptr);
}

ppk_write_plan* plan_create(ppk_context* ctx, hipStream_t stream, const uint32_t* past_lens, uint32_t batch,
                            uint32_t heads, uint32_t head_dim) {
  require(ctx != nullptr, "write plan needs a context");
  require(past_lens && batch > 0 && heads > 0 && head_dim > 0,
          "write plan requires nonempty rows, heads and width");
  require(uint64_t(batch) * heads * head_dim * 4 <= (uint64_t(1) << 40), "write plan index count overflow");
  for (uint32_t b = 0; b < batch; ++b)
    require(past_lens[b] < 0xffffffffu, "write plan offsets must leave a slot inside the maximum context");
  auto plan = std::make_unique<ppk_write_plan>();
  plan->ctx = ctx;
  plan->offsets.assign(past_lens, past_lens + batch);
  plan->heads = heads;
  plan->head_dim = head_dim;
  plan->staged.resize(2 * size_t(batch));
  for (uint32_t b = 0; b < batch; ++b) {
    plan->staged[b] = past_lens[b];
    plan->staged[batch + b] = past_lens[b] + 1;
  }
  DeviceGuard guard(ctx->device);
  const size_t bytes = align256(2 * size_t(batch) * 4);
  {
    std::lock_guard<std::mutex> lock(ctx->plan_mutex);
    auto& pool = ctx->plan_pool;
    for (size_t i = 0; i < pool.size(); ++i)
      if (pool[i].stream == stream && pool[i].bytes >= bytes &&
          hipStreamWaitEvent(stream, pool[i].released, 0) == hipSuccess) {
        plan->dev = pool[i].dev;
        plan->bytes = pool[i].bytes;
        plan->released = pool[i].released;
        pool.erase(pool.begin() + std::ptrdiff_t(i));
        break;
      }
  }
  if (!plan->dev) {
    void* dev = nullptr;
    const hipError_t st = pool_alloc(ctx, &dev, bytes, stream);
    if (st != hipSuccess)
      throw PreconditionError(std::string("write plan allocation failed: ") + hipGetErrorString(st));
    plan->dev = static_cast<uint32_t*>(dev);
    plan->bytes = bytes;
  }
  plan->stream = stream;
  check_exec(hipMemcpyAsync(plan->dev, plan->staged.data(), 2 * size_t(batch) * 4, hipMemcpyHostToDevice, stream),
             "hipMemcpyAsync (write plan)");
  return plan.release();
}

namespace {

// reusable_batch_group (cache.rs:484-531): the first grouped arena among the
// caches is reused only if every row is provably its own: grouped rows sit
// at their own slot with no other owner, and any other row may take over a
// slot that nothing (not even a detached snapshot) still owns.
std::shared_ptr<Arena> reusable_arena(ppk_kv_cache* const* caches, uint32_t batch, uint32_t capacity,
                                      std::vector<uint32_t>& changed) {
  std::shared_ptr<Arena> candidate;
  for (uint32_t b = 0; b < batch && !candidate; ++b)
    if (caches[b]->backing && caches[b]->backing->arena->grouped) candidate = caches[b]->backing->arena;
  if (!candidate) return nullptr;
  if (candidate->batch != batch || candidate->capacity != capacity) return nullptr;
  std::lock_guard<std::mutex> lock(candidate->mu);
  if (candidate->owners.size() != batch) return nullptr;
  changed.clear();
  for (uint32_t row = 0; row < batch; ++row) {
    const std::shared_ptr<Backing>& backing = caches[row]->backing;
    if (backing) {
      if (backing->arena->grouped) {
        if (backing->arena != candidate || backing->slot != row || backing.use_count() != 1) return nullptr;
        const bool registered = candidate->owners[row].lock().get() == backing.get();
        if (!registered) return nullptr;
        continue;
      }
      // Only an independent same-capacity row may take an orphaned slot; a
      // view that aliases the candidate's storage (an adopted graph view over
      // its rows) may not (cache.rs:513-519).
      if (backing->arena->capacity != capacity || candidate->overlaps(*backing->arena)) return nullptr;
    }
    if (!candidate->owners[row].expired()) return nullptr;
    changed.push_back(row);
  }
  return candidate;
}

}  // namespace

// LayerCache::query_batch_with_plan (cache.rs:301-482) and Int8LayerCache::query_batch
// (int8_cache.rs:325-359): one token per sequence into one batch arena.
void query_batch(ppk_context* ctx, hipStream_t stream, ppk_kv_cache* const* caches, uint32_t batch,
                 const uint32_t* past_lens, const PpkKvWrite& w, const ppk_write_plan* plan, PpkKvView* out) {
  require(caches && past_lens && batch > 0, "batch KV requires nonempty [B,H,1,D]");
  for (uint32_t b = 0; b < batch; ++b) require(caches[b] != nullptr, "batch KV null cache");
  const PpkKvConfig& cfg = caches[0]->cfg;
  for (uint32_t b = 0; b < batch; ++b) {
    require(caches[b]->ctx == ctx, "KV cache belongs to another context");
    require(same_config(caches[b]->cfg, cfg), "batch KV existing row is incompatible");
    for (uint32_t o = 0; o < b; ++o) require(caches[o] != caches[b], "batch KV rows must be distinct caches");
  }
  check_write(cfg, w, true);
  require(w.tokens == 1, "batch KV requires one query token per row");
  if (out) require(out->struct_size >= sizeof(PpkKvView), "PpkKvView.struct_size too small");
  if (plan) {
    require(plan->ctx == ctx, "write plan device differs from the current KV device");
    // The plan's vector was uploaded on its own stream and is recycled in that
    // stream's order: another stream could read it before the upload lands, or
    // while a later plan overwrites it.
    require(plan->stream == stream, "write plan was created on another stream");
    require(plan->offsets.size() == batch && std::equal(plan->offsets.begin(), plan->offsets.end(), past_lens) &&
                plan->heads == cfg.heads && plan->head_dim == cfg.head_dim,
            "write plan key does not match the current row offsets and head shape");
  }
  uint32_t capacity = std::min(cfg.min_capacity, cfg.max_context);
  uint64_t max_end = 0;
  for (uint32_t b = 0; b < batch; ++b) {
    const ppk_kv_cache& c = *caches[b];
    require(past_lens[b] == c.committed, "batch KV supplied past length differs from committed history");
    const uint64_t end = uint64_t(past_lens[b]) + 1;
    require(end <= cfg.max_context, "batch KV needs context rebuild");
    max_end = std::max(max_end, end);
    if (c.backing) {
      require(past_lens[b] <= c.backing->arena->capacity, "batch KV existing row is incompatible");
      capacity = std::max(capacity, c.backing->arena->capacity);
    } else {
      require(past_lens[b] == 0, "batch KV committed row has no storage");
    }
  }
  capacity = grown_capacity(cfg, capacity, max_end);
  require(uint64_t(batch) * cfg.heads * capacity * cfg.head_dim * 4 <= (uint64_t(1) << 40),
          "batch KV arena too large");
  // Validation done; device work from here on.
  DeviceGuard guard(ctx->device);
  std::vector<uint32_t> changed;
  std::shared_ptr<Arena> arena = reusable_arena(caches, batch, capacity, changed);
  if (!arena) {
    arena = make_arena(ctx, stream, cfg, capacity, batch, true);
    changed.resize(batch);
    for (uint32_t b = 0; b < batch; ++b) changed[b] = b;
  }
  Arena& a = *arena;
  const size_t src_bytes = size_t(batch) * cfg.heads * cfg.head_dim *
                           (cfg.kind == PPK_KV_INT8 ? (w.src_dtype == PPK_F32 ? 4 : 2) : elem_bytes(cfg.kind));
  const bool reserve = reserves(w);
  SourceSnapshot src(w.k, w.v, reserve ? 0 : src_bytes, a, stream);
  std::vector<std::shared_ptr<Backing>> replacements;
  replacements.reserve(changed.size());
  std::vector<CopyDesc> copies;
  uint64_t copied = 0;
  for (uint32_t row : changed) {
    const ppk_kv_cache& c = *caches[row];
    // Every slot handed out is initialised: committed prefix (if any) + zeros.
    // A reused arena's orphaned slot holds the old owner's data, which the
    // reference keeps until overwritten; it is rewritten the same way here.
    add_prefix(copies, c.backing && c.committed ? c.backing->arena.get() : nullptr,
               c.backing ? c.backing->slot : 0, a, row, c.committed);
    if (c.committed > 0) ++copied;
    auto fresh = std::make_shared<Backing>();
    fresh->arena = arena;
    fresh->slot = row;
    replacements.push_back(fresh);
  }
  run_copy_batch(ctx, stream, copies);
  for (uint32_t row : changed)
    if (caches[row]->committed > 0) caches[row]->backing->arena->last_stream = stream;  // frees follow the copies
  const uint32_t* past_dev = nullptr;
  const uint32_t* lengths_dev = nullptr;
  {
    std::lock_guard<std::mutex> lock(a.mu);
    a.copied_rows += copied;
    if (plan) {
      past_dev = plan->dev;
      lengths_dev = plan->dev + batch;
    } else {
      if (a.cached_offsets.size() != batch || !std::equal(a.cached_offsets.begin(), a.cached_offsets.end(), past_lens)) {
        a.cached_offsets.assign(past_lens, past_lens + batch);
        a.staged.resize(2 * size_t(batch));
        for (uint32_t b = 0; b < batch; ++b) {
          a.staged[b] = past_lens[b];
          a.staged[batch + b] = past_lens[b] + 1;
        }
        check_exec(hipMemcpyAsync(a.offsets, a.staged.data(), 2 * size_t(batch) * 4, hipMemcpyHostToDevice, stream),
                   "hipMemcpyAsync (KV offsets)");
        ++a.offset_uploads;
      }
      past_dev = a.offsets;
      lengths_dev = a.offsets + batch;
    }
  }
  ArenaWrite aw;
  aw.k_src = src.k;
  aw.v_src = src.v;
  aw.src_dtype = w.src_dtype;
  aw.k = a.k;
  aw.v = a.v;
  aw.ks = a.ks;
  aw.vs = a.vs;
  aw.past = past_dev;
  aw.sequences = batch;
  aw.heads = cfg.heads;
  aw.tokens = 1;
  aw.capacity = a.capacity;
  aw.head_dim = cfg.head_dim;
  aw.elem_bytes = cfg.kind == PPK_KV_INT8 ? 0 : uint32_t(elem_bytes(cfg.kind));
  if (!reserve) run_arena_write(ctx, stream, aw);
  a.last_stream = stream;
  {
    std::lock_guard<std::mutex> lock(a.mu);
    for (size_t i = 0; i < changed.size(); ++i) {
      a.owners[changed[i]] = replacements[i];
      caches[changed[i]]->backing = replacements[i];
    }
  }
  if (w.commit)
    for (uint32_t b = 0; b < batch; ++b) caches[b]->committed = past_lens[b] + 1;
  fill_view(out, a, 0, batch * cfg.heads, uint32_t(max_end), batch, past_dev, lengths_dev);
}

ppk_kv_cache* clone(const ppk_kv_cache& c) { return new ppk_kv_cache(c); }
void release(ppk_kv_cache* c) { delete c; }
void plan_release(ppk_write_plan* p) { delete p; }

}  // namespace ppk::kv
