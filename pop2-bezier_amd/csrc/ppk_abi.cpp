// C-ABI shim over the gfx950 code object: context/module management,
// argument validation (status 1, nothing enqueued), stream-ordered launches
// (status 3 once a launch was attempted) and optional event tracing.
//
// Conventions follow the reference C-ABI: status codes and thread-local last
// error (app/native/aten_hip/cpp/painter_ffi.h:20-25, painter_ffi.cpp:12-29);
// validation of every span before the first enqueue (app/src/model/hip_attention.rs:63-88).
#include <dlfcn.h>

#include <cstddef>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>

#include "ppk_internal.hpp"

namespace {

thread_local std::string g_last_error;

template <class Op>
int32_t call(Op&& op) {
  g_last_error.clear();
  try {
    op();
    return PPK_OK;
  } catch (const ppk::PreconditionError& e) {
    g_last_error = e.what();
    if (g_last_error.size() > 6000) g_last_error.resize(6000);
    return PPK_PRECONDITION;
  } catch (const ppk::InvalidOutputError& e) {
    g_last_error = e.what();
    if (g_last_error.size() > 6000) g_last_error.resize(6000);
    return PPK_INVALID_OUTPUT;
  } catch (const ppk::UncertainError& e) {
    g_last_error = e.what();
    if (g_last_error.size() > 6000) g_last_error.resize(6000);
    return PPK_EXECUTION_UNCERTAIN;
  } catch (const std::exception& e) {
    g_last_error = std::string("HIP_EXECUTION_UNCERTAIN: ") + e.what();
    if (g_last_error.size() > 6000) g_last_error.resize(6000);
    return PPK_EXECUTION_UNCERTAIN;
  } catch (...) {
    g_last_error = "HIP_EXECUTION_UNCERTAIN: unrecognised native exception";
    return PPK_EXECUTION_UNCERTAIN;
  }
}

const char* kFnNames[ppk::kFnCount] = {
    "ppk_quantize_d64", "ppk_quantize_d128", "ppk_quantize_d256", "ppk_dequantize",
    "ppk_decode_d64", "ppk_decode_d128", "ppk_decode_d256",
    "ppk_decode_bf16h_d64", "ppk_decode_bf16h_d128", "ppk_decode_bf16h_d256",
    "ppk_attn_merge_d64", "ppk_attn_merge_d128", "ppk_attn_merge_d256",
    "ppk_fdecode_bf16_d64", "ppk_fdecode_bf16_d128", "ppk_fdecode_bf16_d256",
    "ppk_fdecode_f32_d64", "ppk_fdecode_f32_d128", "ppk_fdecode_f32_d256",
    "ppk_fmerge_d64", "ppk_fmerge_d128", "ppk_fmerge_d256",
    "ppk_renyi_sample",
    "ppk_kv_scatter_u16", "ppk_kv_scatter_u4", "ppk_kv_scatter_u2",
    "ppk_copy2d_batch",
    "ppk_quantize_dense_d64", "ppk_quantize_dense_d128", "ppk_quantize_dense_d256",
    "ppk_quantize_append_d64", "ppk_quantize_append_d128", "ppk_quantize_append_d256",
    "ppk_decode_flat_d64", "ppk_decode_flat_d128", "ppk_decode_flat_d256",
    "ppk_decode_flat_bf16h_d64", "ppk_decode_flat_bf16h_d128", "ppk_decode_flat_bf16h_d256",
    "ppk_attn_merge_flat_d64", "ppk_attn_merge_flat_d128", "ppk_attn_merge_flat_d256",
    "ppk_fdecode_flat_bf16_d64", "ppk_fdecode_flat_bf16_d128", "ppk_fdecode_flat_bf16_d256",
    "ppk_fdecode_flat_f32_d64", "ppk_fdecode_flat_f32_d128", "ppk_fdecode_flat_f32_d256",
    "ppk_fmerge_flat_d64", "ppk_fmerge_flat_d128", "ppk_fmerge_flat_d256",
    "ppk_fstep_bf16_d64", "ppk_fstep_bf16_d128", "ppk_fstep_bf16_d256",
    "ppk_fstep_f32_d64", "ppk_fstep_f32_d128", "ppk_fstep_f32_d256",
    "ppk_fstep_flat_bf16_d64", "ppk_fstep_flat_bf16_d128", "ppk_fstep_flat_bf16_d256",
    "ppk_fstep_flat_f32_d64", "ppk_fstep_flat_f32_d128", "ppk_fstep_flat_f32_d256",
};

std::string default_code_object() {
  Dl_info info{};
  if (dladdr(reinterpret_cast<void*>(&ppk_abi_version), &info) == 0 || !info.dli_fname)
    throw ppk::PreconditionError("cannot locate libppk to find the default code object");
  std::string path(info.dli_fname);
  const auto slash = path.find_last_of('/');
  path = (slash == std::string::npos) ? std::string(".") : path.substr(0, slash);
  return path + "/ppk_kernels.hsaco";
}

void check_prep(hipError_t status, const char* what) {
  if (status != hipSuccess) throw ppk::PreconditionError(std::string(what) + ": " + hipGetErrorString(status));
}

int dim_index(uint32_t head_dim) {
  switch (head_dim) {
    case 64: return 0;
    case 128: return 1;
    case 256: return 2;
    default: throw ppk::PreconditionError("head_dim must be 64, 128 or 256, got " + std::to_string(head_dim));
  }
}

bool valid_dtype(uint32_t t) { return t == PPK_F32 || t == PPK_BF16 || t == PPK_F16; }
size_t dtype_bytes(uint32_t t) { return t == PPK_F32 ? 4 : 2; }
bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

template <class Args>
void launch(ppk_context* ctx, int prof_kernel, ppk::Fn fn, uint32_t grid, uint32_t block, uint32_t lds,
            hipStream_t stream, Args& args, uint32_t grid_y = 1, bool traceable = true) {
  void* params[] = {&args};
  ppk::EventPair ev;
  bool traced = false;
  if (traceable && ctx->profiling) {
    std::lock_guard<std::mutex> lock(ctx->prof_mutex);
    if (ctx->pool.empty()) {
      if (hipEventCreate(&ev.start) != hipSuccess || hipEventCreate(&ev.stop) != hipSuccess)
        throw ppk::PreconditionError("hipEventCreate failed for tracing");
    } else {
      ev = ctx->pool.back();
      ctx->pool.pop_back();
    }
    traced = true;
  }
  if (traced && hipEventRecord(ev.start, stream) != hipSuccess)
    throw ppk::UncertainError(std::string("event record before ") + kFnNames[fn]);
  const hipError_t st =
      hipModuleLaunchKernel(ctx->fn[fn], grid, grid_y, 1, block, 1, 1, lds, stream, params, nullptr);
  if (st != hipSuccess) throw ppk::UncertainError(std::string(kFnNames[fn]) + ": " + hipGetErrorString(st));
  if (traced) {
    if (hipEventRecord(ev.stop, stream) != hipSuccess)
      throw ppk::UncertainError(std::string("event record after ") + kFnNames[fn]);
    std::lock_guard<std::mutex> lock(ctx->prof_mutex);
    ctx->pending[prof_kernel].push_back(ev);
  }
}

}  // namespace

namespace ppk {

DeviceGuard::DeviceGuard(int device) {
  if (hipGetDevice(&previous_) != hipSuccess) previous_ = -1;
  if (previous_ != device) {
    const hipError_t st = hipSetDevice(device);
    if (st != hipSuccess) throw PreconditionError(std::string("hipSetDevice: ") + hipGetErrorString(st));
    changed_ = true;
  }
}
DeviceGuard::~DeviceGuard() {
  if (changed_ && previous_ >= 0) (void)hipSetDevice(previous_);
}

AttentionPlan plan_rows(const ppk_context* ctx, uint32_t rows, uint64_t span, uint32_t explicit_split,
                        uint32_t tpl, uint64_t token_bytes, uint32_t head_dim, uint32_t min_split,
                        uint32_t block_waves) {
  AttentionPlan plan;
  plan.head_dim = head_dim;
  uint32_t split;
  if (explicit_split) {
    split = std::min<uint32_t>(std::max<uint32_t>(explicit_split, tpl), 8192u);
    split = (split + tpl - 1) / tpl * tpl;
  } else {
    // Smallest power-of-two tokens per wave (>= 64) that keeps the launch
    // within about eight waves per CU (two per SIMD), all resident at once:
    // each wave streams one long contiguous stretch of K and of V. Measured
    // on MI355X against 16- and 32-wave-per-CU budgets, fewer longer streams
    // read faster (config 5: 164.7 vs 166.8 us; config 4: 23.6 vs 24.9 us).
    const uint64_t budget = uint64_t(std::max(ctx ? ctx->cu_count : 256, 1)) * 8;
    split = 64;
    while (split < 2048 && uint64_t(rows) * ((span + split - 1) / split) > budget) split <<= 1;
    // Then as many waves per row as the budget holds (up to 16, none under
    // 64 tokens), each with an equal share rounded up to whole tiles, instead
    // of full splits and a short last one: the longest wave sets the time.
    // Measured on MI355X (H = 16, D = 64 / 128, per step, power-of-two splits
    // -> equal shares filling the budget), int8: B = 32 x 1100 tokens, 18.4 /
    // 30.1 -> 16.2 / 25.6 us; x 3000, 36.0 / 64.6 -> 34.8 / 64.2 us; x 5000,
    // 59.8 / 112.0 -> 55.4 / 102.3 us; B = 16 x 1500, 12.5 / 20.3 -> 12.0 /
    // 18.2 us. Float, bf16: B = 16 x 1500, 16.0 / 30.4 -> 14.4 / 29.0 us;
    // x 4000, 40.4 / 79.4 -> 39.3 / 77.2 us; B = 32 x 3000, 58.1 / 117.4 ->
    // 57.8 / 114.7 us; B = 32 x 1100 and B = 64 x 600 within 1.5 % (f32 the
    // same within 2 %). B = 32 x 8192 (config 5) is unchanged: its splits
    // are already equal and the budget full.
    uint64_t waves = std::max<uint64_t>(1, (span + split - 1) / split);
    const uint64_t fill = std::min<uint64_t>(16, budget / std::max<uint64_t>(rows, 1));
    waves = std::max<uint64_t>(waves, std::min<uint64_t>(fill, (span + 63) / 64));
    if (waves > block_waves && span * token_bytes <= (128u << 10)) {
      // A row that one block covers gets at most block_waves waves, each
      // streaming a longer share (int8: 8, the kernels bounded to 512 threads
      // with three batches in flight; 9 to 16 waves of 64 tokens in one block
      // measured 17 % slower on one box: 64 rows x 900 tokens at D = 64, 15
      // waves of 64 tokens 9.09 us, 8 waves of 128 tokens 7.53 us; 16 rows x
      // 960, 9.15 -> 7.49 us; 128 rows x 900, 9.53 -> 8.26 us).
      waves = block_waves;
      split = uint32_t(std::max<uint64_t>(((span + waves - 1) / waves + tpl - 1) / tpl * tpl, tpl));
    } else {
      const uint64_t share = ((span + waves - 1) / waves + tpl - 1) / tpl * tpl;
      split = uint32_t(std::min<uint64_t>(split, std::max<uint64_t>(share, tpl)));
    }
  }
  uint64_t waves_per_row = std::max<uint64_t>(1, (span + split - 1) / split);
  // Up to block_waves waves per block; one float of LDS per history token of the block.
  uint64_t max_waves = std::max<uint64_t>(1, std::min<uint64_t>(block_waves, 16384 / split));
  const uint64_t cus = uint64_t(std::max(ctx ? ctx->cu_count : 256, 1));
  const uint64_t row_bytes = span * token_bytes;
  if (!explicit_split && rows < cus && row_bytes > (128u << 10)) {
    // Few, long rows: one block per row would leave most CUs idle (a CU
    // alone streams only a few tens of GB/s). Split rows into blocks of about
    // 256 KiB of history, then shrink blocks until the launch covers every CU;
    // the merge kernel joins the groups. (Config 4 against a 64 KiB target:
    // three-wave blocks and 4 records per row instead of one-wave blocks and
    // 12, 2 % faster warm and cold.)
    // The int8 kernels hold two waves per SIMD, eight per CU: blocks of 1, 2,
    // 4 or 8 waves fill a CU's slots, while blocks of 3, 5, 6 or 7 leave some
    // empty and can push the grid into a second round (32 rows x 8192 tokens
    // at D = 128: 7-wave blocks, 320 of them on 256 CUs, 25.3 us; 4-wave
    // blocks, one round, 17.0 us). The float kernels hold more waves per CU
    // and take any block size.
    const bool pow2 = block_waves <= kInt8WavesPerCu;
    auto fit = [&](uint64_t w) {
      uint64_t p = 1;
      while (pow2 && p * 2 <= w) p *= 2;
      return pow2 ? p : w;
    };
    auto shrink = [&](uint64_t w) { return pow2 ? w / 2 : w - 1; };
    const uint64_t wave_bytes = uint64_t(split) * token_bytes;
    uint64_t w = fit(std::max<uint64_t>(1, std::min<uint64_t>(max_waves, (256u << 10) / wave_bytes)));
    while (w > 1 && rows * ((waves_per_row + w - 1) / w) < cus) w = shrink(w);
    // Blocks of fewer than four waves leave SIMDs of their CU idle while the
    // waves work through their tokens (config 3: one 2-wave block of 64-token
    // waves per CU, 1.56 us of arithmetic per wave after its data arrived).
    // Halve the waves' share, down to min_split tokens and within the wave
    // budget, so that each block gets four: config 3 at D = 128, 32-token
    // waves in 4-wave blocks, 218.0 -> 194.9 us per 24-layer step in a
    // same-box A/B.
    const uint64_t budget = cus * 8;
    while (w < 4 && min_split && split / 2 >= min_split && split % 2 == 0 && (split / 2) % tpl == 0 &&
           rows * ((span + split / 2 - 1) / (split / 2)) <= budget) {
      split /= 2;
      waves_per_row = std::max<uint64_t>(1, (span + split - 1) / split);
      max_waves = std::max<uint64_t>(1, std::min<uint64_t>(block_waves, 16384 / split));
      w = fit(std::max<uint64_t>(1, std::min<uint64_t>(max_waves, (256u << 10) / (uint64_t(split) * token_bytes))));
      while (w > 1 && rows * ((waves_per_row + w - 1) / w) < cus) w = shrink(w);
    }
    // Larger blocks where they land evenly: the row's waves split exactly
    // into the blocks, and the busiest CU runs at most 7 % more waves than
    // the mean (fewer records to merge, fewer block joins). Same-box A/B, H
    // = 16, int8 D = 128: 128 rows x 8192 tokens, 1-wave -> 8-wave blocks,
    // 50.4 -> 44.9 us; 32 x 16384 28.97 -> 25.2; 64 x 8192 27.2 -> 25.6; 96 x
    // 8192 40.3 -> 38.4; 160 x 8192 58.9 -> 55.6; config 4 17.3 -> 17.0; D =
    // 64, 128 x 16384 51.2 -> 48.2; bf16 store, 64 rows x 8192 at D = 64 26.2
    // -> 23.4, 64 x 4096 at D = 128 24.2 -> 22.8; of 52 shapes it changes
    // five lost 0.2-0.5 us and one ragged batch (host lengths, 192 rows of
    // 1422-7798 tokens) 1.4 us of 50. Blocks that land unevenly lost 5-10 %
    // (48 rows x 8192, 2 -> 4-wave blocks: the busiest CUs 8 waves against a
    // mean of 6).
    for (uint64_t u = fit(max_waves); u > w; u = shrink(u)) {
      const uint64_t g = (waves_per_row + u - 1) / u, wv = (waves_per_row + g - 1) / g, nb = rows * g;
      if (nb < cus || g * wv != waves_per_row || (pow2 && nb > cus * (kInt8WavesPerCu / wv))) continue;
      if (100 * ((nb + cus - 1) / cus) * wv * cus <= 107 * rows * waves_per_row) {
        w = u;
        break;
      }
    }
    // int8: a grid whose blocks do not all fit the CUs' eight wave slots at
    // once runs a second round, and its merge launch waits for the last one.
    // When eight waves of a longer share cover each row, one block per row
    // runs in one round with no merge launch, though some CUs stay idle;
    // otherwise the blocks shrink until the grid fits. Same-box A/B of the
    // two-round grid -> one block per row (-> the shrunk blocks), H = 16:
    // 160 rows x 1024 tokens at D = 128 21.1 -> 12.5 (13.5) us, 192 x 1500
    // at D = 128 20.9 -> 15.0 (17.3), 192 x 2048 at D = 128 25.9 -> 18.5
    // (21.5), 224 x 4096 at D = 128 49.8 -> 37.4 (40.4), 160 x 2048 at D =
    // 64 20.9 -> 12.3 (13.4), 224 x 2048 at D = 64 20.8 -> 13.0 (15.6), 192
    // x 4096 at D = 64 26.1 -> 18.8 (21.6), 224 x 8192 at D = 64 51.8 ->
    // 40.1 (41.8). Grids that fit one round keep their plan: one block per
    // row would idle more CUs than a merge costs (192 x 8192 at D = 128
    // splits ten ways, 67.6 us).
    auto blocks = [&](uint64_t n) { return rows * ((waves_per_row + n - 1) / n); };
    if (pow2 && blocks(w) > cus * (kInt8WavesPerCu / w)) {
      const uint64_t whole = std::max<uint64_t>(
          1, ((span + block_waves - 1) / block_waves + tpl - 1) / tpl * tpl);  // 8 waves cover a row
      if (rows * block_waves <= budget && whole * block_waves <= 16384) {
        split = uint32_t(whole);
        waves_per_row = std::max<uint64_t>(1, (span + split - 1) / split);
        w = block_waves;
      } else {
        while (w > 1 && blocks(w) > cus * (kInt8WavesPerCu / w)) w /= 2;
      }
    }
    // And smaller blocks where the chosen ones land unevenly (the busiest CU
    // more than 7 % over the mean) and smaller ones land evenly: the largest
    // such, at most 16 a row (the merge's first pass) and one-wave blocks
    // only at four or more a CU (fewer leave SIMDs idle). Same-box A/B, H =
    // 16, int8: 80 rows x 1024 tokens at D = 128, four 4-wave blocks a row
    // -> sixteen 1-wave, 11.80 -> 10.71 us; 96 x 1024 at D = 64 9.34 -> 8.65;
    // 48 x 4096 at D = 64 11.54 -> 10.83; 96 x 4096 at D = 64 15.51 ->
    // 14.92; bf16 store, 144 rows x 1500 at D = 64 14.67 -> 10.94, 160 x 1500
    // 14.43 -> 11.40; of 31 shapes it changes two lost 0.3 and 0.4 us
    // (80 and 112 rows x 8192 at D = 64), and of 30 float-store shapes one
    // lost (112 x 4096 at D = 128, 38.2 -> 40.3 us) while 29 gained 2-22 %.
    // Without the 16-block bound, 16-32 rows took 47 blocks a row and lost
    // 5-12 %.
    {
      auto even = [&](uint64_t u) {
        const uint64_t g = (waves_per_row + u - 1) / u, wv = (waves_per_row + g - 1) / g, nb = rows * g;
        return nb >= cus && g * wv == waves_per_row && !(pow2 && nb > cus * (kInt8WavesPerCu / wv)) &&
               100 * ((nb + cus - 1) / cus) * wv * cus <= 107 * rows * waves_per_row;
      };
      if (waves_per_row > w && !even(w))
        for (uint64_t u = w > 1 ? shrink(w) : 1; u >= 1 && u < w; u = shrink(u)) {
          if ((waves_per_row + u - 1) / u > 16) break;
          if (even(u) && (u >= 2 || rows * waves_per_row >= 4 * cus)) {
            w = u;
            break;
          }
          if (u == 1) break;
        }
    }
    max_waves = w;
  }
  // At least as many rows as CUs, one block per row: a CU runs the blocks
  // of ceil(rows / CUs) rows while the mean is rows / CUs, and a CU alone
  // streams only ~35 GB/s. int8 blocks of a row's 3, 5, 6 or 7 waves (the
  // budget split over 288-640 rows) also hold only one or two per CU and
  // run a second round. Two remedies: a power-of-two number of waves per
  // row in one block (int8, two-round grids only: no merge, the busiest CUs
  // still stream one row more than the mean), or the row's waves in
  // smaller blocks that spread evenly over the CUs, joined by the merge
  // kernel. The first pays while the busiest CUs' excess is at most 160
  // KiB. The second pays where the excess is larger and the busiest CUs
  // carry at most 1/0.85 of the mean (beyond that HBM, not the busiest CUs,
  // sets the time: 448 rows, 1.75 of 2, lost 2-4 % with it). Same-box A/B,
  // H = 16, previous plan -> this rule (the other remedy, int8): D = 128,
  // int8, 288 rows x 1024 tokens 25.2 -> 17.1 (19.0) us, x 4096 72.1 ->
  // 51.3 (65.1), x 8192 133.7 -> 97.3 (125.4); 320 x 8192 143.9 -> 107.8
  // (128.6); 384 x 1024 27.7 -> 19.8 (21.3), x 8192 158.7 -> 130.4
  // (135.0); 640 x 4096 120.5 -> 110.0 (115.7); D = 64, 384 x 1024 19.5 ->
  // 12.9 (15.4); 288 x 8192 74.3 -> 53.9 (67.5); of 36 int8 shapes measured
  // both ways the rule took the slower remedy on three, by 0.6-0.9 us.
  // bf16 float store, D = 128: 288 x 4096 121.3 -> 91.6, x 8192 239.8 ->
  // 177.5; 320 x 8192 251.3 -> 195.5; 384 x 8192 252.4 -> 240.8; 576 x 4096
  // 211.3 -> 186.7; 640 x 4096 216.9 -> 209.5; D = 64 288 x 8192 123.5 ->
  // 93.8; 576 x 1024 25.0 -> 25.7 (the one loss measured).
  if (!explicit_split && rows >= cus && rows * waves_per_row <= cus * 8) {
    const bool int8 = block_waves <= kInt8WavesPerCu;
    const uint64_t limit = cus * (160u << 10);
    const uint64_t per_cu = (rows + cus - 1) / cus;
    auto groups = [&](uint64_t mw) { return (waves_per_row + mw - 1) / mw; };
    auto fits = [&](uint64_t mw) {
      const uint64_t g = groups(mw), wv = (waves_per_row + g - 1) / g;
      return !int8 || rows * g <= cus * (kInt8WavesPerCu / wv);
    };
    auto excess = [&](uint64_t mw) {  // bytes, times the CU count
      const uint64_t g = groups(mw), wv = (waves_per_row + g - 1) / g, blocks = rows * g;
      return (((blocks + cus - 1) / cus) * cus - blocks) * wv * split * token_bytes;
    };
    const bool two_rounds = !fits(max_waves);
    if (two_rounds && (per_cu * cus - rows) * row_bytes <= limit) {
      uint64_t p = 1;
      while (p * 2 <= waves_per_row) p *= 2;
      split = uint32_t(std::max<uint64_t>(((span + p - 1) / p + tpl - 1) / tpl * tpl, tpl));
      waves_per_row = std::max<uint64_t>(1, (span + split - 1) / split);
      max_waves = std::max<uint64_t>(1, std::min<uint64_t>(block_waves, 16384 / split));
    } else if (two_rounds || (excess(max_waves) > limit && 20 * rows <= 17 * per_cu * cus)) {
      // The largest blocks (powers of two for int8) within the excess, else
      // the smallest excess.
      uint64_t w = max_waves;
      if (int8) {
        w = 1;
        while (w * 2 <= max_waves) w *= 2;
      }
      uint64_t best = w, best_x = ~uint64_t(0);
      for (;;) {
        if (fits(w)) {
          const uint64_t x = excess(w);
          if (x <= limit) {
            best = w;
            break;
          }
          if (x < best_x) {
            best_x = x;
            best = w;
          }
        }
        if (w == 1) break;
        w = int8 ? w / 2 : w - 1;
      }
      max_waves = best;
    }
  }
  plan.split = split;
  if (waves_per_row <= max_waves) {
    plan.waves = uint32_t(waves_per_row);
    plan.ngroups = 1;
  } else {
    // The fewest blocks of at most max_waves waves, then the waves spread
    // evenly over them (16 waves in blocks of 5 are four blocks of 4, not
    // 5 + 5 + 5 + 1, whose last block would leave its CU idle early).
    plan.ngroups = uint32_t((waves_per_row + max_waves - 1) / max_waves);
    plan.waves = uint32_t((waves_per_row + plan.ngroups - 1) / plan.ngroups);
  }
  require(uint64_t(plan.ngroups) * rows <= 0x7fffffffu, "attention grid too large");
  // Per wave: one log2-domain score per token; after the waves are done the
  // same LDS holds one (m, z, pad, pad, y[D]) record per wave.
  plan.lds_bytes = 4u * std::max<uint32_t>(plan.waves * split, plan.waves * (head_dim + 4u));
  if (plan.ngroups > 1) {
    plan.y_bytes = (uint64_t(rows) * plan.ngroups * head_dim * 4 + 255) / 256 * 256;
    plan.mz_bytes = (uint64_t(rows) * plan.ngroups * 2 * 4 + 255) / 256 * 256;
  }
  plan.workspace_bytes = plan.y_bytes + plan.mz_bytes;
  return plan;
}

// The attention argument block up to workspace_bytes is required; past_host
// (added later) is read only when struct_size covers it.
constexpr size_t kAttentionArgsMin = offsetof(PpkAttentionArgs, past_host);
const uint32_t* host_lengths(const PpkAttentionArgs& a) {
  return a.struct_size >= offsetof(PpkAttentionArgs, past_host) + sizeof(a.past_host) ? a.past_host : nullptr;
}

AttentionPlan plan_attention(const ppk_context* ctx, const PpkAttentionArgs& a) {
  require(a.struct_size >= kAttentionArgsMin, "PpkAttentionArgs.struct_size too small");
  dim_index(a.head_dim);
  require(valid_dtype(a.q_dtype) && valid_dtype(a.scratch_dtype) && valid_dtype(a.out_dtype),
          "INT8 attention dtype must be f32, bf16 or f16");
  require((a.flags & ~uint32_t(PPK_ATTN_BF16_HISTORY | kPlanFlags)) == 0, "unknown INT8 attention flags");
  require((a.flags & kPlanFlags) != kPlanFlags, "INT8 attention plan flags PER_ROW and BALANCED both set");
  require(a.heads > 0 && a.rows > 0 && a.rows % a.heads == 0, "INT8 attention geometry differs: rows % heads");
  require(a.capacity > 0, "INT8 attention capacity must be positive");
  require(uint64_t(a.capacity) * a.head_dim <= (uint64_t(1) << 40), "INT8 attention capacity too large");
  require(a.max_past <= a.capacity, "max_past exceeds capacity");
  require(std::isfinite(a.softmax_scale) && a.softmax_scale >= 0.f, "softmax_scale must be finite and >= 0");

  const uint32_t tpl = 64u / (a.head_dim / 16u);
  const uint64_t span = a.max_past ? a.max_past : a.capacity;
  const uint32_t* host = host_lengths(a);
  const uint64_t limit = std::min<uint64_t>(a.capacity, span);
  // Per history token: K and V codes plus two fp32 scales. With the host's
  // lengths (and no plan bit) the per-row plan covers the longest live row
  // instead of the whole span, so no waves are sized for history no row
  // holds; a device length beyond that coverage (a stale host copy) gives
  // NaN rows and PPK_FLAG_STALE_LENGTHS in a decode step.
  const uint64_t cover = host && !(a.flags & kPlanFlags) ? row_cover(host, a.rows / a.heads, limit) : span;
  // The int8 waves' shortest share: one batch (four load tiles).
  AttentionPlan plan =
      plan_rows(ctx, a.rows, cover, a.split_tokens, tpl, 2ull * a.head_dim + 8, a.head_dim, 4 * tpl, 8);
  // With the host's lengths of a ragged batch, the balanced plan gives every
  // wave the same share of the live history; balanced_pays picks between the
  // two plans from a timing model of both.
  if (a.flags & PPK_ATTN_PLAN_BALANCED) {
    require_balanced(ctx, a.rows, a.heads, host, a.split_tokens);
    plan = plan_flat(ctx, a.rows, a.heads, host, limit, a.head_dim);
    plan.span = uint32_t(span);
  } else if (!(a.flags & PPK_ATTN_PLAN_PER_ROW) && host && a.split_tokens == 0 &&
             flat_pays(ctx, a.rows, a.heads, host, limit)) {
    AttentionPlan flat = plan_flat(ctx, a.rows, a.heads, host, limit, a.head_dim);
    if (balanced_pays(ctx, plan, flat, a.rows, a.heads, host, limit, 2ull * a.head_dim + 8)) {
      plan = flat;
      plan.span = uint32_t(span);
    }
  }
  if (!plan.flat) {
    plan.speculate = per_row_speculates(plan, a.rows, a.heads, host, cover, limit);
    plan.span = uint32_t(span);
  }
  return plan;
}

uint64_t row_cover(const uint32_t* host, uint32_t batch, uint64_t limit) {
  return std::max<uint64_t>(longest_live(host, batch, limit), 1);
}

bool per_row_speculates(const AttentionPlan& p, uint32_t rows, uint32_t heads, const uint32_t* host, uint64_t span,
                        uint64_t limit) {
  const uint64_t per_row = uint64_t(p.ngroups) * p.waves;
  uint64_t live = 0;
  for (uint32_t b = 0; b < rows / heads; ++b) {
    const uint64_t len = host ? (host[b] <= limit ? host[b] : 0) : span;
    live += heads * std::min<uint64_t>(per_row, (len + p.split - 1) / p.split);
  }
  const uint64_t total = per_row * rows;
  return (total - live) * 16 < total;
}

// Placement model of an all-resident launch: block i runs on CU i mod cus
// (the dispatcher deals blocks round-robin over the XCDs and, within one,
// over its CUs). Returns the most live history tokens one CU streams.
uint64_t per_row_cu_peak(const AttentionPlan& p, uint32_t rows, uint32_t heads, const uint32_t* host,
                         uint64_t limit, uint32_t cus) {
  std::vector<uint64_t> load(cus, 0);
  const uint64_t per_block = uint64_t(p.waves) * p.split;  // tokens of a row one block covers
  for (uint32_t r = 0; r < rows; ++r) {
    const uint64_t len = host[r / heads] <= limit ? host[r / heads] : 0;
    for (uint64_t g = 0; g < p.ngroups && g * per_block < len; ++g)  // blocks numbered group-major
      load[(g * rows + r) % cus] += std::min(per_block, len - g * per_block);
  }
  return *std::max_element(load.begin(), load.end());
}

uint64_t flat_cu_peak(const AttentionPlan& p, uint32_t heads, uint32_t cus) {
  std::vector<uint64_t> load(cus, 0);
  const FlatTable& t = p.table;
  uint64_t unit = 0;  // unit u on block u / waves (the int8 kernel's assignment)
  for (uint32_t b = 0; b < t.batch; ++b)
    for (uint32_t h = 0; h < heads; ++h)
      for (uint32_t s = 0; s < t.units[b]; ++s, ++unit) {
        const uint64_t t0 = uint64_t(s) * t.share;
        if (t.len[b] > t0) load[(unit / p.waves) % cus] += std::min<uint64_t>(t.share, t.len[b] - t0);
      }
  return *std::max_element(load.begin(), load.end());
}

// Modelled duration in microseconds of an int8 attention launch plan on
// MI355X: a fixed cost, plus the whole live history streamed at `stream`
// bytes/us per CU (a partition of the device has its share), plus the
// busiest CU's bytes beyond the mean at `excess` bytes/us. Fitted per plan
// kind (least squares on the relative error) to 140 ragged batches measured
// with both plans forced on one box (B = 4 .. 64, H = 16, D = 64 / 128;
// uniform U[lo, hi] draws and long rows beside short ones): taking the
// plan the model favours (and the long-wave rule of balanced_pays) lost
// 34.8 us over the 140 steps against always taking the faster one, with 6
// picks more than 2 % slower; the single max(stream, busiest CU) model it
// replaces, fitted before the per-row plan's larger blocks, lost 59.8 us
// with 24.
struct PlanCost {
  double one_launch, with_merge, stream, excess;
};
constexpr PlanCost kPerRowCost{4.75, 7.3, 27.8e3, 64e3};
constexpr PlanCost kBalancedCost{7.0, 9.9, 27.2e3, 63e3};
static double modelled_us(const PlanCost& c, uint64_t total_bytes, uint64_t cu_peak_bytes, bool merge,
                          uint32_t cus) {
  const double mean = double(total_bytes) / cus;
  return (merge ? c.with_merge : c.one_launch) + double(total_bytes) / (c.stream * cus) +
         std::max(0.0, double(cu_peak_bytes) - mean) / c.excess;
}

bool balanced_pays(const ppk_context* ctx, const AttentionPlan& per_row, const AttentionPlan& flat, uint32_t rows,
                   uint32_t heads, const uint32_t* host, uint64_t limit, uint64_t token_bytes) {
  const uint32_t cus = uint32_t(std::max(ctx ? ctx->cu_count : 256, 1));
  const uint64_t row_peak = per_row_cu_peak(per_row, rows, heads, host, limit, cus);
  const uint64_t flat_peak = flat_cu_peak(flat, heads, cus);
  uint64_t total = 0;
  for (uint32_t b = 0; b < rows / heads; ++b) total += host[b] <= limit ? host[b] : 0;
  total *= uint64_t(heads) * token_bytes;
  const double t_row = modelled_us(kPerRowCost, total, row_peak * token_bytes, per_row.ngroups > 1, cus);
  const double t_flat = modelled_us(kBalancedCost, total, flat_peak * token_bytes, flat.ngroups > 1, cus);
  // Balanced when the model has it faster; and when per-row
  // waves would each stream 256 KiB or more and the per-row plan's busiest CU
  // streams at least 1.2 x the balanced plan's (long waves run below the
  // modelled CU rate: 8 x 4096 beside 24 x 1024 tokens at D = 128 measured
  // 53.2 us per-row, 45.2 us balanced).
  return t_flat < t_row ||
         (uint64_t(per_row.split) * token_bytes >= (256u << 10) && 5 * row_peak >= 6 * flat_peak);
}

bool per_row_waves_uneven(uint32_t batch, const uint32_t* host, uint64_t limit, uint32_t split) {
  uint64_t tokens = 0, waves = 0, most = 0;
  for (uint32_t b = 0; b < batch; ++b) {
    const uint64_t len = host[b] <= limit ? host[b] : 0;
    tokens += len;
    waves += (len + split - 1) / split;
    most = std::max(most, std::min<uint64_t>(len, split));
  }
  return waves > 0 && most * waves * 10 > tokens * 11;
}

uint64_t longest_live(const uint32_t* host, uint32_t batch, uint64_t limit) {
  uint64_t most = 0;
  for (uint32_t b = 0; b < batch; ++b)
    if (host[b] <= limit) most = std::max<uint64_t>(most, host[b]);
  return most;
}

bool flat_fits(const ppk_context* ctx, uint32_t rows, uint32_t heads) {
  const uint64_t flat_waves = uint64_t(std::max(ctx ? ctx->cu_count : 256, 1)) * kFlatWavesPerCu;
  return rows / heads <= uint32_t(kFlatMaxBatch) && 2 * uint64_t(rows) <= flat_waves;
}

void require_balanced(const ppk_context* ctx, uint32_t rows, uint32_t heads, const uint32_t* host,
                      uint32_t split_tokens) {
  require(host != nullptr, "PPK_ATTN_PLAN_BALANCED needs the host lengths");
  require(split_tokens == 0, "PPK_ATTN_PLAN_BALANCED needs split_tokens == 0");
  if (!flat_fits(ctx, rows, heads))
    throw PreconditionError("PPK_ATTN_PLAN_BALANCED: at most 64 sequences and 4 rows per CU, got " +
                            std::to_string(rows / heads) + " sequences of " + std::to_string(heads) + " rows");
}

bool flat_pays(const ppk_context* ctx, uint32_t rows, uint32_t heads, const uint32_t* host, uint64_t limit) {
  const uint32_t batch = rows / heads;
  if (!flat_fits(ctx, rows, heads)) return false;
  uint64_t sum = 0, most = 0;
  for (uint32_t b = 0; b < batch; ++b) {
    const uint64_t live = host[b] <= limit ? host[b] : 0;
    sum += live;
    most = std::max(most, live);
  }
  return most * batch * 10 > sum * 11;  // the longest row beyond 1.1 x the mean
}

// Balanced plan (ragged batches with host lengths): eight waves per CU, all
// resident; units of at most Q tokens of one row, Q the least share (>= 64)
// for which the units, sum over rows of max(1, ceil(len / Q)), fit the
// waves; in the int8 decode step waves 0 .. 2 rows - 1 also append the
// current tokens (so waves >= 2 rows).
// Record slots per row = the most units of any row (none when every row is
// one unit: then the decode launch writes every output and no merge runs).
AttentionPlan plan_flat(const ppk_context* ctx, uint32_t rows, uint32_t heads, const uint32_t* host, uint64_t limit,
                        uint32_t head_dim) {
  constexpr uint32_t kWavesPerBlock = 4, kMinUnit = 64;
  AttentionPlan plan;
  plan.head_dim = head_dim;
  plan.flat = true;
  plan.waves = kWavesPerBlock;
  const uint64_t cus = uint64_t(std::max(ctx ? ctx->cu_count : 256, 1));
  plan.blocks = uint32_t(cus * kFlatWavesPerCu / kWavesPerBlock);
  const uint64_t waves = uint64_t(plan.blocks) * kWavesPerBlock;
  require(rows % heads == 0 && rows / heads <= uint32_t(kFlatMaxBatch) && 2 * uint64_t(rows) <= waves,
          "balanced plan: batch or rows beyond its limits");
  FlatTable& t = plan.table;
  t.batch = rows / heads;
  uint64_t total = 0;
  for (uint32_t b = 0; b < t.batch; ++b) {
    t.past[b] = host[b];
    t.len[b] = host[b] <= limit ? host[b] : 0u;
    total += uint64_t(t.len[b]) * heads;
  }
  // The least share whose units fit the waves: units(Q) = sum over rows of
  // max(1, ceil(len / Q)) falls as Q grows, and Q = ceil(T / (waves - rows))
  // always fits (units <= T / Q + rows), so a binary search between 64 and it.
  auto units_for = [&](uint64_t q) {
    uint64_t u = 0;
    for (uint32_t b = 0; b < t.batch; ++b) u += uint64_t(heads) * std::max<uint64_t>(1, (t.len[b] + q - 1) / q);
    return u;
  };
  const uint64_t spare = waves - rows;
  uint64_t lo = kMinUnit, hi = std::max<uint64_t>((total + spare - 1) / spare, kMinUnit);
  while (lo < hi) {
    const uint64_t mid = (lo + hi) / 2;
    if (units_for(mid) <= waves) hi = mid;
    else lo = mid + 1;
  }
  t.share = uint32_t(lo);
  uint64_t first = 0;
  uint32_t most = 1;
  for (uint32_t b = 0; b < uint32_t(kFlatMaxBatch); ++b) {
    if (b >= t.batch) {
      t.first[b] = 0xffffffffu;
      continue;
    }
    t.units[b] = std::max<uint32_t>(1, (t.len[b] + t.share - 1) / t.share);
    t.first[b] = uint32_t(first);
    first += uint64_t(t.units[b]) * heads;
    most = std::max(most, t.units[b]);
  }
  require(first <= waves, "balanced plan: units exceed the launched waves");
  t.units_total = uint32_t(first);
  plan.split = t.share;
  plan.ngroups = most;
  plan.lds_bytes = 0;
  if (most > 1) {
    plan.y_bytes = (uint64_t(rows) * most * head_dim * 4 + 255) / 256 * 256;
    plan.mz_bytes = (uint64_t(rows) * most * 2 * 4 + 255) / 256 * 256;
  }
  plan.workspace_bytes = plan.y_bytes + plan.mz_bytes;
  return plan;
}

// The streaming quantize kernel (dense or append): one 16-byte load per lane
// covers 16 bytes of a source row, so every source must be 16-byte aligned
// and every code array aligned to the 8 (4 for f32 sources) codes a lane
// stores; rows of all tensors are indexed in 32 bits. Batches of 4 units per
// lane, one batch per lane up to 128 blocks of 256 lanes per CU. Returns
// false (nothing launched) when the operands do not fit these conditions.
bool launch_stream_quantize(ppk_context* ctx, hipStream_t stream, int prof_kernel, QuantizeArgs k,
                            uint32_t head_dim) {
  const uint32_t per_lane = k.src_dtype == PPK_F32 ? 4u : 8u;
  for (uint32_t t = 0; t < k.ntensors; ++t)
    if (!aligned(k.src[t], 16) || !aligned(k.codes[t], per_lane)) return false;
  if (uint64_t(k.rows) * k.ntensors >= (uint64_t(1) << 32)) return false;
  const uint64_t units = uint64_t(k.ntensors) * k.rows * (head_dim / per_lane);
  // Below one full block per CU (e.g. a decode round's single-token appends)
  // the one-wave-per-row kernel spreads the rows wider and finishes sooner.
  const uint64_t cus = uint64_t(std::max(ctx->cu_count, 1));
  if (units < cus * 1024) return false;
  const uint64_t grid = std::min<uint64_t>((units + 1023) / 1024, cus * 128);
  const Fn fn = Fn((k.capacity ? kQuantizeAppend64 : kQuantizeDense64) + dim_index(head_dim));
  launch(ctx, prof_kernel, fn, uint32_t(grid), 256, 0, stream, k);
  return true;
}

void run_quantize(ppk_context* ctx, hipStream_t stream, const PpkQuantizeArgs& a) {
  require(a.struct_size >= sizeof(PpkQuantizeArgs), "PpkQuantizeArgs.struct_size too small");
  const int di = dim_index(a.head_dim);
  require(valid_dtype(a.src_dtype), "INT8 KV source dtype must be f32, bf16 or f16");
  require(a.rows > 0, "INT8 KV requires dense [heads,tokens,D] with heads*tokens > 0");
  require(a.rows <= (uint64_t(1) << 36), "INT8 KV dimensions overflow");
  require(a.src && a.codes && a.scales, "INT8 KV null pointer");
  require(aligned(a.src, dtype_bytes(a.src_dtype)) && aligned(a.codes, 4) && aligned(a.scales, 4) &&
              (!a.flags || aligned(a.flags, 4)),
          "INT8 KV operand misaligned");
  QuantizeArgs k{};
  k.src[0] = a.src;
  k.codes[0] = a.codes;
  k.scales[0] = a.scales;
  k.flags = a.flags;
  k.rows = a.rows;
  k.src_dtype = a.src_dtype;
  k.ntensors = 1;
  DeviceGuard guard(ctx->device);
  if (launch_stream_quantize(ctx, stream, PPK_KERNEL_QUANTIZE, k, a.head_dim)) return;
  const uint64_t grid = (a.rows + 3) / 4;
  require(grid <= 0x7fffffffu, "INT8 KV quantize grid too large");
  launch(ctx, PPK_KERNEL_QUANTIZE, Fn(kQuantize64 + di), uint32_t(grid), 256, 0, stream, k);
}

void run_append(ppk_context* ctx, hipStream_t stream, const PpkAppendArgs& a) {
  require(a.struct_size >= sizeof(PpkAppendArgs), "PpkAppendArgs.struct_size too small");
  const int di = dim_index(a.head_dim);
  require(valid_dtype(a.src_dtype), "INT8 KV source dtype must be f32, bf16 or f16");
  require(a.batch > 0 && a.heads > 0 && a.tokens > 0 && a.capacity > 0,
          "INT8 batch requires [B,H,tokens,D] scratch with B, H, tokens, capacity > 0");
  require(a.k_src && a.v_src && a.past && a.k_codes && a.v_codes && a.k_scales && a.v_scales,
          "INT8 append null pointer");
  require(aligned(a.k_src, dtype_bytes(a.src_dtype)) && aligned(a.v_src, dtype_bytes(a.src_dtype)) &&
              aligned(a.k_codes, 4) && aligned(a.v_codes, 4) && aligned(a.k_scales, 4) &&
              aligned(a.v_scales, 4) && aligned(a.past, 4) && (!a.flags || aligned(a.flags, 4)),
          "INT8 append operand misaligned");
  const uint64_t rows = uint64_t(a.batch) * a.heads * a.tokens;
  require(rows <= (uint64_t(1) << 36), "INT8 physical head rows overflow");
  QuantizeArgs k{};
  k.src[0] = a.k_src;
  k.src[1] = a.v_src;
  k.codes[0] = a.k_codes;
  k.codes[1] = a.v_codes;
  k.scales[0] = a.k_scales;
  k.scales[1] = a.v_scales;
  k.past = a.past;
  k.flags = a.flags;
  k.rows = rows;
  k.heads = a.heads;
  k.tokens = a.tokens;
  k.capacity = a.capacity;
  k.src_dtype = a.src_dtype;
  k.ntensors = 2;
  const uint64_t grid = (2 * rows + 3) / 4;
  require(grid <= 0x7fffffffu, "INT8 append grid too large");
  DeviceGuard guard(ctx->device);
  if (launch_stream_quantize(ctx, stream, PPK_KERNEL_APPEND, k, a.head_dim)) return;
  launch(ctx, PPK_KERNEL_APPEND, Fn(kQuantize64 + di), uint32_t(grid), 256, 0, stream, k);
}

void run_dequantize(ppk_context* ctx, hipStream_t stream, const PpkDequantizeArgs& a) {
  require(a.struct_size >= sizeof(PpkDequantizeArgs), "PpkDequantizeArgs.struct_size too small");
  dim_index(a.head_dim);
  require(valid_dtype(a.out_dtype), "INT8 dequantize dtype must be f32, bf16 or f16");
  require(a.rows > 0 && a.rows <= (uint64_t(1) << 36), "INT8 dequantize rows out of range");
  require(a.codes && a.scales && a.out, "INT8 dequantize null pointer");
  require(aligned(a.codes, 16) && aligned(a.out, 16) && aligned(a.scales, 4), "INT8 dequantize operand misaligned");
  DequantizeArgs k{};
  k.codes = a.codes;
  k.scales = a.scales;
  k.out = a.out;
  k.rows = a.rows;
  k.head_dim = a.head_dim;
  k.out_dtype = a.out_dtype;
  k.round_bf16 = a.round_bf16 ? 1u : 0u;
  // One lane per 16-byte output chunk (8 codes, or 4 for f32) and batches of
  // 8 chunks per lane: one batch per lane, up to 128 blocks of 256 lanes per
  // CU, beyond which lanes loop over a grid-stride range.
  constexpr uint64_t kBlocksPerCu = 128, kChunksPerBatch = 8;
  const uint64_t chunks = a.rows * a.head_dim / (a.out_dtype == PPK_F32 ? 4 : 8);
  const uint64_t grid = std::min<uint64_t>((chunks + 256 * kChunksPerBatch - 1) / (256 * kChunksPerBatch),
                                           uint64_t(std::max(ctx->cu_count, 1)) * kBlocksPerCu);
  DeviceGuard guard(ctx->device);
  launch(ctx, PPK_KERNEL_DEQUANTIZE, kDequantize, uint32_t(grid), 256, 0, stream, k);
}

void run_attention(ppk_context* ctx, hipStream_t stream, const PpkAttentionArgs& a, const PpkDecodeStepArgs* step,
                   void* scratch, uint64_t scratch_bytes) {
  const AttentionPlan plan = plan_attention(ctx, a);
  require(a.q && a.k_codes && a.v_codes && a.k_scales && a.v_scales && a.sk && a.sv && a.past && a.out,
          "INT8 attention null pointer");
  require(aligned(a.k_codes, 16) && aligned(a.v_codes, 16), "INT8 codes must be 16-byte aligned");
  require(aligned(a.k_scales, 4) && aligned(a.v_scales, 4) && aligned(a.past, 4), "INT8 scales/lengths misaligned");
  require(aligned(a.q, dtype_bytes(a.q_dtype)) && aligned(a.sk, dtype_bytes(a.scratch_dtype)) &&
              aligned(a.sv, dtype_bytes(a.scratch_dtype)) && aligned(a.out, dtype_bytes(a.out_dtype)),
          "INT8 attention float operand misaligned");
  void* workspace = a.workspace;
  if (scratch) {
    if (plan.workspace_bytes > scratch_bytes)
      throw PreconditionError("INT8 decode step needs " + std::to_string(plan.workspace_bytes) +
                              " bytes of workspace; the no-alloc scratch holds " + std::to_string(scratch_bytes));
    workspace = scratch;
  } else if (plan.workspace_bytes) {
    require(a.workspace && aligned(a.workspace, 256), "INT8 attention workspace missing or not 256-byte aligned");
    if (a.workspace_bytes < plan.workspace_bytes)
      throw PreconditionError("INT8 attention workspace too small: need " + std::to_string(plan.workspace_bytes) +
                              " bytes");
  }
  if (step) {
    require(step->struct_size >= offsetof(PpkDecodeStepArgs, attn) + kAttentionArgsMin,
            "PpkDecodeStepArgs.struct_size too small");
    require(valid_dtype(step->new_dtype), "INT8 decode step new-token dtype must be f32, bf16 or f16");
    require(step->k_new && step->v_new, "INT8 decode step null new-token pointer");
    require(aligned(step->k_new, dtype_bytes(step->new_dtype)) && aligned(step->v_new, dtype_bytes(step->new_dtype)) &&
                (!step->flags || aligned(step->flags, 4)),
            "INT8 decode step operand misaligned");
  }
  const int di = dim_index(a.head_dim);
  const float scale = a.softmax_scale > 0.f ? a.softmax_scale : 1.0f / std::sqrt(float(a.head_dim));
  const float scale_log2 = scale * 1.4426950408889634f;

  DecodeArgs d{};
  d.q = a.q;
  // The arenas are written only by the fused append, at slot past[b].
  d.k = const_cast<uint8_t*>(a.k_codes);
  d.v = const_cast<uint8_t*>(a.v_codes);
  d.ks = const_cast<float*>(a.k_scales);
  d.vs = const_cast<float*>(a.v_scales);
  d.sk = a.sk;
  d.sv = a.sv;
  d.past = a.past;
  d.part_y = plan.workspace_bytes ? static_cast<float*>(workspace) : nullptr;
  d.part_mz = plan.workspace_bytes ? reinterpret_cast<float*>(static_cast<char*>(workspace) + plan.y_bytes) : nullptr;
  d.out = a.out;
  if (step) {
    d.k_new = step->k_new;
    d.v_new = step->v_new;
    d.flags = step->flags;
    d.new_dtype = step->new_dtype;
    d.append = 1;
  }
  d.rows = a.rows;
  d.heads = a.heads;
  d.capacity = a.capacity;
  d.split_tokens = plan.split;
  d.ngroups = plan.ngroups;
  d.q_dtype = a.q_dtype;
  d.scratch_dtype = a.scratch_dtype;
  d.out_dtype = a.out_dtype;
  d.scale_log2 = scale_log2;
  d.speculate = plan.speculate ? 1u : 0u;
  d.span = plan.span;
  if (ctx && ctx->wave_clock) {
    std::lock_guard<std::mutex> lock(ctx->prof_mutex);
    d.clock = ctx->wave_clock;
    d.clock_seq = ctx->wave_clock_seq++;
    d.clock_cap = ctx->wave_clock_cap;
  }

  const bool bf16h = (a.flags & PPK_ATTN_BF16_HISTORY) != 0;
  const bool traceable = scratch == nullptr;
  if (plan.flat) {
    DecodeFlatArgs f{};
    f.d = d;
    f.t = plan.table;
    const Fn flat = Fn((bf16h ? kDecodeFlatBf16h64 : kDecodeFlat64) + di);
    DeviceGuard guard(ctx->device);
    launch(ctx, PPK_KERNEL_ATTENTION, flat, plan.blocks, 64 * plan.waves, 0, stream, f, 1, traceable);
    if (plan.ngroups < 2) return;  // every row was one unit: the decode launch wrote them all
    MergeFlatArgs m{};
    m.m.q = a.q;
    m.m.sk = a.sk;
    m.m.sv = a.sv;
    m.m.past = a.past;
    m.m.part_y = d.part_y;
    m.m.part_mz = d.part_mz;
    m.m.out = a.out;
    m.m.rows = a.rows;
    m.m.heads = a.heads;
    m.m.capacity = a.capacity;
    m.m.split_tokens = plan.split;
    m.m.nsplits = plan.ngroups;
    m.m.q_dtype = a.q_dtype;
    m.m.scratch_dtype = a.scratch_dtype;
    m.m.out_dtype = a.out_dtype;
    m.m.scale_log2 = scale_log2;
    m.m.span = plan.span;
    m.t = plan.table;
    launch(ctx, PPK_KERNEL_ATTN_MERGE, Fn(kMergeFlat64 + di), a.rows, 64, 0, stream, m, 1, traceable);
    return;
  }
  // The int8 plan's blocks hold at most 8 waves: the kernels are bounded to
  // 512 threads (two waves per SIMD, up to 256 VGPRs, three batches in flight).
  require(plan.waves <= 8, "internal: int8 decode block of more than 8 waves");
  const Fn decode = Fn((bf16h ? kDecodeBf16h64 : kDecode64) + di);
  DeviceGuard guard(ctx->device);
  launch(ctx, PPK_KERNEL_ATTENTION, decode, plan.ngroups * a.rows, 64 * plan.waves, plan.lds_bytes, stream, d, 1,
         traceable);
  if (plan.ngroups > 1) {
    MergeArgs m{};
    m.q = a.q;
    m.sk = a.sk;
    m.sv = a.sv;
    m.past = a.past;
    m.part_y = d.part_y;
    m.part_mz = d.part_mz;
    m.out = a.out;
    m.rows = a.rows;
    m.heads = a.heads;
    m.capacity = a.capacity;
    m.split_tokens = plan.split * plan.waves;  // tokens per group
    m.nsplits = plan.ngroups;
    m.q_dtype = a.q_dtype;
    m.scratch_dtype = a.scratch_dtype;
    m.out_dtype = a.out_dtype;
    m.scale_log2 = scale_log2;
    m.clock = d.clock;
    m.clock_seq = d.clock_seq;
    m.clock_cap = d.clock_cap;
    launch(ctx, PPK_KERNEL_ATTN_MERGE, Fn(kMerge64 + di), a.rows, 64, 0, stream, m, 1, traceable);
  }
}

// Float-KV decode attention (app/src/model/hip_attention.rs:47-113). The
// reference requires head_dim 64, size <= 1024 and F32 Q/out; here head_dim
// 64/128/256, any size, and f32/bf16/f16 Q and output are accepted. Every
// span is checked against the stated strides before the first enqueue.
// The float argument block up to workspace_bytes is required; lengths_host
// (added later) is read only when struct_size covers it.
constexpr size_t kFloatArgsMin = offsetof(PpkFloatAttentionArgs, lengths_host);
const uint32_t* host_lengths(const PpkFloatAttentionArgs& a) {
  return a.struct_size >= offsetof(PpkFloatAttentionArgs, lengths_host) + sizeof(a.lengths_host) ? a.lengths_host
                                                                                                  : nullptr;
}

AttentionPlan plan_float_attention(const ppk_context* ctx, const PpkFloatAttentionArgs& a) {
  require(a.struct_size >= kFloatArgsMin, "PpkFloatAttentionArgs.struct_size too small");
  dim_index(a.head_dim);
  require(a.kv_dtype == PPK_BF16 || a.kv_dtype == PPK_F32, "float attention K/V dtype must be bf16 or f32");
  require(valid_dtype(a.q_dtype) && valid_dtype(a.out_dtype), "float attention Q/out dtype must be f32, bf16 or f16");
  require(a.heads > 0 && a.rows > 0 && a.rows % a.heads == 0, "float attention geometry differs: rows % heads");
  require(a.size > 0, "float attention requires at least one stored token per row");
  require(a.max_length <= a.size, "max_length exceeds size");
  require(a.max_length == 0 || a.lengths != nullptr, "max_length requires per-sequence lengths");
  require(std::isfinite(a.softmax_scale) && a.softmax_scale >= 0.f, "softmax_scale must be finite and >= 0");
  require((a.flags & ~kPlanFlags) == 0, "unknown float attention flags");
  require((a.flags & kPlanFlags) != kPlanFlags, "float attention plan flags PER_ROW and BALANCED both set");
  const uint64_t eb = a.kv_dtype == PPK_BF16 ? 2 : 4;
  const uint64_t row_elems = uint64_t(a.size) * a.head_dim;
  require(row_elems <= (uint64_t(1) << 40), "float attention size too large");
  const uint64_t ks = a.k_row_stride ? a.k_row_stride : row_elems;
  const uint64_t vs = a.v_row_stride ? a.v_row_stride : row_elems;
  require(ks >= row_elems && vs >= row_elems, "float attention K/V row stride smaller than size * head_dim");
  require((ks * eb) % 16 == 0 && (vs * eb) % 16 == 0, "float attention K/V row stride must be a multiple of 16 bytes");
  require(uint64_t(a.rows) * std::max(ks, vs) <= (uint64_t(1) << 46), "float attention K/V span too large");
  const uint32_t tpl = 64u / (a.head_dim / uint32_t(16 / eb));
  const uint64_t span = a.max_length ? a.max_length : a.size;
  const uint32_t* host = host_lengths(a);
  require(!host || a.lengths, "float attention lengths_host needs the device lengths");
  const uint32_t batch = a.rows / a.heads;
  // As on the int8 path: with the host's lengths (and no plan bit) the
  // per-row plan covers the longest live row; a device length beyond it
  // gives NaN rows (and PPK_FLAG_STALE_LENGTHS in a decode step).
  const uint64_t cover = host && !(a.flags & kPlanFlags) ? row_cover(host, batch, span) : span;
  // Few long rows: blocks of fewer than four waves halve their waves' share
  // as on the int8 path, but not below 16 KiB of K and V per wave (the float
  // waves do less arithmetic per byte, so shorter streams cost more than the
  // idle SIMDs). Same-box A/B, H = 16, one launch pair per step: B = 1 x 2048
  // bf16 D = 128 8.28 -> 7.18 us, x 1536 8.58 -> 6.99 us, fused step 8.68 ->
  // 7.87 us; f32 D = 64 x 1024 7.04 -> 6.25 us, f32 D = 128 x 2048 10.82 ->
  // 8.73 us; bf16 D = 64 (16 KiB per 64-token wave) unchanged, where halving
  // to 8 KiB had cost 4 %.
  const uint64_t token_bytes = 2ull * eb * a.head_dim;
  const uint32_t min_split = std::max<uint32_t>(4 * std::max(tpl, 1u), uint32_t((16u << 10) / token_bytes));
  AttentionPlan plan =
      plan_rows(ctx, a.rows, cover, a.split_tokens, std::max(tpl, 1u), token_bytes, a.head_dim, min_split, 16);
  // With the host's copy of the lengths, a ragged batch takes the balanced
  // plan (the int8 path's table) when its longest row holds more than
  // 512 KiB of K and V and the per-row plan's waves are uneven (the most
  // tokens a wave streams beyond 1.1 x the mean over the waves that stream
  // any): the float kernel streams at the rate of its slowest waves, not
  // CU by CU. Measured on MI355X (bf16, H = 16, D = 64 / 128, per step,
  // per-row -> balanced), taken: 4 sequences of 8192 tokens beside 28 of
  // 512, 57.3 -> 37.4 / 112.0 -> 67.1 us; 2 of 16384 beside 14 of 256, 74.0
  // -> 30.3 / 147.7 -> 53.8 us; 1 of 8192 beside 31 of 256, 53.7 -> 17.8 /
  // 106.4 -> 28.8 us; B = 16 of 256..16384, 94.1 -> 90.7 / 187.3 -> 172.4
  // us; B = 32 of 256..8192 and B = 64 of 64..4096 within 2 %. Kept
  // per-row (balanced was slower): 8 of 4096 beside 24 of 1024, 39.3 /
  // 71.4 us (balanced 41.7 / 78.2); config 4, 15.7 / 24.9 us (17.6 /
  // 28.9); rows of at most 512 KiB, e.g. 4 of 1024 beside 28 of 64 at
  // D = 64, 9.3 us (11.5: the merge launch costs more than the balance
  // gains).
  constexpr uint64_t kFloatFlatMinRowBytes = 512u << 10;
  if (a.flags & PPK_ATTN_PLAN_BALANCED) {
    require_balanced(ctx, a.rows, a.heads, host, a.split_tokens);
    plan = plan_flat(ctx, a.rows, a.heads, host, span, a.head_dim);
  } else if (!(a.flags & PPK_ATTN_PLAN_PER_ROW) && host && a.split_tokens == 0 &&
             flat_pays(ctx, a.rows, a.heads, host, span) &&
             longest_live(host, batch, span) * 2 * eb * a.head_dim > kFloatFlatMinRowBytes &&
             per_row_waves_uneven(batch, host, span, plan.split)) {
    plan = plan_flat(ctx, a.rows, a.heads, host, span, a.head_dim);
  }
  plan.span = uint32_t(span);
  return plan;
}

void run_float_attention(ppk_context* ctx, hipStream_t stream, const PpkFloatAttentionArgs& a,
                         const PpkFloatDecodeStepArgs* step) {
  const AttentionPlan plan = plan_float_attention(ctx, a);
  if (step) {
    require(step->struct_size >= sizeof(PpkFloatDecodeStepArgs), "PpkFloatDecodeStepArgs.struct_size too small");
    require(a.lengths != nullptr, "the float decode step needs the device lengths");
    require(valid_dtype(step->new_dtype), "float decode step new-token dtype must be f32, bf16 or f16");
    require(step->k_new && step->v_new, "float decode step null new token");
    require(aligned(step->k_new, dtype_bytes(step->new_dtype)) && aligned(step->v_new, dtype_bytes(step->new_dtype)) &&
                (!step->flags || aligned(step->flags, 4)),
            "float decode step operand misaligned");
  }
  require(a.q && a.k && a.v && a.out, "float attention null pointer");
  require(aligned(a.k, 16) && aligned(a.v, 16), "float attention K/V must be 16-byte aligned");
  require(aligned(a.q, dtype_bytes(a.q_dtype)) && aligned(a.out, dtype_bytes(a.out_dtype)) &&
              (!a.lengths || aligned(a.lengths, 4)),
          "float attention operand misaligned");
  const uint64_t qs = a.q_row_stride ? a.q_row_stride : a.head_dim;
  require(qs >= a.head_dim, "float attention Q row stride smaller than head_dim");
  if (plan.workspace_bytes) {
    require(a.workspace && aligned(a.workspace, 256), "float attention workspace missing or not 256-byte aligned");
    if (a.workspace_bytes < plan.workspace_bytes)
      throw PreconditionError("float attention workspace too small: need " + std::to_string(plan.workspace_bytes) +
                              " bytes");
  }
  const int di = dim_index(a.head_dim);
  const float scale = a.softmax_scale > 0.f ? a.softmax_scale : 1.0f / std::sqrt(float(a.head_dim));
  const uint64_t row_elems = uint64_t(a.size) * a.head_dim;

  FloatDecodeArgs d{};
  d.q = a.q;
  d.k = a.k;
  d.v = a.v;
  d.lengths = a.lengths;
  d.part_y = plan.workspace_bytes ? static_cast<float*>(a.workspace) : nullptr;
  d.part_mz = plan.workspace_bytes ? reinterpret_cast<float*>(static_cast<char*>(a.workspace) + plan.y_bytes) : nullptr;
  d.out = a.out;
  d.q_stride = qs;
  d.k_stride = a.k_row_stride ? a.k_row_stride : row_elems;
  d.v_stride = a.v_row_stride ? a.v_row_stride : row_elems;
  d.rows = a.rows;
  d.heads = a.heads;
  d.size = a.size;
  d.split_tokens = plan.split;
  d.ngroups = plan.ngroups;
  d.q_dtype = a.q_dtype;
  d.out_dtype = a.out_dtype;
  d.scale_log2 = scale * 1.4426950408889634f;
  d.span = plan.span;
  if (step) {
    d.k_new = step->k_new;
    d.v_new = step->v_new;
    d.flags = step->flags;
    d.new_dtype = step->new_dtype;
  }

  FloatMergeArgs m{};
  m.lengths = a.lengths;
  m.part_y = d.part_y;
  m.part_mz = d.part_mz;
  m.out = a.out;
  m.rows = a.rows;
  m.heads = a.heads;
  m.size = a.size;
  m.nsplits = plan.ngroups;
  m.out_dtype = a.out_dtype;
  m.span = plan.span;
  const bool bf16 = a.kv_dtype == PPK_BF16;
  if (step) {
    m.step = 1;
    m.q = a.q;
    m.q_stride = qs;
    m.q_dtype = a.q_dtype;
    m.k_new = step->k_new;
    m.v_new = step->v_new;
    m.new_dtype = step->new_dtype;
    m.kv_bf16 = bf16 ? 1u : 0u;
    m.scale_log2 = d.scale_log2;
  }
  DeviceGuard guard(ctx->device);
  if (plan.flat) {
    FloatDecodeFlatArgs fd{};
    fd.d = d;
    fd.t = plan.table;
    const Fn flat = step ? Fn((bf16 ? kFStepFlatBf16_64 : kFStepFlatF32_64) + di)
                         : Fn((bf16 ? kFDecodeFlatBf16_64 : kFDecodeFlatF32_64) + di);
    launch(ctx, PPK_KERNEL_FLOAT_ATTENTION, flat, plan.blocks, 64 * plan.waves, 0, stream, fd);
    if (plan.ngroups > 1) {
      FloatMergeFlatArgs fm{};
      fm.m = m;
      fm.m.split_tokens = plan.split;
      fm.t = plan.table;
      launch(ctx, PPK_KERNEL_FLOAT_MERGE, Fn(kFMergeFlat64 + di), a.rows, 64, 0, stream, fm);
    }
    return;
  }
  const Fn decode = step ? Fn((bf16 ? kFStepBf16_64 : kFStepF32_64) + di)
                        : Fn((bf16 ? kFDecodeBf16_64 : kFDecodeF32_64) + di);
  launch(ctx, PPK_KERNEL_FLOAT_ATTENTION, decode, plan.ngroups * a.rows, 64 * plan.waves, plan.lds_bytes, stream, d);
  if (plan.ngroups > 1) {
    m.split_tokens = plan.split * plan.waves;  // tokens per group
    launch(ctx, PPK_KERNEL_FLOAT_MERGE, Fn(kFMerge64 + di), a.rows, 64, 0, stream, m);
  }
}

// CFG + Renyi sampler (app/src/inference/hip_sampling.rs:18-69 validation,
// :150-214 launch): metadata is checked on the host; device values (bounds,
// uniforms, logits) are judged by the kernel, which marks bad rows valid = 0.
void run_renyi_sample(ppk_context* ctx, hipStream_t stream, const PpkRenyiSampleArgs& a) {
  require(a.struct_size >= sizeof(PpkRenyiSampleArgs), "PpkRenyiSampleArgs.struct_size too small");
  require((a.guidance == 1 || a.guidance == 2) && a.batch > 0 && a.choices >= 1 &&
              a.choices <= uint32_t(kSamplerMaxChoices),
          "HIP sampler needs 1/2 guidance rows and a nonempty head of at most 2048 choices");
  require(a.batch <= 0x7fffffffu, "HIP sampler logical row, uniform or bounds shape mismatch");
  require(std::isfinite(a.alpha) && a.alpha > 1.f && std::isfinite(a.cfg) && a.cfg >= 0.f &&
              (a.guidance != 1 || a.cfg == 1.f),
          "invalid HIP sampler alpha/CFG/guidance combination");
  require(uint64_t(a.token_offset) + (a.choices - 1) <= 0xffffffffull, "HIP sampler token range overflow");
  require(a.raw && a.uniforms && a.bounds && a.out, "HIP sampler null pointer");
  require(aligned(a.raw, 4) && aligned(a.uniforms, 4) && aligned(a.bounds, 4) && aligned(a.out, 4),
          "HIP sampler operand misaligned");
  RenyiArgs k{};
  k.raw = a.raw;
  k.uniforms = a.uniforms;
  k.bounds = a.bounds;
  k.out = a.out;
  k.batch = a.batch;
  k.choices = a.choices;
  k.guidance = a.guidance;
  k.token_offset = a.token_offset;
  k.alpha = a.alpha;
  k.cfg = a.cfg;
  DeviceGuard guard(ctx->device);
  launch(ctx, PPK_KERNEL_RENYI_SAMPLE, kRenyiSample, a.batch, kSamplerThreads, 0, stream, k);
}

void run_arena_write(ppk_context* ctx, hipStream_t stream, const ArenaWrite& w) {
  const uint64_t rows = w.sequences * w.heads;
  DeviceGuard guard(ctx->device);
  if (w.elem_bytes == 0) {
    QuantizeArgs k{};
    k.src[0] = w.k_src;
    k.src[1] = w.v_src;
    k.codes[0] = w.k;
    k.codes[1] = w.v;
    k.scales[0] = w.ks;
    k.scales[1] = w.vs;
    k.past = w.past;
    k.rows = rows * w.tokens;
    k.heads = w.heads;
    k.tokens = w.tokens;
    k.capacity = w.capacity;
    k.src_dtype = w.src_dtype;
    k.ntensors = 2;
    k.uniform_past = w.uniform_past;
    const uint64_t grid = (2 * k.rows + 3) / 4;
    require(grid <= 0x7fffffffu, "KV append grid too large");
    if (launch_stream_quantize(ctx, stream, PPK_KERNEL_APPEND, k, w.head_dim)) return;
    launch(ctx, PPK_KERNEL_APPEND, Fn(kQuantize64 + dim_index(w.head_dim)), uint32_t(grid), 256, 0, stream, k);
    return;
  }
  const uint64_t record = uint64_t(w.head_dim) * w.elem_bytes;
  auto fits = [&](uint64_t unit) {
    return record % unit == 0 && aligned(w.k_src, unit) && aligned(w.v_src, unit) && aligned(w.k, unit) &&
           aligned(w.v, unit);
  };
  const uint32_t unit = fits(16) ? 16 : fits(4) ? 4 : 2;
  require(record % unit == 0 && aligned(w.k_src, unit) && aligned(w.v_src, unit), "KV append source misaligned");
  ScatterArgs a{};
  a.src[0] = static_cast<const uint8_t*>(w.k_src);
  a.src[1] = static_cast<const uint8_t*>(w.v_src);
  a.dst[0] = w.k;
  a.dst[1] = w.v;
  a.past = w.past;
  a.rows = rows;
  a.heads = w.heads;
  a.tokens = w.tokens;
  a.capacity = w.capacity;
  a.uniform_past = w.uniform_past;
  a.row_units = uint32_t(record / unit);
  const uint64_t units = 2 * rows * w.tokens * a.row_units;
  const uint64_t grid = std::min<uint64_t>((units + 255) / 256, uint64_t(std::max(ctx->cu_count, 1)) * 16);
  launch(ctx, PPK_KERNEL_APPEND, unit == 16 ? kScatter16 : unit == 4 ? kScatter4 : kScatter2, uint32_t(grid), 256, 0,
         stream, a);
}

void run_copy_batch(ppk_context* ctx, hipStream_t stream, const std::vector<CopyDesc>& in) {
  if (in.empty()) return;
  // Like-sized rectangles share a launch, so one grid shape fits them all.
  std::vector<CopyDesc> copies(in);
  for (const CopyDesc& c : copies)  // every rectangle checked before the first launch
    require(c.width <= c.fill && c.fill <= c.dpitch && c.fill <= 0xffffffffu && (c.width == 0 || c.width <= c.spitch) &&
                (c.width == 0 || c.src) && c.dst,
            "arena copy rectangle out of its rows");
  std::stable_sort(copies.begin(), copies.end(), [](const CopyDesc& x, const CopyDesc& y) {
    return uint64_t(x.height) * x.fill > uint64_t(y.height) * y.fill;
  });
  DeviceGuard guard(ctx->device);
  for (size_t first = 0; first < copies.size(); first += kMaxCopies) {
    const size_t n = std::min<size_t>(kMaxCopies, copies.size() - first);
    CopyBatchArgs a{};
    a.n = uint32_t(n);
    uint64_t most = 0;
    for (size_t i = 0; i < n; ++i) {
      const CopyDesc& c = copies[first + i];
      uint32_t unit = 16;
      while (unit > 1 && (c.width % unit || c.fill % unit || c.spitch % unit || c.dpitch % unit ||
                          !aligned(c.src, unit) || !aligned(c.dst, unit)))
        unit >>= unit == 16 ? 2 : 1;
      a.c[i].src = static_cast<const uint8_t*>(c.src);
      a.c[i].dst = static_cast<uint8_t*>(c.dst);
      a.c[i].spitch = c.spitch;
      a.c[i].dpitch = c.dpitch;
      a.c[i].width = uint32_t(c.width);
      a.c[i].fill = uint32_t(c.fill);
      a.c[i].height = c.height;
      a.c[i].unit = unit;
      most = std::max<uint64_t>(most, uint64_t(c.height) * (c.fill / unit));
    }
    // About sixteen resident blocks per CU over the whole launch, eight units per thread per pass.
    const uint64_t cus = uint64_t(std::max(ctx->cu_count, 1));
    const uint64_t gx = std::max<uint64_t>(1, std::min<uint64_t>((most + 2047) / 2048, (cus * 16 + n - 1) / n));
    launch(ctx, PPK_KERNEL_COPY, kCopyBatch, uint32_t(gx), 256, 0, stream, a, uint32_t(n));
  }
}

}  // namespace ppk

extern "C" {

uint32_t ppk_abi_version(void) { return PPK_ABI_VERSION; }

const char* ppk_last_error(void) { return g_last_error.c_str(); }

int32_t ppk_context_create(int32_t device, const char* code_object_path, ppk_context** out) {
  if (out) *out = nullptr;
  return call([&] {
    ppk::require(out != nullptr, "ppk_context_create: null output pointer");
    int count = 0;
    check_prep(hipGetDeviceCount(&count), "hipGetDeviceCount");
    ppk::require(device >= 0 && device < count, "HIP device ordinal out of range");
    auto ctx = std::make_unique<ppk_context>();
    ctx->device = device;
    ppk::DeviceGuard guard(device);
    hipDeviceProp_t prop{};
    check_prep(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    ppk::require(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0,
                 std::string("code object is built for gfx950, device is ") + prop.gcnArchName);
    ctx->cu_count = prop.multiProcessorCount;
    ctx->code_object = code_object_path ? std::string(code_object_path) : default_code_object();
    check_prep(hipModuleLoad(&ctx->module, ctx->code_object.c_str()),
               ("hipModuleLoad " + ctx->code_object).c_str());
    for (int i = 0; i < ppk::kFnCount; ++i) {
      const hipError_t st = hipModuleGetFunction(&ctx->fn[i], ctx->module, kFnNames[i]);
      if (st != hipSuccess) {
        (void)hipModuleUnload(ctx->module);
        ctx->module = nullptr;
        throw ppk::PreconditionError(std::string("kernel symbol missing: ") + kFnNames[i]);
      }
    }
    // The no-alloc entry point's scratch: this GPU's device address, looked
    // up once per device (a failure only disables that entry point).
    try {
      ctx->scratch = ppk::scratch_lookup(device);
    } catch (const std::exception& e) {
      ctx->scratch = nullptr;
      ctx->scratch_error = e.what();
    }
    size_t total_mem = 0;
    if (hipDeviceTotalMem(&total_mem, device) == hipSuccess && total_mem > 0)
      ctx->block_cache_limit = std::min(ppk_context::kBlockCacheBytes, total_mem / 8);
    hipMemPoolProps props{};
    props.allocType = hipMemAllocationTypePinned;
    props.handleTypes = hipMemHandleTypeNone;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = device;
    uint64_t keep = UINT64_MAX;
    if (hipMemPoolCreate(&ctx->mem_pool, &props) != hipSuccess ||
        hipMemPoolSetAttribute(ctx->mem_pool, hipMemPoolAttrReleaseThreshold, &keep) != hipSuccess) {
      if (ctx->mem_pool) (void)hipMemPoolDestroy(ctx->mem_pool);
      (void)hipModuleUnload(ctx->module);
      throw ppk::PreconditionError("device memory pool set-up failed");
    }
    *out = ctx.release();
  });
}

int32_t ppk_context_trim(ppk_context* ctx, uint64_t* released_bytes) {
  if (released_bytes) *released_bytes = 0;
  return call([&] {
    ppk::require(ctx != nullptr, "ppk_context_trim: null context");
    const uint64_t freed = ppk::kv::drain_blocks(ctx);
    if (released_bytes) *released_bytes = freed;
  });
}

int32_t ppk_context_release(ppk_context* ctx) {
  return call([&] {
    if (!ctx) return;
    std::unique_ptr<ppk_context> owned(ctx);
    ppk::DeviceGuard guard(ctx->device);
    for (auto& list : ctx->pending)
      for (auto& ev : list) {
        (void)hipEventDestroy(ev.start);
        (void)hipEventDestroy(ev.stop);
      }
    for (auto& ev : ctx->pool) {
      (void)hipEventDestroy(ev.start);
      (void)hipEventDestroy(ev.stop);
    }
    // Recycled write-plan vectors: a synchronous free (their streams may be gone).
    for (auto& b : ctx->plan_pool) {
      (void)hipFree(b.dev);
      if (b.released) (void)hipEventDestroy(b.released);
    }
    for (auto& b : ctx->block_cache) {  // released arenas kept for reuse
      (void)hipEventSynchronize(b.released);
      (void)hipEventDestroy(b.released);
      (void)hipFree(b.ptr);
    }
    for (hipEvent_t ev : ctx->spare_events) (void)hipEventDestroy(ev);
    if (ctx->mem_pool) (void)hipMemPoolDestroy(ctx->mem_pool);
    if (ctx->module) (void)hipModuleUnload(ctx->module);
  });
}

int32_t ppk_quantize(ppk_context* ctx, void* stream, const PpkQuantizeArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_quantize: null context or arguments");
    ppk::run_quantize(ctx, static_cast<hipStream_t>(stream), *args);
  });
}

int32_t ppk_quantize_append(ppk_context* ctx, void* stream, const PpkAppendArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_quantize_append: null context or arguments");
    ppk::run_append(ctx, static_cast<hipStream_t>(stream), *args);
  });
}

int32_t ppk_dequantize(ppk_context* ctx, void* stream, const PpkDequantizeArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_dequantize: null context or arguments");
    ppk::run_dequantize(ctx, static_cast<hipStream_t>(stream), *args);
  });
}

int32_t ppk_attention_workspace_bytes(ppk_context* ctx, const PpkAttentionArgs* args, uint64_t* bytes) {
  if (bytes) *bytes = 0;
  return call([&] {
    ppk::require(args && bytes, "ppk_attention_workspace_bytes: null argument");
    *bytes = ppk::plan_attention(ctx, *args).workspace_bytes;
  });
}

int32_t ppk_attention_plan(ppk_context* ctx, const PpkAttentionArgs* args, uint32_t* split_tokens,
                           uint32_t* nsplits, uint64_t* workspace_bytes) {
  return call([&] {
    ppk::require(args != nullptr, "ppk_attention_plan: null arguments");
    const ppk::AttentionPlan plan = ppk::plan_attention(ctx, *args);
    if (split_tokens) *split_tokens = plan.split;
    if (nsplits) *nsplits = plan.ngroups;
    if (workspace_bytes) *workspace_bytes = plan.workspace_bytes;
  });
}

namespace {
void fill_plan_info(const ppk::AttentionPlan& plan, uint32_t rows, PpkAttentionPlanInfo* info) {
  ppk::require(info != nullptr && info->struct_size >= sizeof(PpkAttentionPlanInfo),
               "PpkAttentionPlanInfo missing or struct_size too small");
  info->kind = plan.flat ? PPK_ATTN_PLAN_BALANCED : PPK_ATTN_PLAN_PER_ROW;
  info->split_tokens = plan.split;
  info->nsplits = plan.ngroups;
  info->waves_per_block = plan.waves;
  info->blocks = plan.flat ? plan.blocks : plan.ngroups * rows;
  info->launches = plan.flat ? (plan.ngroups >= 2 ? 2u : 1u) : (plan.ngroups > 1 ? 2u : 1u);
  info->reserved = 0;
  info->workspace_bytes = plan.workspace_bytes;
}
}  // namespace

int32_t ppk_attention_plan_info(ppk_context* ctx, const PpkAttentionArgs* args, PpkAttentionPlanInfo* info) {
  return call([&] {
    ppk::require(args != nullptr, "ppk_attention_plan_info: null arguments");
    fill_plan_info(ppk::plan_attention(ctx, *args), args->rows, info);
  });
}

int32_t ppk_decode_attention(ppk_context* ctx, void* stream, const PpkAttentionArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_decode_attention: null context or arguments");
    ppk::run_attention(ctx, static_cast<hipStream_t>(stream), *args);
  });
}

int32_t ppk_decode_step(ppk_context* ctx, void* stream, const PpkDecodeStepArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_decode_step: null context or arguments");
    ppk::run_attention(ctx, static_cast<hipStream_t>(stream), args->attn, args);
  });
}

int32_t ppk_decode_step_noalloc(ppk_context* ctx, void* stream, const PpkDecodeStepArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_decode_step_noalloc: null context or arguments");
    if (!ctx->scratch) throw ppk::PreconditionError("no-alloc scratch unavailable on this device: " + ctx->scratch_error);
    ppk::run_attention(ctx, static_cast<hipStream_t>(stream), args->attn, args, ctx->scratch, ppk::kScratchBytes);
  });
}

int32_t ppk_float_attention_plan(ppk_context* ctx, const PpkFloatAttentionArgs* args, uint32_t* split_tokens,
                                 uint32_t* nsplits, uint64_t* workspace_bytes) {
  if (workspace_bytes) *workspace_bytes = 0;
  return call([&] {
    ppk::require(args != nullptr, "ppk_float_attention_plan: null arguments");
    const ppk::AttentionPlan plan = ppk::plan_float_attention(ctx, *args);
    if (split_tokens) *split_tokens = plan.split;
    if (nsplits) *nsplits = plan.ngroups;
    if (workspace_bytes) *workspace_bytes = plan.workspace_bytes;
  });
}

int32_t ppk_float_attention_plan_info(ppk_context* ctx, const PpkFloatAttentionArgs* args,
                                      PpkAttentionPlanInfo* info) {
  return call([&] {
    ppk::require(args != nullptr, "ppk_float_attention_plan_info: null arguments");
    fill_plan_info(ppk::plan_float_attention(ctx, *args), args->rows, info);
  });
}

int32_t ppk_float_decode_attention(ppk_context* ctx, void* stream, const PpkFloatAttentionArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_float_decode_attention: null context or arguments");
    ppk::run_float_attention(ctx, static_cast<hipStream_t>(stream), *args);
  });
}

int32_t ppk_float_decode_step(ppk_context* ctx, void* stream, const PpkFloatDecodeStepArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_float_decode_step: null context or arguments");
    ppk::require(args->struct_size >= sizeof(PpkFloatDecodeStepArgs), "PpkFloatDecodeStepArgs.struct_size too small");
    ppk::run_float_attention(ctx, static_cast<hipStream_t>(stream), args->attn, args);
  });
}

int32_t ppk_renyi_sample(ppk_context* ctx, void* stream, const PpkRenyiSampleArgs* args) {
  return call([&] {
    ppk::require(ctx && args, "ppk_renyi_sample: null context or arguments");
    ppk::run_renyi_sample(ctx, static_cast<hipStream_t>(stream), *args);
  });
}

int32_t ppk_kv_cache_create(ppk_context* ctx, const PpkKvConfig* config, ppk_kv_cache** out) {
  if (out) *out = nullptr;
  return call([&] {
    ppk::require(ctx && config && out, "ppk_kv_cache_create: null argument");
    *out = ppk::kv::create(ctx, *config);
  });
}

int32_t ppk_kv_cache_clone(const ppk_kv_cache* cache, ppk_kv_cache** out) {
  if (out) *out = nullptr;
  return call([&] {
    ppk::require(cache && out, "ppk_kv_cache_clone: null argument");
    *out = ppk::kv::clone(*cache);
  });
}

int32_t ppk_kv_cache_release(ppk_kv_cache* cache) {
  return call([&] { ppk::kv::release(cache); });
}

int32_t ppk_kv_cache_info(const ppk_kv_cache* cache, PpkKvInfo* out) {
  return call([&] {
    ppk::require(cache != nullptr, "ppk_kv_cache_info: null cache");
    ppk::kv::info(*cache, out);
  });
}

int32_t ppk_kv_cache_truncate(ppk_kv_cache* cache, uint32_t new_len) {
  return call([&] {
    ppk::require(cache != nullptr, "ppk_kv_cache_truncate: null cache");
    ppk::kv::truncate(*cache, new_len);
  });
}

int32_t ppk_kv_cache_adopt(ppk_context* ctx, const PpkKvConfig* config, void* k, void* v, uint32_t capacity,
                           uint32_t committed_len, ppk_kv_cache** out) {
  if (out) *out = nullptr;
  return call([&] {
    ppk::require(ctx && config && out, "ppk_kv_cache_adopt: null argument");
    *out = ppk::kv::adopt(ctx, *config, k, v, capacity, committed_len);
  });
}

int32_t ppk_kv_cache_advance(ppk_kv_cache* cache, uint32_t previous, uint32_t next) {
  return call([&] {
    ppk::require(cache != nullptr, "ppk_kv_cache_advance: null cache");
    ppk::kv::advance(*cache, previous, next);
  });
}

int32_t ppk_kv_cache_view(const ppk_kv_cache* cache, PpkKvView* out) {
  return call([&] {
    ppk::require(cache != nullptr, "ppk_kv_cache_view: null cache");
    ppk::kv::view(*cache, out);
  });
}

int32_t ppk_kv_query(ppk_context* ctx, void* stream, ppk_kv_cache* cache, uint32_t past, const PpkKvWrite* write,
                     PpkKvView* out) {
  return call([&] {
    ppk::require(ctx && cache && write, "ppk_kv_query: null argument");
    ppk::kv::query(ctx, static_cast<hipStream_t>(stream), *cache, past, *write, out);
  });
}

int32_t ppk_write_plan_create(ppk_context* ctx, void* stream, const uint32_t* past_lens, uint32_t batch,
                              uint32_t heads, uint32_t head_dim, ppk_write_plan** out) {
  if (out) *out = nullptr;
  return call([&] {
    ppk::require(out != nullptr, "ppk_write_plan_create: null output");
    *out = ppk::kv::plan_create(ctx, static_cast<hipStream_t>(stream), past_lens, batch, heads, head_dim);
  });
}

int32_t ppk_write_plan_release(ppk_write_plan* plan) {
  return call([&] { ppk::kv::plan_release(plan); });
}

int32_t ppk_kv_query_batch(ppk_context* ctx, void* stream, ppk_kv_cache* const* caches, uint32_t batch,
                           const uint32_t* past_lens, const PpkKvWrite* write, const ppk_write_plan* plan,
                           PpkKvView* out) {
  return call([&] {
    ppk::require(ctx && write, "ppk_kv_query_batch: null argument");
    ppk::kv::query_batch(ctx, static_cast<hipStream_t>(stream), caches, batch, past_lens, *write, plan, out);
  });
}

int32_t ppk_float_attention_prepare(ppk_context* ctx) {
  return call([&] {
    ppk::require(ctx != nullptr, "ppk_float_attention_prepare: null context");
    ppk::float_attention_self_check(ctx);
  });
}

int32_t ppk_prepare(ppk_context* ctx) {
  return call([&] {
    ppk::require(ctx != nullptr, "ppk_prepare: null context");
    ppk::prepare_self_check(ctx);
  });
}

int32_t ppk_prepare_int8_kv(ppk_context* ctx, uint32_t requested, uint32_t head_dim, PpkInt8KvStatus* out) {
  auto text = [](char* dst, size_t cap, const std::string& src) {
    const size_t n = std::min(cap - 1, src.size());
    std::memcpy(dst, src.data(), n);
    dst[n] = '\0';
  };
  return call([&] {
    ppk::require(ctx && out, "ppk_prepare_int8_kv: null argument");
    ppk::require(out->struct_size >= sizeof(PpkInt8KvStatus), "PpkInt8KvStatus.struct_size too small");
    const uint32_t size = out->struct_size;
    std::memset(out, 0, sizeof(PpkInt8KvStatus));
    out->struct_size = size;
    out->requested = requested ? 1 : 0;
    out->available = (head_dim == 64 || head_dim == 128 || head_dim == 256) ? 1 : 0;
    out->packed_bytes_per_token_head = 2 * head_dim;
    out->scale_bytes_per_token_head = 8;
    text(out->format, sizeof(out->format), "BF16/F32");
    std::lock_guard<std::mutex> lock(ctx->prepare_mutex);
    out->ready = ctx->int8_ready ? 1 : 0;
    if (!requested) {
      text(out->reason, sizeof(out->reason), "int8 KV history disabled; the ordinary floating cache is kept");
      return;
    }
    if (!out->available) {
      text(out->reason, sizeof(out->reason),
           "int8 KV history on this backend needs gfx950 and 64/128/256-channel heads; the ordinary floating "
           "cache is kept");
      return;
    }
    if (!ctx->int8_ready) {
      try {
        ppk::prepare_self_check(ctx);
      } catch (const std::exception& e) {
        text(out->reason, sizeof(out->reason), std::string("int8 KV preparation incomplete: ") + e.what());
        throw;
      }
      ctx->int8_ready = true;
      out->ready = 1;
    }
    out->enabled = 1;
    text(out->format, sizeof(out->format), "INT8 symmetric per-token/head + FP32 scales");
    text(out->reason, sizeof(out->reason),
         "committed history is int8; the current K/V stay floating; attention dequantises on read");
  });
}

int32_t ppk_context_set_wave_clock(ppk_context* ctx, void* buffer, uint64_t bytes) {
  return call([&] {
    ppk::require(ctx != nullptr, "ppk_context_set_wave_clock: null context");
    ppk::require(buffer == nullptr || (bytes >= 2 * ppk::kWaveClockWords * 8 &&
                                       reinterpret_cast<uintptr_t>(buffer) % 16 == 0),
                 "ppk_context_set_wave_clock: buffer must be 16-byte aligned and hold at least one record");
    std::lock_guard<std::mutex> lock(ctx->prof_mutex);
    ctx->wave_clock = static_cast<uint64_t*>(buffer);
    ctx->wave_clock_seq = 0;
    const uint64_t records = buffer ? bytes / (ppk::kWaveClockWords * 8) - 1 : 0;  // after the header record
    ctx->wave_clock_cap = uint32_t(std::min<uint64_t>(records, 0xffffffffu));
  });
}

int32_t ppk_context_set_profiling(ppk_context* ctx, int32_t enable) {
  return call([&] {
    ppk::require(ctx != nullptr, "ppk_context_set_profiling: null context");
    std::lock_guard<std::mutex> lock(ctx->prof_mutex);
    ctx->profiling = enable != 0;
  });
}

int32_t ppk_context_kernel_stats(ppk_context* ctx, uint32_t kernel, uint64_t* launches, double* total_ms,
                                 uint32_t reset) {
  return call([&] {
    ppk::require(ctx && kernel < PPK_KERNEL_COUNT, "ppk_context_kernel_stats: bad context or kernel id");
    std::lock_guard<std::mutex> lock(ctx->prof_mutex);
    ppk::DeviceGuard guard(ctx->device);
    for (auto& ev : ctx->pending[kernel]) {
      const hipError_t st = hipEventSynchronize(ev.stop);
      if (st != hipSuccess) throw ppk::UncertainError(std::string("hipEventSynchronize: ") + hipGetErrorString(st));
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, ev.start, ev.stop) != hipSuccess)
        throw ppk::UncertainError("hipEventElapsedTime failed");
      ctx->launches[kernel] += 1;
      ctx->total_ms[kernel] += ms;
      ctx->pool.push_back(ev);
    }
    ctx->pending[kernel].clear();
    if (launches) *launches = ctx->launches[kernel];
    if (total_ms) *total_ms = ctx->total_ms[kernel];
    if (reset) {
      ctx->launches[kernel] = 0;
      ctx->total_ms[kernel] = 0.0;
    }
  });
}

}  // extern "C"
