// Streaming-read probe: the HBM read rate one launch sustains at the int8
// decode kernels' geometry (same waves, waves per block, blocks per CU, tile
// and batch size, batches in flight), with no arithmetic beyond one xor per
// loaded word. bench.py --probe times it beside the decode kernel, so the
// decode's bandwidth can be compared with what a pure read of the same shape
// reaches on the same box. It is a measurement tool built into its own
// library (ppk/libppk_probe.so), not part of the decode library's C-ABI.
//
// Each wave reads two contiguous ranges of `tiles` 1 KiB tiles (standing for
// its K codes, then its V codes): one nontemporal dwordx4 load per lane per
// tile (the decode's code loads are nontemporal too), kU tiles per batch, NB
// batches in flight, the ring carried from the first range into the second
// without draining (as the decode's stream does). Wave w of row r starts at
// r * row_stride + w * wave_stride (16-byte units): with the arenas' own
// strides (capacity * D per row, split * D per wave) the probe reads the
// decode's history bytes at the decode's addresses (bench.py also times a
// packed placement, every range starting a power of two apart, to show how
// much the placement matters). Every lane stores its checksum, so no load is
// dead code.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
constexpr int kU = 4;          // tiles per batch (4 KiB per wave)
constexpr int kTileU4 = 64;    // a 1 KiB tile is 64 lanes x 16 B

template <int NB>
__global__ __launch_bounds__(512) void read_probe(const u4* __restrict__ k, const u4* __restrict__ v,
                                                  uint32_t tiles, uint32_t waves_per_row, uint64_t row_stride,
                                                  uint64_t wave_stride, uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t base = size_t(wave / waves_per_row) * row_stride + size_t(wave % waves_per_row) * wave_stride +
                      size_t(lane);
  const uint32_t nb = tiles / kU;  // batches per range (the host checks tiles % kU == 0, tiles > 0)
  const uint32_t total = 2 * nb;
  u4 r[NB][kU];
  // Batch i of the wave's sequence: the K range, then the V range. Past the
  // end it re-reads the last batch (clamped, so every load is in bounds; the
  // re-read lines are still in L2).
  auto load = [&](uint32_t i, u4 (&dst)[kU]) {
    const uint32_t j = min(i, total - 1);
    const u4* src = j < nb ? k : v;
    const size_t t0 = size_t(j < nb ? j : j - nb) * kU;
#pragma unroll
    for (int u = 0; u < kU; ++u) dst[u] = __builtin_nontemporal_load(src + base + (t0 + u) * kTileU4);
    // Pins the loads where they are issued: without it the compiler folds the
    // ring's loop-carried registers back into loads at the top of each
    // iteration (same addresses), and every iteration drains the ring.
    asm volatile("" ::: "memory");
  };
#pragma unroll
  for (int b = 0; b < NB; ++b) load(uint32_t(b), r[b]);
  u4 acc = {0u, 0u, 0u, 0u};
  for (uint32_t i0 = 0; i0 < total; i0 += NB) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      // A mask rather than a branch: the consume stays straight-line code,
      // so each batch waits only for its own loads.
      const uint32_t keep = i0 + b < total ? ~0u : 0u;
#pragma unroll
      for (int u = 0; u < kU; ++u) acc ^= r[b][u] & keep;
      __builtin_amdgcn_sched_barrier(0);  // batch b is consumed before its slot is refilled, in this order
      load(i0 + b + NB, r[b]);
    }
  }
  out[size_t(wave) * 64 + lane] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace

// Launch the probe on `stream`: `waves` waves in blocks of `waves_per_block`,
// at most `blocks_per_cu` blocks resident per CU (enforced by reserving LDS
// the kernel does not use: 160 KiB per CU), `ring` batches in flight per wave
// (2, 3, 4 or 6), `waves_per_row` consecutive waves per row. `k` and `v` each
// hold (rows - 1) * row_stride + (waves_per_row - 1) * wave_stride +
// tiles * 64 16-byte units, rows = waves / waves_per_row (the caller sizes
// them; the strides must keep every range 16-byte aligned, which units of
// 16 bytes do). `out` holds waves * 64 words. Returns 0, -1 for arguments out
// of range, or the HIP error of the launch.
extern "C" __attribute__((visibility("default"))) int ppk_read_probe(const void* k, const void* v, uint32_t tiles,
                                                                     uint32_t waves, uint32_t waves_per_block,
                                                                     uint32_t blocks_per_cu, uint32_t ring,
                                                                     uint32_t waves_per_row, uint64_t row_stride,
                                                                     uint64_t wave_stride, uint32_t* out,
                                                                     hipStream_t stream) {
  if (!k || !v || !out || tiles == 0 || tiles % kU != 0 || waves_per_block == 0 || waves_per_block > 8 ||
      waves == 0 || waves % waves_per_block != 0 || blocks_per_cu < 2 || blocks_per_cu > 32 ||
      waves_per_row == 0 || waves % waves_per_row != 0 || wave_stride < uint64_t(tiles) * kTileU4 ||
      row_stride < (waves_per_row - 1) * wave_stride + uint64_t(tiles) * kTileU4)
    return -1;
  constexpr uint32_t kLdsPerCu = 160u * 1024u;
  // The smallest multiple of 1 KiB that keeps a further block off the CU.
  const uint32_t lds = (kLdsPerCu / (blocks_per_cu + 1) / 1024u + 1u) * 1024u;
  if (lds > 64u * 1024u || lds * blocks_per_cu > kLdsPerCu) return -1;
  const dim3 grid(waves / waves_per_block), block(64 * waves_per_block);
  const u4* kk = static_cast<const u4*>(k);
  const u4* vv = static_cast<const u4*>(v);
  const uint32_t wpr = waves_per_row;
  (void)hipGetLastError();  // the launch's own status below, not an earlier call's
  switch (ring) {
    case 2: hipLaunchKernelGGL(read_probe<2>, grid, block, lds, stream, kk, vv, tiles, wpr, row_stride, wave_stride, out); break;
    case 3: hipLaunchKernelGGL(read_probe<3>, grid, block, lds, stream, kk, vv, tiles, wpr, row_stride, wave_stride, out); break;
    case 4: hipLaunchKernelGGL(read_probe<4>, grid, block, lds, stream, kk, vv, tiles, wpr, row_stride, wave_stride, out); break;
    case 6: hipLaunchKernelGGL(read_probe<6>, grid, block, lds, stream, kk, vv, tiles, wpr, row_stride, wave_stride, out); break;
    default: return -1;
  }
  return int(hipGetLastError());
}
