// Host-side launch description for the W4A16 GEMV kernels (w4a16_gemv.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "w4a16_device.h"

namespace fk {

enum class GemvMode : int {
  kDirect = 0,    // one workgroup per (tile, m-tile) covers all of K, writes the output
  kFixup = 1,     // split-K, last-arriving workgroup of a tile reduces partials in-kernel
  kPartials = 2,  // split-K, writes fp32 partials [S_k, M, N] (reference layout, no reduce)
};

struct GemvLaunch {
  const void* x = nullptr;
  const void* packets = nullptr;
  void* out = nullptr;
  void* partials = nullptr;   // kFixup: scratch, kPartials: [S_k, M, N] fp32
  void* counters = nullptr;   // kFixup only: zero-initialised uint32 per (tile, m-tile)
  int M = 0, N = 0, K = 0;
  int group_size = 128;
  Act act = Act::kF16;
  GemvMode mode = GemvMode::kDirect;
  int m_tile = 1;
  int splits = 1;
  int gps = 0;  // groups per split
};

int gemv_m_tile_for_batch(int batch);

// fp32 scratch floats and counters the kFixup mode needs for a launch.
inline size_t gemv_fixup_partial_floats(int n, int batch, int m_tile, int splits) {
  const size_t tiles = static_cast<size_t>(n / kTileCols);
  const size_t mtiles = static_cast<size_t>((batch + m_tile - 1) / m_tile);
  return tiles * mtiles * static_cast<size_t>(splits) * m_tile * kTileCols;
}
inline size_t gemv_fixup_counters(int n, int batch, int m_tile) {
  return static_cast<size_t>(n / kTileCols) * static_cast<size_t>((batch + m_tile - 1) / m_tile);
}

hipError_t launch_w4a16_gemv(const GemvLaunch& launch, hipStream_t stream);

}  // namespace fk
