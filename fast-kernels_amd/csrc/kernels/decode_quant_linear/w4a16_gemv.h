// Host-side launch description for the W4A16 GEMV kernels (w4a16_gemv.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "w4a16_device.h"

namespace fk {

enum class GemvMode : int {
  kStreamK = 0,   // equal runs of (tile, group) units per workgroup, in-kernel fix-up
  kPartials = 1,  // fixed split-K, writes fp32 partials [S_k, M, N] (reference layout)
};

// Decode-step neighbours fused into the native-slab GEMV (w4a16_gemv_fused.hip):
//  kRmsNorm: y = W . rmsnorm(x), rmsnorm(x) = gamma * round(x * rsqrt(mean(x^2) + eps)), rounded
//            to the activation dtype after each product as the unfused pipeline does.
//  kSiluMul: W = [W_gate; W_up] stacked along N; out[M, N/2] = silu(g) * u in the activation
//            dtype, g and u rounded to it first.
//  kRmsNormSiluMul: both (the gate_up projection of a Llama block with its input norm).
enum class GemvFuse : int { kNone = 0, kRmsNorm = 1, kSiluMul = 2, kRmsNormSiluMul = 3 };

struct GemvLaunch {
  const void* x = nullptr;
  const void* packets = nullptr;
  void* out = nullptr;
  void* partials = nullptr;   // kStreamK: scratch, kPartials: [S_k, M, N] fp32
  void* counters = nullptr;   // kStreamK: zero-initialised uint32 per (tile, m-tile)
  int M = 0, N = 0, K = 0;
  int group_size = 128;
  Act act = Act::kF16;
  GemvMode mode = GemvMode::kStreamK;
  int m_tile = 1;
  int splits = 1;               // kPartials
  int gps = 0;                  // kPartials: groups per split
  int units_per_workgroup = 0;  // kStreamK: group units per workgroup
  int max_contributors = 0;     // kStreamK: partial slots per slice in the scratch
  int slice_cols = kTileCols;   // kStreamK: columns per workgroup slice (128, 64 or 32)
  PacketFormat format = PacketFormat::kArc;  // kStreamK: packet format of `packets`
  GemvFuse fuse = GemvFuse::kNone;           // native formats: fused decode-step neighbour
  const void* norm_weight = nullptr;         // GemvFuse::kRmsNorm: gamma [K], activation dtype
  float eps = 0.0f;                          // GemvFuse::kRmsNorm: epsilon
  // Native formats, unfused: each workgroup run streams two adjacent whole 32-column slices at
  // once (two waves per slice), which needs units_per_workgroup to be a multiple of 2 K/G.
  bool slice_pair = false;
  // Native formats, one activation row, unfused: the persistent stream schedule
  // (w4a16_gemv_stream.hip), the activation row staged whole in LDS.
  bool stream = false;
  int stream_waves = 0;   // stream schedule: streaming waves per workgroup (kStreamWaves)
  int stream_depth = 0;   // stream schedule: units in flight per wave
  int stream_grid = 0;    // stream schedule: workgroups
  int stream_whole = 0;   // stream schedule: whole slices (or half-slices) per workgroup
  // The slices left over past stream_grid * stream_whole (fewer than the workgroups) are dealt
  // as equal block ranges, a head and a tail piece per workgroup, finished through the
  // workspace: counters, one per slice; partials, 2 * 32 floats per workgroup.
  bool stream_pieces = false;
  // Half-slices (G = 128, one row): workgroup b streams the stream_whole half-slices
  // b * stream_whole .., half-slice hs being the 16 columns 16 * (hs & 1) .. of slice hs / 2
  // (half of every slab); stream_grid * stream_whole = 2 * slices.
  bool stream_half = false;
  // One row over the reference packets by 32-column quarters or 16-column eighths
  // (w4a16_gemv_arc_quarter.hip, with slice_cols == kSliceCols or kSliceCols / 2):
  // floor(2^32 / (K/G)) + 1, the reciprocal that turns a unit's linear (unit, group) index into
  // its unit.
  uint32_t ng_magic = 0;
  // Matrix-core stream kernel (m_tile == kMfmaRows), no pieces: K split into stream_parts equal
  // parts. Workgroup b takes part b / (stream_grid / stream_parts) of stream_whole slices, stages
  // only that part's activations and writes fp32 partial sums ([parts, M, N] in `partials`),
  // which a second launch adds in part order.
  int stream_parts = 1;
};

// Longest K the stream schedule stages (its LDS holds the whole activation row).
constexpr int kStreamMaxK = 32768;
// Dynamic LDS of the stream schedule for num_groups group slots (K / G and one spare): the
// re-paired row (G/8 16-byte words per group), four float2 offset terms and one float staging
// scale per group.
inline size_t stream_lds_bytes(int group_size, int num_groups) {
  return static_cast<size_t>(num_groups) * (static_cast<size_t>(group_size / 8) * 16 + 32 + 4);
}
// Streaming waves per workgroup of the stream schedule and the weights in flight per wave (4 KB:
// two G = 128 slabs of 2 KB or four G = 64 slabs of 1 KB). K/G must be a multiple of
// kStreamWaves * depth (a block).
constexpr int kStreamWaves = 8;
constexpr int kStreamKB = 4;
constexpr int stream_depth_for_kb(int group_size, int kb) { return kb / (group_size == 128 ? 2 : 1); }
// Most 32-column slices a stream launch with pieces may have (one arrival counter each).
constexpr int kStreamMaxSlices = 16384;
// Static LDS of the stream kernel besides the dynamic part, per activation row: ten reduction
// slots (two for pieces, a ring of eight for whole slices) of 8 waves x 32 floats, and the 8
// waves' RMS partial sums.
constexpr size_t kStreamStaticLdsBytes = (10 * 8 * 32 + 8) * sizeof(float);
// Workspace floats of a stream launch with pieces: two partial slots of rows x 32 per workgroup
// (the matrix-core stream kernel's slots hold 16 rows whatever the batch).
inline size_t stream_partial_floats(int grid, int rows) {
  return static_cast<size_t>(grid) * 2 * rows * kSliceCols;
}

// Activation rows per m-tile for a batch: 1, 2, 4, 8 on the dot2 GEMV kernel, kMfmaRows (from
// kMfmaMinBatch rows) on the matrix-core kernel.
constexpr int kMfmaRows = 16;
constexpr int kMfmaMinBatch = 8;
int gemv_m_tile_for_batch(int batch);
// m-tile of the reference split-K protocol (kPartials), served by the dot2 kernel only.
int gemv_partials_m_tile_for_batch(int batch);
hipError_t launch_w4a16_gemv_fused(const GemvLaunch& l, hipStream_t stream);

// Tiles (128 columns x m_tile rows) of a launch; the stream-K scratch holds one counter per slice
// (tiles x 128 / slice_cols) and max_contributors fp32 partial slots of m_tile x 128 floats per
// tile (the slices of a tile share its slots' size).
inline size_t gemv_tiles(int n, int batch, int m_tile) {
  return static_cast<size_t>(n / kTileCols) * static_cast<size_t>((batch + m_tile - 1) / m_tile);
}
inline size_t gemv_streamk_partial_floats(int n, int batch, int m_tile, int max_contributors) {
  return gemv_tiles(n, batch, m_tile) * static_cast<size_t>(max_contributors) * m_tile * kTileCols;
}

hipError_t launch_w4a16_gemv(const GemvLaunch& launch, hipStream_t stream);
// Matrix-core kernel for m_tile == kMfmaRows (w4a16_gemm_mfma.hip) and the dot2 kernels over the
// native packet formats (w4a16_gemv_native.hip); launch_w4a16_gemv forwards such launches.
hipError_t launch_w4a16_gemm_mfma(const GemvLaunch& launch, hipStream_t stream);
hipError_t launch_w4a16_gemv_native(const GemvLaunch& launch, hipStream_t stream);
hipError_t launch_w4a16_gemv_stream(const GemvLaunch& launch, hipStream_t stream);
// One row over the reference packets on the stream schedule (w4a16_gemv_arc_stream.hip): whole
// 128-column tiles per workgroup plus pieces of the tiles left over; arc_stream_lds: its dynamic
// LDS bytes.
hipError_t launch_w4a16_gemv_arc_stream(const GemvLaunch& launch, hipStream_t stream);
size_t arc_stream_lds(int group_size, int k);
// One row over the reference packets by 32-column quarters of the packets (slice_cols 32), or by
// 16-column eighths (slice_cols 16, G = 128, no pieces), on the native stream schedule
// (w4a16_gemv_arc_quarter.hip): whole units per workgroup plus pieces of the units left over.
// arc_quarter_lds: its dynamic LDS bytes; arc_quarter_magic: GemvLaunch::ng_magic for K/G;
// arc_quarter_magic_exact: whether that reciprocal is exact over every unit index of the launch.
hipError_t launch_w4a16_gemv_arc_quarter(const GemvLaunch& launch, hipStream_t stream);
size_t arc_quarter_lds(int group_size, int k, int cols = kSliceCols);
uint32_t arc_quarter_magic(int num_groups);
bool arc_quarter_magic_exact(int num_groups, long long slices);
// Matrix-core kernel on the stream schedule (w4a16_gemm_mfma_stream.hip): native slabs, 1-16 rows
// (m_tile == kMfmaRows), the rows staged whole in LDS. mfma_stream_fits: K/G a multiple of the
// waves and a wave's staging within its registers; mfma_stream_lds: its dynamic LDS bytes.
hipError_t launch_w4a16_gemm_mfma_stream(const GemvLaunch& launch, hipStream_t stream);
bool mfma_stream_fits(int group_size, int k, int batch);
size_t mfma_stream_lds(int group_size, int k, int batch);

}  // namespace fk
