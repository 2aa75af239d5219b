// Validation, launch policy and vendor baseline behind the ARC W4A16 op API (arc_w4a16.h).
//
// Validation rules and error classes follow the reference (arc_w4a16.cu:23-85, 649-828):
// group_size in {64,128}; batch, k > 0; k % group_size == 0; n > 0 and n % 128 == 0;
// packet_stride_bytes == 128*G/2 + 512; 1 < split_k_slices <= K/G for the split-K entry point.
// Every check runs before any device call. HIP errors are checked after every launch.
#include "ops/decode_quant_linear/arc_w4a16.h"

#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <array>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>

#include "kernels/decode_quant_linear/w4a16_aux.h"
#include "kernels/decode_quant_linear/w4a16_gemv.h"
#include "ops/decode_quant_linear/w4a16_scratch.h"

namespace fast_kernels::decode_quant_linear {
namespace {

constexpr int kTileCols = fk::kTileCols;
constexpr int kMaxDevices = 64;
constexpr std::size_t kCounterRegionAlign = 256;
// Split-K workspace layout: a fixed counter region (one uint32 per (tile, m-tile)) followed by
// the fp32 partials. Fixing the region's size keeps every shape's counters clear of any other
// shape's partials, so one zero-filled workspace serves calls of different shapes.
constexpr std::size_t kMaxFixupCounters = 16384;
constexpr std::size_t kCounterRegionBytes = kMaxFixupCounters * sizeof(std::uint32_t);

[[noreturn]] void throw_invalid(const std::string& message) { throw std::invalid_argument(message); }

void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) {
    std::ostringstream oss;
    oss << what << " failed: " << hipGetErrorString(status);
    throw std::runtime_error(oss.str());
  }
}

void validate_group_size_and_k(int batch, int k, int group_size) {
  if (batch <= 0 || k <= 0) {
    throw_invalid("batch and k must be positive");
  }
  if (group_size != 64 && group_size != 128) {
    throw_invalid("group_size must be 64 or 128");
  }
  if (k % group_size != 0) {
    throw_invalid("k must be divisible by group_size");
  }
}

void validate_dimensions(int batch, int n, int k, int group_size) {
  validate_group_size_and_k(batch, k, group_size);
  if (n <= 0) {
    throw_invalid("n must be positive");
  }
  if (n % kTileCols != 0) {
    throw_invalid("n must be a multiple of 128");
  }
}

void validate_packet_stride(int group_size, int packet_stride_bytes) {
  const int expected = fk::packet_stride_bytes(group_size);
  if (packet_stride_bytes != expected) {
    std::ostringstream oss;
    oss << "packet_stride_bytes=" << packet_stride_bytes << " does not match expected " << expected;
    throw_invalid(oss.str());
  }
}

void validate_pointer(std::uintptr_t ptr, std::size_t alignment, const char* name) {
  if (ptr == 0) {
    throw_invalid(std::string(name) + " must not be null");
  }
  if (ptr % alignment != 0) {
    std::ostringstream oss;
    oss << name << " must be " << alignment << "-byte aligned";
    throw_invalid(oss.str());
  }
}

void validate_activation_dtype(int activation_dtype) {
  if (activation_dtype != kActivationF16 && activation_dtype != kActivationBF16) {
    throw_invalid("activation_dtype must be 0 (fp16) or 1 (bf16)");
  }
}

// CU count per device, read once (the reference queries device properties on every call,
// arc_w4a16.cu:512-518).
int device_cu_count() {
  static std::array<int, kMaxDevices> cache{};
  static std::mutex mutex;
  int device = 0;
  check_hip(hipGetDevice(&device), "hipGetDevice");
  if (device < 0 || device >= kMaxDevices) {
    throw std::runtime_error("device index out of range");
  }
  std::lock_guard<std::mutex> lock(mutex);
  if (cache[device] == 0) {
    int count = 0;
    check_hip(hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device),
              "hipDeviceGetAttribute(multiProcessorCount)");
    cache[device] = std::max(count, 1);
  }
  return cache[device];
}


// Largest LDS one workgroup may hold on the current device, read once. A host-only plan (a given
// CU count) assumes gfx950's 160 KB.
constexpr std::size_t kGfx950LdsBytes = 160 * 1024;

std::size_t device_lds_per_block() {
  static std::array<std::size_t, kMaxDevices> cache{};
  static std::mutex mutex;
  int device = 0;
  check_hip(hipGetDevice(&device), "hipGetDevice");
  if (device < 0 || device >= kMaxDevices) {
    throw std::runtime_error("device index out of range");
  }
  std::lock_guard<std::mutex> lock(mutex);
  if (cache[device] == 0) {
    int bytes = 0;
    check_hip(hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, device),
              "hipDeviceGetAttribute(maxSharedMemoryPerBlock)");
    cache[device] = static_cast<std::size_t>(std::max(bytes, 1));
  }
  return cache[device];
}

// Smallest run per workgroup: two groups per wave, so every wave has a buffered group behind
// the one it computes.
constexpr int kMinGroupsPerWorkgroup = 8;
// Longest run the automatic policy gives a workgroup before splitting K further: one staging
// chunk of activations for narrow slices.
constexpr int kMaxRunGroups = 64;
// Several rows (m-tiles of 4 and up): shortest run of a K split.
constexpr int kMinRowsRunGroups = 16;
// Narrowest column slice (the GEMV kernel serves 128, 64 and 32 columns per workgroup).
constexpr int kMaxSlicesPerTile = 4;
// Longest K for which one-row native plans stream slice pairs.
constexpr int kMaxPairK = 4096;

// Grid, run length and fix-up workspace of a stream-K plan over tiles x slices x num_groups units.
void finish_plan(ArcW4A16Plan& plan, long long tiles, long long slices, int num_groups,
                 long long per, int n, int batch) {
  plan.slice_cols = static_cast<int>(fk::kTileCols / slices);
  plan.schedule = kScheduleRuns;
  const long long units = tiles * slices * num_groups;
  const long long workgroups = (units + per - 1) / per;
  if (workgroups > 0x7fffffffLL || per > 0x7fffffffLL) {
    throw_invalid("shape too large for one launch");
  }
  plan.workgroups = static_cast<int>(workgroups);
  plan.groups_per_workgroup = static_cast<int>(per);
  const bool aligned = per % num_groups == 0;  // every slice lies inside one run
  plan.max_tile_contributors = aligned ? 1 : static_cast<int>((num_groups + per - 1) / per + 1);
  if (aligned) {
    plan.workspace_bytes = 0;
  } else {
    if (static_cast<std::size_t>(tiles * slices) > kMaxFixupCounters) {
      throw_invalid("n * ceil(batch / m_tile) / 128 exceeds the split tile capacity (16384)");
    }
    plan.workspace_bytes =
        kCounterRegionBytes + fk::gemv_streamk_partial_floats(n, batch, plan.m_tile,
                                                              plan.max_tile_contributors) *
                                  sizeof(float);
  }
}

fk::PacketFormat to_packet_format(int packet_format, bool allow_arc) {
  switch (packet_format) {
    case kPacketArc:
      if (allow_arc) return fk::PacketFormat::kArc;
      break;
    case kPacketNativeSym: return fk::PacketFormat::kNativeSym;
    case kPacketNativeAsym: return fk::PacketFormat::kNativeAsym;
    default: break;
  }
  throw_invalid(allow_arc ? "packet_format must be 0 (reference), 1 (native symmetric) or 2 "
                            "(native asymmetric)"
                          : "packet_format must be 1 (native symmetric) or 2 (native asymmetric)");
}

// Native slabs: shortest K run worth splitting a slice across workgroups.
constexpr int kMinNativeRunGroups = 32;
// Long K: one more split of every slice while that keeps at most two workgroups per CU and runs of
// at least this many groups. Measured on MI355X at 70B down (256 slices x 224 groups): runs of
// 112 over 512 workgroups take 24.9 us, whole slices 26.6 us; 70B o (64 groups) gets slower.
constexpr int kMinLongRunGroups = 96;

}  // namespace

namespace {

// Activation rows per m-tile for a kernel choice: the automatic dispatch, the dot2 loop forced
// (at most 8-row tiles) or the matrix-core kernel forced (16-row tiles).
int m_tile_for_kernel(int batch, int kernel) {
  switch (kernel) {
    case kKernelAuto: return fk::gemv_m_tile_for_batch(batch);
    case kKernelDot2: return fk::gemv_partials_m_tile_for_batch(batch);
    case kKernelMfma: return fk::kMfmaRows;
    default: throw_invalid("kernel must be 0 (automatic), 1 (dot2) or 2 (matrix cores)");
  }
}

ArcW4A16Plan plan_arc_impl(int batch, int n, int k, int group_size, int activation_dtype,
                           int split_k_slices, int cu_count, int m_tile);
bool arc_stream_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
                     int split_k_slices, int cu_count, bool cu_count_given);
bool arc_quarter_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
                      int split_k_slices, int cu_count, bool cu_count_given);
bool arc_mfma_stream_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
                          int split_k_slices, int cu_count, bool cu_count_given);

}  // namespace

ArcW4A16Plan plan_arc_w4a16_for_cu_count(int batch, int n, int k, int group_size,
                                         int activation_dtype, int split_k_slices, int cu_count) {
  validate_dimensions(batch, n, k, group_size);
  ArcW4A16Plan plan = plan_arc_impl(batch, n, k, group_size, activation_dtype, split_k_slices,
                                    cu_count, fk::gemv_m_tile_for_batch(batch));
  if (!arc_mfma_stream_plan(plan, batch, n, k, group_size, split_k_slices, cu_count, true) &&
      !arc_stream_plan(plan, batch, n, k, group_size, split_k_slices, cu_count, true)) {
    arc_quarter_plan(plan, batch, n, k, group_size, split_k_slices, cu_count, true);
  }
  return plan;
}

namespace {

ArcW4A16Plan plan_arc_impl(int batch, int n, int k, int group_size, int activation_dtype,
                           int split_k_slices, int cu_count, int m_tile) {
  validate_dimensions(batch, n, k, group_size);
  validate_activation_dtype(activation_dtype);
  if (split_k_slices < 0) {
    throw_invalid("split_k_slices must be >= 0 (0 = automatic)");
  }
  if (cu_count <= 0) {
    throw_invalid("cu_count must be positive");
  }
  ArcW4A16Plan plan{};
  plan.m_tile = m_tile;
  const int num_groups = k / group_size;
  const long long tiles = static_cast<long long>(fk::gemv_tiles(n, batch, plan.m_tile));
  long long slices = 1;
  long long per = 0;
  if (split_k_slices > 0) {
    const int s_req = std::min(split_k_slices, num_groups);
    per = (num_groups + s_req - 1) / s_req;
  } else {
    // Measured on MI355X over the Llama-7B/8B/70B decode shapes. One activation row: one
    // workgroup per CU with long runs is best. Shapes with at least as many tiles as half the
    // CUs run whole tiles over all of K. Otherwise K is split (power of two) until runs are at
    // most kMaxRunGroups long while the runs still fit on the CUs, and then tiles are cut into
    // 64- or 32-column slices while those fit: narrow slices add workgroups without the
    // cross-workgroup fix-up a K split costs. Several rows (more arithmetic per byte): two
    // workgroups per CU, from K splits alone, runs of at least kMinGroupsPerWorkgroup groups.
    long long s_split = 1;
    if (plan.m_tile == 1) {
      auto can_split = [&](long long s) {
        return tiles * s * 2 <= cu_count && num_groups / (s * 2) >= kMinGroupsPerWorkgroup;
      };
      while (num_groups / s_split > kMaxRunGroups && can_split(s_split)) {
        s_split *= 2;
      }
      while (slices < kMaxSlicesPerTile && tiles * s_split * slices * 2 <= cu_count) {
        slices *= 2;
      }
    } else {
      // from four rows, runs of at least 16 groups (long K over the reference packets:
      // 4096 x 14336 G64 at 4 rows 15.3 -> 14.8 us, at 8 rows 15.8 -> 14.3, with 28-group runs)
      const int min_run = plan.m_tile >= 4 ? kMinRowsRunGroups : kMinGroupsPerWorkgroup;
      while (tiles * s_split * 2 <= 2LL * cu_count && num_groups / (s_split * 2) >= min_run) {
        s_split *= 2;
      }
    }
    per = (num_groups + s_split - 1) / s_split;
  }
  finish_plan(plan, tiles, slices, num_groups, per, n, batch);
  return plan;
}

// Stream schedule switches, read once: FK_W4A16_STREAM=0 turns it off (the per-slice runs then
// serve one-row native plans), FK_W4A16_STREAM_WPC=2 runs two workgroups per CU.
bool stream_schedule_enabled() {
  static const bool enabled = [] {
    const char* v = std::getenv("FK_W4A16_STREAM");
    return v == nullptr || std::string(v) != "0";
  }();
  return enabled;
}

// FK_W4A16_STREAM_PIECES=0 keeps shapes whose slices do not divide over the CUs off the stream
// schedule.
bool env_enabled(const char* name) {
  const char* v = std::getenv(name);
  return v == nullptr || std::string(v) != "0";
}
bool stream_pieces_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_STREAM_PIECES");
  return enabled;
}


// FK_W4A16_STREAM_DIVISOR=0 keeps shapes whose slices divide only over fewer workgroups than
// CUs off the stream schedule's divisor grids.
bool stream_divisor_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_STREAM_DIVISOR");
  return enabled;
}

// The largest grid of at least 7/8 of the CUs that divides more slices than CUs: every workgroup
// then streams the same whole slices with no piece to hand off, the idle CUs costing less than
// the pieces' imbalance (blocks do not divide evenly either) and hand-offs. 0 when there is none.
long long divisor_grid(long long slices, long long cus) {
  if (slices <= cus || !stream_divisor_enabled()) {
    return 0;
  }
  for (long long g = cus; 8 * g >= 7 * cus; --g) {
    if (slices % g == 0) {
      return g;
    }
  }
  return 0;
}

// FK_W4A16_MFMA_STREAM=0 keeps 2-16-row native launches off the matrix-core stream kernel.
constexpr int kMfmaStreamMinBatch = 2;
constexpr int kMfmaStreamMaxBatch = 16;
constexpr int kMfmaPiecesMinBatch = 3;
constexpr int kMfmaPiecesMaxBatch = 8;
bool mfma_stream_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_MFMA_STREAM");
  return enabled;
}

// FK_W4A16_STREAM_HALF=0 keeps shapes with at most half as many slices as CUs off half-slices.
bool stream_half_enabled() {
  static const bool enabled = [] {
    const char* v = std::getenv("FK_W4A16_STREAM_HALF");
    return v == nullptr || std::string(v) != "0";
  }();
  return enabled;
}

// FK_W4A16_HALF_WHOLE=0 keeps shapes whose half-slices (not slices) divide over the CUs off the
// stream schedule.
constexpr long long kMaxHalvesPerCu = 4;
bool stream_half_whole_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_HALF_WHOLE");
  return enabled;
}

// FK_W4A16_STREAM_SMALL=0 keeps shapes with fewer slices than CUs on the per-slice runs.
bool stream_small_enabled() {
  static const bool enabled = [] {
    const char* v = std::getenv("FK_W4A16_STREAM_SMALL");
    return v == nullptr || std::string(v) != "0";
  }();
  return enabled;
}

int stream_workgroups_per_cu() {
  static const int wpc = [] {
    const char* v = std::getenv("FK_W4A16_STREAM_WPC");
    const int n = v == nullptr ? 1 : std::atoi(v);
    return n >= 1 && n <= 4 ? n : 1;
  }();
  return wpc;
}

// FK_W4A16_STREAM_FUSED=0 keeps the fused decode-step neighbours on their per-slice kernels.
bool stream_fused_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_STREAM_FUSED");
  return enabled;
}

// FK_W4A16_ARC_STREAM=0 keeps one-row launches over the reference packets off the stream
// schedule (w4a16_gemv_arc_stream.hip).
bool arc_stream_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_ARC_STREAM");
  return enabled;
}

// One row over the reference packets on the stream schedule: whole 128-column tiles per CU plus
// pieces of the tiles left over (the native stream kernel's split, tiles for slices), or whole
// tiles only over a divisor grid of at least 7/8 of the CUs when one exists. Blocks are
// 2 D groups (D = 2 at G = 128, 4 at G = 64). Only with at least one whole tile per CU: measured
// on MI355X (bench.py --packets arc, alternating runs), 70B gate_up (448 tiles, one whole tile and
// a piece per CU) 39.6 -> 39.1 us against the per-tile runs, while the shapes with fewer tiles than
// CUs, all pieces, got slower (70B qkv 11.3 -> 13.2 us, o 8.4 -> 10.4, down 22.4 -> 23.4). False
// (plan unchanged) when it does not apply.
bool arc_stream_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
                     int split_k_slices, int cu_count, bool cu_count_given) {
  if (batch != 1 || plan.m_tile != 1 || split_k_slices != 0 || k > fk::kStreamMaxK ||
      !arc_stream_enabled()) {
    return false;
  }
  const int num_groups = k / group_size;
  const int per_block = group_size == 128 ? 4 : 8;
  const std::size_t lds = fk::arc_stream_lds(group_size, k) + 16 * 1024;
  const std::size_t lds_limit = cu_count_given ? kGfx950LdsBytes : device_lds_per_block();
  if (num_groups % per_block != 0 || lds > lds_limit) {
    return false;
  }
  const long long nbt = num_groups / per_block;
  const long long tiles = n / fk::kTileCols;
  // Tiles that do not divide over the CUs but over a divisor grid of at least 7/8 of them: that
  // grid, whole tiles only (70B gate_up, 448 tiles: 2 per workgroup on 224 CUs 37.8-38.1 us
  // against 1 tile and pieces on 256 CUs 39.3-39.4, and 40.9-41.4 by packet quarters, 8 per
  // workgroup on 224 CUs; alternating runs on one GPU).
  long long cus = cu_count;
  if (const long long dgrid = divisor_grid(tiles, cus); dgrid > 0 && tiles % cus != 0) {
    cus = dgrid;
  }
  const long long whole = tiles / cus;
  const long long left = tiles - whole * cus;
  const bool pieces = left > 0;
  if (whole < 1 || tiles > fk::kStreamMaxSlices || (pieces && (left * nbt < cus ||
                                                  left * nbt * cus >= (1LL << 31)))) {
    return false;
  }
  plan.schedule = kScheduleStream;
  plan.slice_cols = fk::kTileCols;
  plan.workgroups = static_cast<int>(cus);
  plan.stream_depth = group_size == 128 ? 2 : 4;
  plan.stream_whole = static_cast<int>(whole);
  plan.stream_pieces = pieces ? 1 : 0;
  plan.stream_half = 0;
  const long long piece_blocks = pieces ? (left * nbt + cus - 1) / cus : 0;
  plan.groups_per_workgroup = static_cast<int>(whole * num_groups + piece_blocks * per_block);
  plan.max_tile_contributors =
      pieces ? static_cast<int>((nbt * cus + left * nbt - 1) / (left * nbt) + 1) : 1;
  plan.workspace_bytes =
      pieces ? kCounterRegionBytes + static_cast<std::size_t>(cus) * 2 * fk::kTileCols * sizeof(float)
             : 0;
  return true;
}

// FK_W4A16_ARC_QUARTER=0 keeps one-row launches over the reference packets off the quarter
// schedule (w4a16_gemv_arc_quarter.hip).
bool arc_quarter_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_ARC_QUARTER");
  return enabled;
}

// FK_W4A16_ARC_MFMA_STREAM=0 keeps 2-16-row launches over the reference packets off the
// matrix-core stream kernel.
bool arc_mfma_stream_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_ARC_MFMA_STREAM");
  return enabled;
}

// FK_W4A16_ARC_EIGHTHS=0 keeps the quarter schedule over reference packets off 16-column units.
bool arc_eighths_enabled() {
  static const bool enabled = env_enabled("FK_W4A16_ARC_EIGHTHS");
  return enabled;
}

// One row over the reference packets by 32-column quarters of the packets, for the shapes with
// fewer 128-column tiles than CUs (the whole-tile stream schedule, arc_stream_plan, takes the
// others: 70B gate_up 39.7 us on it against 41.0 by quarters). The slices are dealt like the
// native stream kernel's: whole slices per CU when they divide, pieces of the slices left over
// when there are more slices than CUs and K is long (K/G >= 64), a divisor grid of at least 7/8
// of the CUs, one 16-column eighth per workgroup when there are at most half as many slices as
// CUs and K is short (G = 128, K/G <= 32), or one slice per workgroup when there are fewer slices
// than CUs and the per-tile runs would not split K either. Blocks are 8 waves x D groups (D = 2 at G = 128, 4 at G = 64).
// Measured on MI355X (bench.py --packets arc, alternating runs against the per-tile runs): 70B
// qkv 11.4 -> 10.0 us, o 8.4 -> 7.7, down 22.4 -> 21.8; 7B o 5.06 -> 4.24. False (plan
// unchanged) when it does not apply.
bool arc_quarter_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
                      int split_k_slices, int cu_count, bool cu_count_given) {
  if (batch != 1 || plan.m_tile != 1 || split_k_slices != 0 || k > fk::kStreamMaxK ||
      !arc_quarter_enabled()) {
    return false;
  }
  const int num_groups = k / group_size;
  const int depth = group_size == 128 ? 2 : 4;
  const int per_block = fk::kStreamWaves * depth;
  const std::size_t lds = fk::arc_quarter_lds(group_size, k) + fk::kStreamStaticLdsBytes;
  const std::size_t lds_limit = cu_count_given ? kGfx950LdsBytes : device_lds_per_block();
  const long long slices = n / fk::kSliceCols;
  if (num_groups % per_block != 0 || lds > lds_limit || slices > fk::kStreamMaxSlices ||
      !fk::arc_quarter_magic_exact(num_groups, slices)) {
    return false;
  }
  constexpr int kMinPieceGroups = 64;
  // 16-column eighths, one per workgroup, for short K only (measured on MI355X, bench.py
  // --packets arc, alternating runs: 7B o 4.20-4.23 -> 4.03-4.06 us, 8B o 4.34-4.37 -> 4.07-4.08;
  // 8B down, K/G = 112, 9.07-9.19 -> 9.01-9.56; 7B qkv as three eighths per CU 6.9 -> 9.8).
  constexpr int kMaxEighthGroups = 32;
  const long long nbs = num_groups / per_block;
  const long long cus = cu_count;
  const long long left = slices % cus;
  long long grid = 0;
  int whole = 0;
  bool pieces = false;
  bool eighths = false;
  if (slices >= cus && left == 0) {
    grid = cus;
    whole = static_cast<int>(slices / cus);
  } else if (const long long dgrid = divisor_grid(slices, cus); dgrid > 0) {
    // ahead of pieces, as on native slabs; the per-tile runs are faster still at G = 64
    // (14336 x 4096 G64: pieces 10.4 us, quarters on 224 CUs 7.6, 64-column runs on 224 7.2) and
    // where the whole tiles alone fill 7/8 of the CUs (28672 x 4096, 224 tiles: 11.96 against
    // 11.68 us; 28672 x 8192: 21.6 against 21.3)
    if (group_size != 128 || 8 * (slices / 4) >= 7 * cus) {
      return false;
    }
    grid = dgrid;
    whole = static_cast<int>(slices / dgrid);
  } else if (slices > cus && left * nbs >= cus && num_groups >= kMinPieceGroups &&
             left * nbs * cus < (1LL << 31)) {
    grid = cus;
    whole = static_cast<int>(slices / cus);
    pieces = true;
  } else if (group_size == 128 && 2 * slices <= cus && num_groups <= kMaxEighthGroups &&
             arc_eighths_enabled() && fk::arc_quarter_magic_exact(num_groups, 2 * slices)) {
    grid = 2 * slices;
    whole = 1;
    eighths = true;
  } else if (slices < cus && plan.groups_per_workgroup == num_groups) {
    grid = slices;
    whole = 1;
  } else {
    return false;
  }
  if (eighths && fk::arc_quarter_lds(group_size, k, fk::kSliceCols / 2) +
                         fk::kStreamStaticLdsBytes > lds_limit) {
    return false;
  }
  plan.schedule = kScheduleStream;
  plan.slice_cols = eighths ? fk::kSliceCols / 2 : fk::kSliceCols;
  plan.workgroups = static_cast<int>(grid);
  plan.stream_depth = depth;
  plan.stream_whole = whole;
  plan.stream_pieces = pieces ? 1 : 0;
  plan.stream_half = 0;
  const long long left_blocks = (slices - grid * whole) * nbs;
  const long long piece_blocks = pieces ? (left_blocks + grid - 1) / grid : 0;
  plan.groups_per_workgroup = static_cast<int>(whole * num_groups + piece_blocks * per_block);
  plan.max_tile_contributors =
      pieces ? static_cast<int>((nbs * grid + left_blocks - 1) / left_blocks + 1) : 1;
  plan.workspace_bytes =
      pieces ? kCounterRegionBytes +
                   fk::stream_partial_floats(static_cast<int>(grid), 1) * sizeof(float)
             : 0;
  return true;
}

// The stream kernel with a fused neighbour (one row, w4a16_gemv_stream.hip's kFuse): whole units
// per workgroup, a unit being a 32-column slice (RMSNorm prologue) or a gate slice with its up
// slice (SiLU epilogue, up to 4 pairs per workgroup): over every CU when they divide, else over a
// divisor grid of at least 7/8 of them, else one unit per workgroup when there are fewer units
// than CUs. No pieces and no half slices. False when the shape does not fit (the per-slice fused
// kernels then serve it). Measured on MI355X (Llama-8B, bf16, rocprofv3 over the decode-step
// suite): RMSNorm + gate_up + SiLU 13.9 -> 12.0 us (the plain gate_up: 11.6), RMSNorm + qkv 5.8
// either way (the prologue's barrier and conversions sit ahead of a short stream); the 32-layer
// fused chain 1011 -> 920 us.
bool fused_stream_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size, bool silu,
                       int cu_count) {
  if (batch != 1 || k > fk::kStreamMaxK || !stream_schedule_enabled() || !stream_fused_enabled()) {
    return false;
  }
  const bool cu_count_given = cu_count > 0;
  if (!cu_count_given) {
    cu_count = device_cu_count();
  }
  const int num_groups = k / group_size;
  const int depth = fk::stream_depth_for_kb(group_size, fk::kStreamKB);
  const std::size_t lds =
      fk::stream_lds_bytes(group_size, num_groups + 1) + fk::kStreamStaticLdsBytes;
  const std::size_t lds_limit = cu_count_given ? kGfx950LdsBytes : device_lds_per_block();
  const long long slices = n / fk::kSliceCols;
  if (num_groups % (fk::kStreamWaves * depth) != 0 || lds > lds_limit ||
      (silu && slices % 2 != 0)) {
    return false;
  }
  const long long units = silu ? slices / 2 : slices;
  const long long cus = cu_count;
  long long grid = 0;
  if (units % cus == 0) {
    grid = cus;
  } else if (const long long dgrid = divisor_grid(units, cus); dgrid > 0) {
    grid = dgrid;
  } else if (units < cus) {
    grid = units;
  }
  if (grid == 0 || (silu && units / grid > 4)) {
    return false;
  }
  plan.m_tile = 1;
  plan.schedule = kScheduleStream;
  plan.slice_cols = fk::kSliceCols;
  plan.workgroups = static_cast<int>(grid);
  plan.stream_depth = depth;
  plan.stream_whole = static_cast<int>(units / grid) * (silu ? 2 : 1);
  plan.stream_pieces = 0;
  plan.stream_half = 0;
  plan.groups_per_workgroup = plan.stream_whole * num_groups;
  plan.max_tile_contributors = 1;
  plan.workspace_bytes = 0;
  return true;
}

// The matrix cores on the stream schedule (w4a16_gemm_mfma_stream.hip) for 2-16 rows: the rows
// staged whole in LDS, one workgroup per CU streaming whole 32-column slices of native slabs, or
// (arc) 32-column quarters of the reference packets. False (plan unchanged) when the shape does
// not fit. Measured on MI355X (benchmark configuration 3, 14336 x 4096, G = 64, asymmetric, fp16:
// 448 slices, two per workgroup on a divisor grid of 224 CUs; alternating runs on one GPU against
// the plans without it): 2 rows 9.8 -> 8.6 us, 4 rows 10.9 -> 8.6, 8 rows 12.5 -> 10.0, 16 rows
// 13.0 -> 11.4. With pieces of the slices left over (256 CUs, a block of 32 groups the unit, so
// ranges of 1 or 2 blocks) the same shape took 11.0 us at 4 rows and 12.6 at 8, and two and
// sixteen rows were slower than without the stream schedule: pieces only for 3-8 rows.
// K too long to stage whole rows: K in the fewest equal parts whose rows fit the staging, each
// workgroup streaming whole slices over one part (the slices in groups of `whole`, every part with
// the same groups), over a grid of 7/8 of the CUs or more; the parts' fp32 sums go to the
// workspace and a second launch adds them in part order. Within kMaxPartsBytes of partials, from
// kMfmaPartsMinBatch rows. Measured on MI355X (plan sweep, against the best per-tile plan): 4096 x
// 14336 G64 at 4 rows 14.8 -> 12.9 us (reference packets) and 13.7 -> 12.6 (native), 70B qkv at
// 4 rows 18.0 -> 14.7, 70B down at 4 rows 31.1 -> 29.0 and at 8 rows 31.9 -> 29.2; at 8 rows of
// 4096 x 14336 even (14.2); at 2 rows slower (11.5 -> 12.5 us: the second launch and the parts'
// slice ends cost more than two rows gain).
constexpr int kMfmaPartsMinBatch = 3;
bool mfma_stream_parts_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
                            int cu_count, std::size_t lds_limit) {
  constexpr long long kMaxPartsBytes = 6LL << 20;
  const int depth = fk::stream_depth_for_kb(group_size, fk::kStreamKB);
  const int num_groups = k / group_size;
  const int quantum = fk::kStreamWaves * depth;
  const long long slices = n / fk::kSliceCols;
  const long long cus = cu_count;
  for (int parts = 2; parts <= num_groups / quantum; ++parts) {
    const int ngs = num_groups / parts;
    if (num_groups % parts != 0 || ngs % quantum != 0 ||
        !fk::mfma_stream_fits(group_size, ngs * group_size, batch) ||
        fk::mfma_stream_lds(group_size, ngs * group_size, batch) > lds_limit ||
        static_cast<long long>(parts) * batch * n * 4 > kMaxPartsBytes) {
      continue;
    }
    // slice groups per part: the most that keep parts x groups within the CUs and at 7/8 or more
    long long groups = 0;
    for (long long gs = cus / parts; gs >= 1 && 8 * parts * gs >= 7 * cus; --gs) {
      if (slices % gs == 0) {
        groups = gs;
        break;
      }
    }
    if (groups == 0) {
      continue;
    }
    plan.m_tile = fk::kMfmaRows;
    plan.schedule = kScheduleStream;
    plan.slice_cols = fk::kSliceCols;
    plan.workgroups = static_cast<int>(parts * groups);
    plan.stream_depth = depth;
    plan.stream_whole = static_cast<int>(slices / groups);
    plan.stream_pieces = 0;
    plan.stream_half = 0;
    plan.groups_per_workgroup = plan.stream_whole * ngs;
    plan.max_tile_contributors = parts;
    plan.workspace_bytes =
        kCounterRegionBytes + static_cast<std::size_t>(parts) * batch * n * sizeof(float);
    return true;
  }
  return false;
}

bool mfma_stream_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size, bool arc,
                      int cu_count, bool cu_count_given) {
  const std::size_t lds_limit = cu_count_given ? kGfx950LdsBytes : device_lds_per_block();
  const int depth = fk::stream_depth_for_kb(group_size, fk::kStreamKB);
  const int num_groups = k / group_size;
  const int nbs = num_groups / (fk::kStreamWaves * depth);
  const long long slices = n / fk::kSliceCols;
  const long long cus = cu_count;
  if (num_groups % (fk::kStreamWaves * depth) != 0 || slices > fk::kStreamMaxSlices) {
    return false;
  }
  if (!fk::mfma_stream_fits(group_size, k, batch) ||
      fk::mfma_stream_lds(group_size, k, batch) > lds_limit) {
    return batch >= kMfmaPartsMinBatch &&
           mfma_stream_parts_plan(plan, batch, n, k, group_size, cu_count, lds_limit);
  }
  if (arc && !fk::arc_quarter_magic_exact(num_groups, slices)) {
    return false;
  }
  const long long left = slices % cus;
  const long long dgrid = divisor_grid(slices, cus);
  long long grid = 0;
  int whole = 0;
  bool pieces = false;
  if (slices >= cus && left == 0) {
    grid = cus;
    whole = static_cast<int>(slices / cus);
  } else if (dgrid > 0) {
    grid = dgrid;
    whole = static_cast<int>(slices / dgrid);
  } else if (slices > cus && left * nbs >= cus && batch >= kMfmaPiecesMinBatch &&
             batch <= kMfmaPiecesMaxBatch && !arc) {
    // (pieces over the reference packets spill registers: no pieces there)
    grid = cus;
    whole = static_cast<int>(slices / cus);
    pieces = true;
  } else if (slices < cus) {
    // fewer slices than CUs: one each (4096 x 4096, two rows over reference packets: 7.6 -> 5.25
    // us at G = 64, 6.9 -> 4.9 at G = 128, against the per-tile kernels)
    grid = slices;
    whole = 1;
  } else {
    return false;
  }
  plan.m_tile = fk::kMfmaRows;
  plan.schedule = kScheduleStream;
  plan.slice_cols = fk::kSliceCols;
  plan.workgroups = static_cast<int>(grid);
  plan.stream_depth = depth;
  plan.stream_whole = whole;
  plan.stream_pieces = pieces ? 1 : 0;
  plan.stream_half = 0;
  const long long left_blocks = (slices - grid * whole) * nbs;
  const long long piece_blocks = pieces ? (left_blocks + grid - 1) / grid : 0;
  plan.groups_per_workgroup =
      static_cast<int>(whole * num_groups + piece_blocks * fk::kStreamWaves * depth);
  plan.max_tile_contributors =
      pieces ? static_cast<int>((nbs * grid + left_blocks - 1) / left_blocks + 1) : 1;
  plan.workspace_bytes =
      pieces ? kCounterRegionBytes +
                   fk::stream_partial_floats(static_cast<int>(grid), fk::kMfmaRows) * sizeof(float)
             : 0;
  return true;
}

// The reference-signature plan's matrix-core stream schedule over the reference packets (the
// automatic kernel choice).
bool arc_mfma_stream_plan(ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
                          int split_k_slices, int cu_count, bool cu_count_given) {
  return split_k_slices == 0 && batch >= kMfmaStreamMinBatch && batch <= kMfmaStreamMaxBatch &&
         mfma_stream_enabled() && arc_mfma_stream_enabled() &&
         mfma_stream_plan(plan, batch, n, k, group_size, true, cu_count, cu_count_given);
}

// plan_w4a16_for_format for a kernel choice (kKernelDot2 is what the fused kernels need).
ArcW4A16Plan plan_for_format_impl(int batch, int n, int k, int group_size, int activation_dtype,
                                  int split_k_slices, int cu_count, int packet_format,
                                  int kernel, bool plain = true) {
  const fk::PacketFormat format = to_packet_format(packet_format, true);
  validate_dimensions(batch, n, k, group_size);
  const bool cu_count_given = cu_count > 0;
  if (cu_count == 0) {
    cu_count = device_cu_count();
  }
  ArcW4A16Plan plan = plan_arc_impl(batch, n, k, group_size, activation_dtype, split_k_slices,
                                    cu_count, m_tile_for_kernel(batch, kernel));
  if (plain && split_k_slices == 0 && batch >= kMfmaStreamMinBatch &&
      batch <= kMfmaStreamMaxBatch && kernel != kKernelDot2 && mfma_stream_enabled() &&
      (format != fk::PacketFormat::kArc || arc_mfma_stream_enabled()) &&
      mfma_stream_plan(plan, batch, n, k, group_size, format == fk::PacketFormat::kArc, cu_count,
                       cu_count_given)) {
    return plan;
  }
  if (format == fk::PacketFormat::kArc && plain && kernel != kKernelMfma &&
      !arc_stream_plan(plan, batch, n, k, group_size, split_k_slices, cu_count, cu_count_given)) {
    arc_quarter_plan(plan, batch, n, k, group_size, split_k_slices, cu_count, cu_count_given);
  }
  if (format == fk::PacketFormat::kArc || plan.m_tile == fk::kMfmaRows) {
    return plan;  // the matrix-core kernel reads whole tiles in every format
  }
  // Native slabs: stream-K over 32-column slices, whose groups are contiguous in memory. Measured
  // on MI355X over the Llama-7B/8B/70B decode shapes: a workgroup per whole slice, over all of K,
  // whatever the slice count (more slices than resident workgroups simply run in later rounds).
  // Only when the slices leave at least half the CUs idle and K is long is K split (power of two),
  // keeping runs of at least kMinNativeRunGroups groups, since the fix-up of a split slice costs
  // about as much as streaming 30 groups. With very long K (kMinLongRunGroups) one split more is
  // taken while it keeps at most two workgroups per CU.
  const int num_groups = k / group_size;
  const long long slices = static_cast<long long>(fk::gemv_tiles(n, batch, plan.m_tile)) * fk::kSlicesPerTile;
  long long per = 0;
  if (split_k_slices > 0) {
    const int s_req = std::min(split_k_slices, num_groups);
    per = (num_groups + s_req - 1) / s_req;
  } else {
    long long s_split = 1;
    while (slices * s_split * 2 <= cu_count && num_groups / (s_split * 2) >= kMinNativeRunGroups) {
      s_split *= 2;
    }
    // (several rows: runs of kMinNativeRunGroups suffice; 4096 x 14336 G64 at 4 rows, 128
    // slices: 16.3 -> 13.7 us with 56-group runs on 512 workgroups)
    const int min_long = batch > 1 ? kMinNativeRunGroups : kMinLongRunGroups;
    while (slices * s_split * 2 <= 2LL * cu_count && num_groups / (s_split * 2) >= min_long) {
      s_split *= 2;
    }
    per = (num_groups + s_split - 1) / s_split;
  }
  // Slice pairs (one row, whole slices): a workgroup streams two adjacent slices at once, two waves
  // each, i.e. 64 columns over all of K. Half the workgroups, each with twice the loads in flight
  // and half the per-workgroup start-up cost per byte. Taken when the pairs fill the chip's rounds
  // of workgroups at least as evenly as the single slices: ceil(S / CUs) >= 2 ceil(S / (2 CUs)).
  // Measured on MI355X: 7B qkv (384 slices) 8.2 -> 7.8 us, 8B gate_up (896) 14.6 -> 13.6 us,
  // 7B gate_up (688 slices, 344 pairs) got 1 us slower, pairs that leave part of the chip idle
  // (70B o, 256 slices) 3 us slower, and with longer K, whose single-slice runs already stream
  // 135 KB, pairs gain nothing (70B qkv, K = 8192: 12.12 -> 12.20 us).
  // The stream schedule (w4a16_gemv_stream.hip): one activation row staged whole in LDS, one
  // workgroup per CU streaming its share of whole slices as one contiguous range, with
  // 4 KB of weights in flight per wave. Measured on MI355X (bench, Llama-70B bf16): o 8.07 ->
  // 7.73 us, down 22.6 -> 21.3, gate_up 39.6 -> 39.8 (equal within the run-to-run spread); 8 and
  // 16 KB per wave are slower (gate_up 39.9 and 41.5 us). Slices that do not divide evenly:
  //  * more slices than CUs and long K: the left-over slices are dealt as equal block ranges
  //    (pieces) on top of the whole slices, and handed off while the whole slices stream;
  //  * at most half as many slices as CUs (G = 128, one row): a half-slice (16 columns, the first
  //    or second KB of every slab) per workgroup, so every CU streams and no slice is split over
  //    K (8B o 4.0 -> 3.9 us, 8B down 8.8 -> 8.0);
  //  * twice the slices a multiple of the CUs, up to kMaxHalvesPerCu half-slices per CU: an even
  //    share of half-slices, 4 KB of half-slabs in flight per wave (7B qkv, 3 per CU, 7.35 ->
  //    6.97 us against slice pairs; 8B gate_up, 7 per CU, 13.5 -> 13.9 us, stays on pairs);
  //  * more slices than CUs with a divisor of them over at least 7/8 of the CUs: that many
  //    workgroups of whole slices, no pieces (8B gate_up, 896 slices, 4 per CU on 224 CUs: 12.4 ->
  //    11.4 us against slice pairs);
  //  * otherwise fewer slices than CUs and K too short to split (per == K/G): one whole slice per
  //    workgroup (8B qkv 5.16 -> 4.44 us, 7B o 4.67 -> 4.15). Pieces with no whole slice to hide
  //    their hand-off behind cost more than they save (8B o 4.8 -> 5.7 us), and 8B down as whole
  //    slices on 128 workgroups is slower than its runs split over K (8.8 -> 10.0 us).
  // Pieces only for long K: measured on MI355X (bench, alternating runs on one GPU), 70B qkv
  // (K/G = 64) 11.9 -> 10.6 us, but 8B gate_up (K/G = 32) 12.6 -> 13.2 us against slice pairs and
  // 7B gate_up 10.5 -> 11.9 us against per-slice runs.
  constexpr int kMinPieceGroups = 64;
  constexpr long long kLargeSlicesPerCu = 4;
  if (plain && split_k_slices == 0 && batch == 1 && plan.m_tile == 1 &&
      k <= fk::kStreamMaxK && stream_schedule_enabled()) {
    const std::size_t lds =
        fk::stream_lds_bytes(group_size, num_groups + 1) + fk::kStreamStaticLdsBytes;
    const std::size_t lds_limit = cu_count_given ? kGfx950LdsBytes : device_lds_per_block();
    const int depth = fk::stream_depth_for_kb(group_size, fk::kStreamKB);
    const int nbs = num_groups / (fk::kStreamWaves * depth);  // blocks per slice
    const long long cus = static_cast<long long>(cu_count) * stream_workgroups_per_cu();
    // Whole blocks per slice, except for half slices, whose last block may be partial (7B down,
    // K/G = 86: 7.4 -> 7.0 us against runs split over K).
    const bool exact = num_groups % (fk::kStreamWaves * depth) == 0;
    if (nbs >= 1 && lds <= lds_limit) {
      long long grid = 0;
      int whole = 0;
      bool pieces = false;
      bool half = false;
      const long long left = slices % cus;
      // Many slices per CU: a divisor grid of 7/8 of the CUs or more when one exists, ahead of
      // every CU (70B gate_up, 1792 slices: 8 per workgroup on 224 CUs 37.0 us against 7 on 256
      // 37.6-38.1, the 70B step 74.3 -> 73.25 us; alternating runs on one GPU). Shapes with one
      // slice per CU measured slower on fewer CUs (70B o, down and qkv on 192-224 workgroups).
      const long long dgrid_large =
          exact && slices >= kLargeSlicesPerCu * cus ? divisor_grid(slices, cus - 1) : 0;
      if (dgrid_large > 0) {
        grid = dgrid_large;
        whole = static_cast<int>(slices / dgrid_large);
      } else if (exact && slices >= cus && left == 0) {
        grid = cus;
        whole = static_cast<int>(slices / cus);
      } else if (const long long dgrid = exact ? divisor_grid(slices, cus) : 0; dgrid > 0) {
        // a divisor grid ahead of pieces (14336 x 4096 G64: 448 slices, 2 per workgroup on 224
        // CUs 6.8 us against 9.3 with pieces of 1 or 2 blocks on 256)
        grid = dgrid;
        whole = static_cast<int>(slices / dgrid);
      } else if (exact && slices > cus && left * nbs >= cus && num_groups >= kMinPieceGroups &&
                 slices <= fk::kStreamMaxSlices && stream_pieces_enabled()) {
        grid = cus;
        whole = static_cast<int>(slices / cus);
        pieces = true;
      } else if (batch == 1 && group_size == 128 && 2 * slices > cus && (2 * slices) % cus == 0 &&
                 2 * slices <= kMaxHalvesPerCu * cus && stream_half_whole_enabled()) {
        grid = cus;
        whole = static_cast<int>(2 * slices / cus);
        half = true;
      } else if (batch == 1 && group_size == 128 && 2 * slices <= cus && stream_half_enabled()) {
        grid = 2 * slices;
        whole = 1;
        half = true;
      } else if (exact && slices < cus && per == num_groups && stream_small_enabled()) {
        grid = slices;
        whole = 1;
      }
      if (grid > 0) {
        plan.schedule = kScheduleStream;
        plan.slice_cols = half ? fk::kSliceCols / 2 : fk::kSliceCols;
        plan.workgroups = static_cast<int>(grid);
        // Half-slices keep a whole slice's 4 KB in flight per wave (four half-slabs) when there are
        // several per workgroup, or one of short K (8B and 7B o, K/G = 32: 3.72 -> 3.53 and 3.64
        // -> 3.52 us); one half-slice of long K measured no better with them.
        const bool deep = half && (whole > 1 || num_groups <= 32) &&
                          num_groups % (fk::kStreamWaves * 2 * depth) == 0;
        plan.stream_depth = deep ? 2 * depth : depth;
        plan.stream_whole = whole;
        plan.stream_pieces = pieces ? 1 : 0;
        plan.stream_half = half ? 1 : 0;
        // groups a workgroup streams (the most, with pieces)
        const long long left_blocks = (slices - grid * whole) * nbs;
        const long long piece_blocks = pieces ? (left_blocks + grid - 1) / grid : 0;
        plan.groups_per_workgroup = static_cast<int>(
            whole * num_groups + piece_blocks * fk::kStreamWaves * depth);
        plan.max_tile_contributors =
            pieces ? static_cast<int>((nbs * grid + left_blocks - 1) / left_blocks + 1) : 1;
        plan.workspace_bytes =
            pieces ? kCounterRegionBytes +
                         fk::stream_partial_floats(static_cast<int>(grid), 1) * sizeof(float)
                   : 0;
        return plan;
      }
    }
  }
  if (plain && split_k_slices == 0 && per == num_groups && plan.m_tile == 1 &&
      k <= kMaxPairK) {
    const long long rounds = (slices + cu_count - 1) / cu_count;
    const long long pair_rounds = (slices / 2 + cu_count - 1) / cu_count;
    if (rounds >= 2 * pair_rounds) {
      finish_plan(plan, fk::gemv_tiles(n, batch, plan.m_tile), fk::kSlicesPerTile / 2,
                  num_groups, per, n, batch);
      plan.schedule = kSchedulePairs;
      return plan;
    }
  }
  finish_plan(plan, fk::gemv_tiles(n, batch, plan.m_tile), fk::kSlicesPerTile, num_groups, per, n,
              batch);
  return plan;
}

}  // namespace

ArcW4A16Plan plan_w4a16_for_format(int batch, int n, int k, int group_size, int activation_dtype,
                                   int split_k_slices, int cu_count, int packet_format) {
  return plan_for_format_impl(batch, n, k, group_size, activation_dtype, split_k_slices, cu_count,
                              packet_format, kKernelAuto);
}

ArcW4A16Plan plan_w4a16_for_kernel(int batch, int n, int k, int group_size, int activation_dtype,
                                   int split_k_slices, int cu_count, int packet_format,
                                   int kernel) {
  return plan_for_format_impl(batch, n, k, group_size, activation_dtype, split_k_slices, cu_count,
                              packet_format, kernel);
}

namespace {

// Library-owned fix-up workspace for the reference-signature forward, which has no workspace
// argument: one per (device, stream), so that calls on different streams never share counters or
// partials. Grown on demand (so the first call for a larger shape on a stream allocates and must
// not run under stream capture): the old buffer is freed after synchronising its stream, its only
// user. The counter region is zeroed, stream-ordered, at allocation, and the kernel leaves it
// zeroed. (The reference shares one cached group_sums buffer across streams instead,
// decode_quant_linear.py:150-168.)
struct StreamWorkspace {
  void* ptr = nullptr;
  std::size_t bytes = 0;
};

void* library_workspace(std::size_t bytes, hipStream_t stream) {
  static std::map<std::pair<int, hipStream_t>, StreamWorkspace> spaces;
  static std::mutex mutex;
  int device = 0;
  check_hip(hipGetDevice(&device), "hipGetDevice");
  std::lock_guard<std::mutex> lock(mutex);
  StreamWorkspace& ws = spaces[{device, stream}];
  if (ws.bytes < bytes) {
    if (ws.ptr != nullptr) {
      check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
      check_hip(hipFree(ws.ptr), "hipFree");
      ws.ptr = nullptr;
      ws.bytes = 0;
    }
    const std::size_t grown = std::max<std::size_t>(bytes, 1u << 20);
    check_hip(hipMalloc(&ws.ptr, grown), "hipMalloc(workspace)");
    check_hip(hipMemsetAsync(ws.ptr, 0, grown, stream), "hipMemsetAsync(workspace)");
    ws.bytes = grown;
  }
  return ws.ptr;
}

void run_gemv(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr, std::uintptr_t output_ptr,
              void* workspace, const ArcW4A16Plan& plan, int batch, int n, int k, int group_size,
              int activation_dtype, hipStream_t stream,
              fk::PacketFormat format = fk::PacketFormat::kArc,
              fk::GemvFuse fuse = fk::GemvFuse::kNone, std::uintptr_t norm_weight_ptr = 0,
              float eps = 0.0f) {
  // The kernels index stream-K units (row tile, 32-column slice, group) in 32 bits.
  const long long units_bound = static_cast<long long>(n / 32) * batch * (k / group_size);
  if (units_bound >= (1LL << 31)) {
    throw_invalid("W4A16: batch * (n / 32) * (k / group_size) must stay below 2^31");
  }
  fk::GemvLaunch l;
  l.x = reinterpret_cast<const void*>(activations_ptr);
  l.packets = reinterpret_cast<const void*>(packets_ptr);
  l.out = reinterpret_cast<void*>(output_ptr);
  l.M = batch;
  l.N = n;
  l.K = k;
  l.group_size = group_size;
  l.act = activation_dtype == kActivationBF16 ? fk::Act::kBF16 : fk::Act::kF16;
  l.m_tile = plan.m_tile;
  l.mode = fk::GemvMode::kStreamK;
  l.units_per_workgroup = plan.groups_per_workgroup;
  l.max_contributors = plan.max_tile_contributors;
  l.slice_cols = plan.slice_cols;
  if (plan.schedule == kSchedulePairs) {
    // Native slice pairs: the kernel counts its units in 32-column slices, and every run is a
    // whole pair over all of K.
    if (format == fk::PacketFormat::kArc || plan.m_tile != 1 ||
        plan.slice_cols != 2 * fk::kSliceCols || plan.groups_per_workgroup != k / group_size) {
      throw std::logic_error("slice-pair schedule on a plan that is not one row of whole pairs");
    }
    l.slice_cols = fk::kSliceCols;
    l.slice_pair = true;
    l.units_per_workgroup = 2 * plan.groups_per_workgroup;
  } else if (plan.schedule == kScheduleStream && format == fk::PacketFormat::kArc &&
             plan.m_tile == fk::kMfmaRows) {
    // 2-16 rows over the packets' quarters on the matrix-core stream kernel
    if (batch > fk::kMfmaRows || plan.slice_cols != fk::kSliceCols || plan.stream_half != 0 ||
        fuse != fk::GemvFuse::kNone) {
      throw std::logic_error("matrix-core stream schedule on a reference-packet plan it does not take");
    }
    l.stream = true;
    l.slice_cols = fk::kSliceCols;
    l.ng_magic = fk::arc_quarter_magic(k / group_size);
    l.stream_waves = fk::kStreamWaves;
    l.stream_depth = plan.stream_depth;
    l.stream_grid = plan.workgroups;
    l.stream_whole = plan.stream_whole;
    l.stream_pieces = plan.stream_pieces != 0;
    l.stream_parts = plan.stream_pieces != 0 ? 1 : plan.max_tile_contributors;
  } else if (plan.schedule == kScheduleStream && format == fk::PacketFormat::kArc) {
    if (batch != 1 || plan.m_tile != 1 ||
        (plan.slice_cols != fk::kTileCols && plan.slice_cols != fk::kSliceCols &&
         plan.slice_cols != fk::kSliceCols / 2) ||
        fuse != fk::GemvFuse::kNone) {
      throw std::logic_error("stream schedule on a reference-packet plan it does not take");
    }
    l.stream = true;
    l.slice_cols = plan.slice_cols;
    l.ng_magic = fk::arc_quarter_magic(k / group_size);
    l.stream_depth = plan.stream_depth;
    l.stream_grid = plan.workgroups;
    l.stream_whole = plan.stream_whole;
    l.stream_pieces = plan.stream_pieces != 0;
  } else if (plan.schedule == kScheduleStream) {
    const int cols = plan.stream_half ? fk::kSliceCols / 2 : fk::kSliceCols;
    const bool rows_ok = plan.m_tile == fk::kMfmaRows ? batch <= fk::kMfmaRows : plan.m_tile == batch;
    if (format == fk::PacketFormat::kArc || !rows_ok || plan.slice_cols != cols ||
        (fuse != fk::GemvFuse::kNone && (batch != 1 || plan.stream_pieces || plan.stream_half))) {
      throw std::logic_error("stream schedule on a plan the stream kernel does not take");
    }
    l.stream = true;
    l.slice_cols = fk::kSliceCols;
    l.stream_waves = fk::kStreamWaves;
    l.stream_depth = plan.stream_depth;
    l.stream_grid = plan.workgroups;
    l.stream_whole = plan.stream_whole;
    l.stream_pieces = plan.stream_pieces != 0;
    l.stream_half = plan.stream_half != 0;
    if (plan.m_tile == fk::kMfmaRows && plan.stream_pieces == 0) {
      l.stream_parts = plan.max_tile_contributors;
    }
  }
  l.format = format;
  l.fuse = fuse;
  l.norm_weight = reinterpret_cast<const void*>(norm_weight_ptr);
  l.eps = eps;
  if (plan.workspace_bytes > 0) {
    l.counters = workspace;
    l.partials = static_cast<char*>(workspace) + kCounterRegionBytes;
  }
  check_hip(fk::launch_w4a16_gemv(l, stream), "w4a16_gemv launch");
}

void validate_forward_buffers(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                              std::uintptr_t output_ptr) {
  validate_pointer(activations_ptr, 16, "activations");
  validate_pointer(packets_ptr, 16, "packets");
  validate_pointer(output_ptr, 2, "output");
}

// ---- vendor baseline: dequantised fp16 weight x hipBLASLt --------------------------------

void check_blas(hipblasStatus_t status, const char* what) {
  if (status != HIPBLAS_STATUS_SUCCESS) {
    std::ostringstream oss;
    oss << what << " failed with hipblasStatus " << static_cast<int>(status);
    throw std::runtime_error(oss.str());
  }
}

hipblasLtHandle_t blaslt_handle() {
  static std::array<hipblasLtHandle_t, kMaxDevices> handles{};
  static std::mutex mutex;
  int device = 0;
  check_hip(hipGetDevice(&device), "hipGetDevice");
  std::lock_guard<std::mutex> lock(mutex);
  if (handles[device] == nullptr) {
    check_blas(hipblasLtCreate(&handles[device]), "hipblasLtCreate");
  }
  return handles[device];
}

// Y[M,N] = X[M,K] W[N,K]^T, row-major fp16, fp32 compute. hipBLASLt is column-major, so this is
// issued as Y^T[N,M] = W^T(op T on the [K,N] column-major view of W) x X^T.
void run_blaslt_matmul(const void* activations, const void* weight, void* output, void* workspace,
                       std::size_t workspace_bytes, int batch, int n, int k, hipStream_t stream) {
  hipblasLtHandle_t handle = blaslt_handle();
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a_desc = nullptr, b_desc = nullptr, c_desc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  struct Cleanup {
    hipblasLtMatmulDesc_t& op;
    hipblasLtMatrixLayout_t& a;
    hipblasLtMatrixLayout_t& b;
    hipblasLtMatrixLayout_t& c;
    hipblasLtMatmulPreference_t& p;
    ~Cleanup() {
      if (p) hipblasLtMatmulPreferenceDestroy(p);
      if (c) hipblasLtMatrixLayoutDestroy(c);
      if (b) hipblasLtMatrixLayoutDestroy(b);
      if (a) hipblasLtMatrixLayoutDestroy(a);
      if (op) hipblasLtMatmulDescDestroy(op);
    }
  } cleanup{op, a_desc, b_desc, c_desc, pref};

  const hipblasOperation_t trans_a = HIPBLAS_OP_T;
  const hipblasOperation_t trans_b = HIPBLAS_OP_N;
  check_blas(hipblasLtMatmulDescCreate(&op, HIPBLAS_COMPUTE_32F, HIP_R_32F), "hipblasLtMatmulDescCreate");
  check_blas(hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSA, &trans_a, sizeof(trans_a)),
             "set TRANSA");
  check_blas(hipblasLtMatmulDescSetAttribute(op, HIPBLASLT_MATMUL_DESC_TRANSB, &trans_b, sizeof(trans_b)),
             "set TRANSB");
  check_blas(hipblasLtMatrixLayoutCreate(&a_desc, HIP_R_16F, k, n, k), "layout A");
  check_blas(hipblasLtMatrixLayoutCreate(&b_desc, HIP_R_16F, k, batch, k), "layout B");
  check_blas(hipblasLtMatrixLayoutCreate(&c_desc, HIP_R_16F, n, batch, n), "layout C");
  check_blas(hipblasLtMatmulPreferenceCreate(&pref), "hipblasLtMatmulPreferenceCreate");
  std::uint64_t ws_bytes = workspace == nullptr ? 0 : workspace_bytes;
  check_blas(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                   &ws_bytes, sizeof(ws_bytes)),
             "set max workspace");
  hipblasLtMatmulHeuristicResult_t heuristic{};
  int returned = 0;
  check_blas(hipblasLtMatmulAlgoGetHeuristic(handle, op, a_desc, b_desc, c_desc, c_desc, pref, 1,
                                             &heuristic, &returned),
             "hipblasLtMatmulAlgoGetHeuristic");
  if (returned == 0 && ws_bytes != 0) {
    ws_bytes = 0;
    workspace = nullptr;
    check_blas(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                     &ws_bytes, sizeof(ws_bytes)),
               "set max workspace");
    check_blas(hipblasLtMatmulAlgoGetHeuristic(handle, op, a_desc, b_desc, c_desc, c_desc, pref, 1,
                                               &heuristic, &returned),
               "hipblasLtMatmulAlgoGetHeuristic");
  }
  if (returned == 0) {
    throw std::runtime_error("hipblasLtMatmulAlgoGetHeuristic returned no usable algorithm");
  }
  const float alpha = 1.0f;
  const float beta = 0.0f;
  check_blas(hipblasLtMatmul(handle, op, &alpha, weight, a_desc, activations, b_desc, &beta, output,
                             c_desc, output, c_desc, &heuristic.algo, workspace,
                             static_cast<std::size_t>(ws_bytes), stream),
             "hipblasLtMatmul");
}

}  // namespace

void pack_arc_w4a16_packets(std::uintptr_t q_ptr, std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
                            std::uintptr_t packets_ptr, int n, int k, int group_size,
                            int packet_stride_bytes, std::uintptr_t stream_ptr) {
  validate_dimensions(1, n, k, group_size);
  validate_packet_stride(group_size, packet_stride_bytes);
  validate_pointer(q_ptr, 16, "q");
  validate_pointer(alpha_ptr, 2, "alpha");
  validate_pointer(beta_ptr, 2, "beta");
  validate_pointer(packets_ptr, 16, "packets");
  check_hip(fk::launch_pack_packets(reinterpret_cast<const void*>(q_ptr),
                                    reinterpret_cast<const void*>(alpha_ptr),
                                    reinterpret_cast<const void*>(beta_ptr),
                                    reinterpret_cast<void*>(packets_ptr), n, k, group_size,
                                    reinterpret_cast<hipStream_t>(stream_ptr)),
            "pack_packets launch");
}

void compute_arc_w4a16_group_sums(std::uintptr_t activations_ptr, std::uintptr_t sums_ptr,
                                  int batch, int k, int group_size, std::uintptr_t stream_ptr) {
  validate_group_size_and_k(batch, k, group_size);
  validate_pointer(activations_ptr, 4, "activations");
  validate_pointer(sums_ptr, 4, "sums");
  check_hip(fk::launch_group_sums(reinterpret_cast<const void*>(activations_ptr),
                                  reinterpret_cast<void*>(sums_ptr), batch, k, group_size,
                                  reinterpret_cast<hipStream_t>(stream_ptr)),
            "group_sums launch");
}

// group_sums_ptr is accepted for signature compatibility and not read: the kernel derives the
// per-group activation sums it needs from the activations themselves, in the same launch.
void arc_w4a16_forward(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                       std::uintptr_t group_sums_ptr, std::uintptr_t output_ptr, int batch, int n,
                       int k, int group_size, int packet_stride_bytes, std::uintptr_t stream_ptr) {
  (void)group_sums_ptr;
  validate_dimensions(batch, n, k, group_size);
  validate_packet_stride(group_size, packet_stride_bytes);
  validate_forward_buffers(activations_ptr, packets_ptr, output_ptr);
  const auto stream = reinterpret_cast<hipStream_t>(stream_ptr);
  const ArcW4A16Plan plan =
      plan_arc_w4a16_for_cu_count(batch, n, k, group_size, kActivationF16, 0, device_cu_count());
  void* workspace = plan.workspace_bytes > 0 ? library_workspace(plan.workspace_bytes, stream) : nullptr;
  run_gemv(activations_ptr, packets_ptr, output_ptr, workspace, plan, batch, n, k, group_size,
           kActivationF16, stream);
}

void arc_w4a16_forward_split_k(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                               std::uintptr_t group_sums_ptr, std::uintptr_t partials_ptr,
                               int batch, int n, int k, int group_size, int packet_stride_bytes,
                               int split_k_slices, std::uintptr_t stream_ptr) {
  (void)group_sums_ptr;
  validate_dimensions(batch, n, k, group_size);
  validate_packet_stride(group_size, packet_stride_bytes);
  if (split_k_slices <= 1) {
    throw_invalid("split_k_slices must be greater than 1");
  }
  const int num_groups = k / group_size;
  if (split_k_slices > num_groups) {
    throw_invalid("split_k_slices must not exceed the number of groups");
  }
  validate_pointer(activations_ptr, 16, "activations");
  validate_pointer(packets_ptr, 16, "packets");
  validate_pointer(partials_ptr, 4, "partials");
  // Slice z covers groups [z*gps, (z+1)*gps) with gps = ceil(NG / S), as in the reference
  // (arc_w4a16.cu:341-386, 463). A slice past the end writes zeros instead of leaving its
  // partials unwritten.
  fk::GemvLaunch l;
  l.x = reinterpret_cast<const void*>(activations_ptr);
  l.packets = reinterpret_cast<const void*>(packets_ptr);
  l.partials = reinterpret_cast<void*>(partials_ptr);
  l.M = batch;
  l.N = n;
  l.K = k;
  l.group_size = group_size;
  l.act = fk::Act::kF16;
  l.mode = fk::GemvMode::kPartials;
  l.m_tile = fk::gemv_partials_m_tile_for_batch(batch);
  l.splits = split_k_slices;
  l.gps = (num_groups + split_k_slices - 1) / split_k_slices;
  check_hip(fk::launch_w4a16_gemv(l, reinterpret_cast<hipStream_t>(stream_ptr)),
            "w4a16_gemv split-K launch");
}

void reduce_arc_w4a16_split_k_partials(std::uintptr_t partials_ptr, std::uintptr_t output_ptr,
                                       int batch, int n, int split_k_slices,
                                       std::uintptr_t stream_ptr) {
  if (batch <= 0 || n <= 0 || split_k_slices <= 1) {
    throw_invalid("batch, n, and split_k_slices must be positive with split_k_slices > 1");
  }
  validate_pointer(partials_ptr, 4, "partials");
  validate_pointer(output_ptr, 2, "output");
  check_hip(fk::launch_reduce_partials(reinterpret_cast<const void*>(partials_ptr),
                                       reinterpret_cast<void*>(output_ptr), batch, n,
                                       split_k_slices, reinterpret_cast<hipStream_t>(stream_ptr)),
            "reduce_partials launch");
}

void dequant_w4a16_to_fp16(std::uintptr_t q_ptr, std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
                           std::uintptr_t output_ptr, int n, int k, int group_size,
                           std::uintptr_t stream_ptr) {
  validate_dimensions(1, n, k, group_size);
  validate_pointer(q_ptr, 4, "q");
  validate_pointer(alpha_ptr, 2, "alpha");
  validate_pointer(beta_ptr, 2, "beta");
  validate_pointer(output_ptr, 16, "output");
  check_hip(fk::launch_dequant(reinterpret_cast<const void*>(q_ptr),
                               reinterpret_cast<const void*>(alpha_ptr),
                               reinterpret_cast<const void*>(beta_ptr),
                               reinterpret_cast<void*>(output_ptr), n, k, group_size,
                               reinterpret_cast<hipStream_t>(stream_ptr)),
            "dequant launch");
}

void dequant_arc_w4a16_packets_to_fp16(std::uintptr_t packets_ptr, std::uintptr_t output_ptr, int n,
                                       int k, int group_size, int packet_stride_bytes,
                                       std::uintptr_t stream_ptr) {
  validate_dimensions(1, n, k, group_size);
  validate_packet_stride(group_size, packet_stride_bytes);
  validate_pointer(packets_ptr, 16, "packets");
  validate_pointer(output_ptr, 16, "output");
  check_hip(fk::launch_dequant_packets(reinterpret_cast<const void*>(packets_ptr),
                                       reinterpret_cast<void*>(output_ptr), n, k, group_size,
                                       reinterpret_cast<hipStream_t>(stream_ptr)),
            "dequant_packets launch");
}

void cublaslt_fp16_with_weight(std::uintptr_t activations_ptr, std::uintptr_t weight_ptr,
                               std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                               std::size_t workspace_bytes, int batch, int n, int k,
                               std::uintptr_t stream_ptr) {
  if (batch <= 0 || n <= 0 || k <= 0) {
    throw_invalid("batch, n, and k must be positive");
  }
  validate_pointer(activations_ptr, 2, "activations");
  validate_pointer(weight_ptr, 2, "weight");
  validate_pointer(output_ptr, 2, "output");
  run_blaslt_matmul(reinterpret_cast<const void*>(activations_ptr),
                    reinterpret_cast<const void*>(weight_ptr), reinterpret_cast<void*>(output_ptr),
                    reinterpret_cast<void*>(workspace_ptr), workspace_bytes, batch, n, k,
                    reinterpret_cast<hipStream_t>(stream_ptr));
}

void cublaslt_fp16_after_packet_dequant(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                                        std::uintptr_t output_ptr, std::uintptr_t weight_ptr,
                                        std::uintptr_t workspace_ptr, std::size_t workspace_bytes,
                                        int batch, int n, int k, int group_size,
                                        int packet_stride_bytes, std::uintptr_t stream_ptr) {
  validate_dimensions(batch, n, k, group_size);
  validate_packet_stride(group_size, packet_stride_bytes);
  dequant_arc_w4a16_packets_to_fp16(packets_ptr, weight_ptr, n, k, group_size, packet_stride_bytes,
                                    stream_ptr);
  cublaslt_fp16_with_weight(activations_ptr, weight_ptr, output_ptr, workspace_ptr, workspace_bytes,
                            batch, n, k, stream_ptr);
}

void cublaslt_fp16_after_dequant(std::uintptr_t activations_ptr, std::uintptr_t q_ptr,
                                 std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
                                 std::uintptr_t output_ptr, std::uintptr_t weight_ptr,
                                 std::uintptr_t workspace_ptr, std::size_t workspace_bytes,
                                 int batch, int n, int k, int group_size,
                                 std::uintptr_t stream_ptr) {
  validate_dimensions(batch, n, k, group_size);
  dequant_w4a16_to_fp16(q_ptr, alpha_ptr, beta_ptr, weight_ptr, n, k, group_size, stream_ptr);
  cublaslt_fp16_with_weight(activations_ptr, weight_ptr, output_ptr, workspace_ptr, workspace_bytes,
                            batch, n, k, stream_ptr);
}

ArcW4A16Plan plan_arc_w4a16(int batch, int n, int k, int group_size, int activation_dtype,
                            int split_k_slices) {
  validate_dimensions(batch, n, k, group_size);
  return plan_arc_w4a16_for_cu_count(batch, n, k, group_size, activation_dtype, split_k_slices,
                                     device_cu_count());
}

namespace {

void forward_with_format(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                         std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                         std::size_t workspace_bytes, int batch, int n, int k, int group_size,
                         fk::PacketFormat format, int activation_dtype, int split_k_slices,
                         std::uintptr_t stream_ptr, int kernel = kKernelAuto) {
  validate_activation_dtype(activation_dtype);
  validate_forward_buffers(activations_ptr, packets_ptr, output_ptr);
  if (split_k_slices < 0) {
    throw_invalid("split_k_slices must be >= 0 (0 = automatic)");
  }
  const ArcW4A16Plan plan =
      plan_w4a16_for_kernel(batch, n, k, group_size, activation_dtype, split_k_slices,
                            device_cu_count(), static_cast<int>(format), kernel);
  if (plan.workspace_bytes > 0) {
    validate_pointer(workspace_ptr, kCounterRegionAlign, "workspace");
    if (workspace_bytes < plan.workspace_bytes) {
      std::ostringstream oss;
      oss << "workspace_bytes=" << workspace_bytes << " is smaller than the " << plan.workspace_bytes
          << " bytes this launch needs";
      throw_invalid(oss.str());
    }
  }
  run_gemv(activations_ptr, packets_ptr, output_ptr, reinterpret_cast<void*>(workspace_ptr), plan,
           batch, n, k, group_size, activation_dtype, reinterpret_cast<hipStream_t>(stream_ptr),
           format);
}

// One uint32 flag per device for arc -> native conversions, allocated on first use.
void* conversion_flag() {
  static std::array<void*, kMaxDevices> flags{};
  static std::mutex mutex;
  int device = 0;
  check_hip(hipGetDevice(&device), "hipGetDevice");
  std::lock_guard<std::mutex> lock(mutex);
  if (flags[device] == nullptr) {
    check_hip(hipMalloc(&flags[device], sizeof(std::uint32_t)), "hipMalloc(flag)");
  }
  return flags[device];
}

}  // namespace

void arc_w4a16_forward_ex(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                          std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                          std::size_t workspace_bytes, int batch, int n, int k, int group_size,
                          int packet_stride_bytes, int activation_dtype, int split_k_slices,
                          std::uintptr_t stream_ptr) {
  validate_dimensions(batch, n, k, group_size);
  validate_packet_stride(group_size, packet_stride_bytes);
  forward_with_format(activations_ptr, packets_ptr, output_ptr, workspace_ptr, workspace_bytes,
                      batch, n, k, group_size, fk::PacketFormat::kArc, activation_dtype,
                      split_k_slices, stream_ptr);
}

int packet_format_stride_bytes(int group_size, int packet_format) {
  if (group_size != 64 && group_size != 128) {
    throw_invalid("group_size must be 64 or 128");
  }
  return fk::format_packet_stride(group_size, to_packet_format(packet_format, true));
}

void pack_native_w4a16_packets(std::uintptr_t q_ptr, std::uintptr_t alpha_ptr,
                               std::uintptr_t zero_points_ptr, std::uintptr_t packets_ptr, int n,
                               int k, int group_size, int packet_format, std::uintptr_t stream_ptr) {
  validate_dimensions(1, n, k, group_size);
  const fk::PacketFormat format = to_packet_format(packet_format, false);
  validate_pointer(q_ptr, 16, "q");
  validate_pointer(alpha_ptr, 2, "alpha");
  validate_pointer(packets_ptr, 16, "packets");
  if (format == fk::PacketFormat::kNativeAsym) {
    validate_pointer(zero_points_ptr, 1, "zero_points");
  }
  check_hip(fk::launch_pack_native(reinterpret_cast<const void*>(q_ptr),
                                   reinterpret_cast<const void*>(alpha_ptr),
                                   reinterpret_cast<const void*>(zero_points_ptr),
                                   reinterpret_cast<void*>(packets_ptr), n, k, group_size, format,
                                   reinterpret_cast<hipStream_t>(stream_ptr)),
            "pack_native launch");
}

void convert_arc_w4a16_packets_to_native(std::uintptr_t arc_packets_ptr,
                                         std::uintptr_t native_packets_ptr, int n, int k,
                                         int group_size, int packet_format,
                                         std::uintptr_t stream_ptr) {
  validate_dimensions(1, n, k, group_size);
  const fk::PacketFormat format = to_packet_format(packet_format, false);
  validate_pointer(arc_packets_ptr, 16, "arc_packets");
  validate_pointer(native_packets_ptr, 16, "native_packets");
  const auto stream = reinterpret_cast<hipStream_t>(stream_ptr);
  void* flag = conversion_flag();
  check_hip(hipMemsetAsync(flag, 0, sizeof(std::uint32_t), stream), "hipMemsetAsync(flag)");
  check_hip(fk::launch_arc_to_native(reinterpret_cast<const void*>(arc_packets_ptr),
                                     reinterpret_cast<void*>(native_packets_ptr), n, k, group_size,
                                     format, flag, stream),
            "arc_to_native launch");
  std::uint32_t bad = 0;
  check_hip(hipMemcpyAsync(&bad, flag, sizeof(bad), hipMemcpyDeviceToHost, stream),
            "hipMemcpyAsync(flag)");
  check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
  if (bad != 0) {
    throw_invalid(format == fk::PacketFormat::kNativeSym
                      ? "packets are not symmetric: some beta is not half_rn(-8 * alpha)"
                      : "packets are not affine int4: some beta is not half_rn(-alpha * zp) for "
                        "an integer zero point 0..15");
  }
}

void convert_native_w4a16_packets_to_arc(std::uintptr_t native_packets_ptr,
                                         std::uintptr_t arc_packets_ptr, int n, int k,
                                         int group_size, int packet_format,
                                         std::uintptr_t stream_ptr) {
  validate_dimensions(1, n, k, group_size);
  const fk::PacketFormat format = to_packet_format(packet_format, false);
  validate_pointer(native_packets_ptr, 16, "native_packets");
  validate_pointer(arc_packets_ptr, 16, "arc_packets");
  check_hip(fk::launch_native_to_arc(reinterpret_cast<const void*>(native_packets_ptr),
                                     reinterpret_cast<void*>(arc_packets_ptr), n, k, group_size,
                                     format, reinterpret_cast<hipStream_t>(stream_ptr)),
            "native_to_arc launch");
}

void arc_w4a16_forward_native(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                              std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                              std::size_t workspace_bytes, int batch, int n, int k, int group_size,
                              int packet_format, int activation_dtype, int split_k_slices,
                              std::uintptr_t stream_ptr) {
  validate_dimensions(batch, n, k, group_size);
  forward_with_format(activations_ptr, packets_ptr, output_ptr, workspace_ptr, workspace_bytes,
                      batch, n, k, group_size, to_packet_format(packet_format, true),
                      activation_dtype, split_k_slices, stream_ptr);
}

void w4a16_forward_kernel(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                          std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                          std::size_t workspace_bytes, int batch, int n, int k, int group_size,
                          int packet_format, int activation_dtype, int split_k_slices, int kernel,
                          std::uintptr_t stream_ptr) {
  validate_dimensions(batch, n, k, group_size);
  m_tile_for_kernel(batch, kernel);  // validates the choice before any pointer check
  forward_with_format(activations_ptr, packets_ptr, output_ptr, workspace_ptr, workspace_bytes,
                      batch, n, k, group_size, to_packet_format(packet_format, true),
                      activation_dtype, split_k_slices, stream_ptr, kernel);
}

void w4a16_forward_noalloc(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                           std::uintptr_t output_ptr, int batch, int n, int k, int group_size,
                           int packet_format, int activation_dtype, std::uintptr_t stream_ptr) {
  validate_dimensions(batch, n, k, group_size);
  const fk::PacketFormat format = to_packet_format(packet_format, true);
  validate_activation_dtype(activation_dtype);
  validate_forward_buffers(activations_ptr, packets_ptr, output_ptr);
  const auto stream = reinterpret_cast<hipStream_t>(stream_ptr);
  // The plan of arc_w4a16_forward_native, checked against the scratch size before any device
  // work; then the set-up on the first call on a device (address lookup, counter clear), and the
  // launch with the scratch array standing in for the workspace.
  const ArcW4A16Plan plan = plan_w4a16_for_kernel(batch, n, k, group_size, activation_dtype, 0,
                                                  device_cu_count(), packet_format, kKernelAuto);
  if (plan.workspace_bytes > kNoAllocScratchBytes) {
    std::ostringstream oss;
    oss << "this launch needs " << plan.workspace_bytes << " bytes of fix-up scratch; the "
        << "no-allocation entry point holds " << kNoAllocScratchBytes << " per device";
    throw_invalid(oss.str());
  }
  if (plan.workspace_bytes > 0) {
    noalloc_claim_stream(stream);
  }
  void* scratch = noalloc_scratch(kCounterRegionBytes, stream);
  run_gemv(activations_ptr, packets_ptr, output_ptr, scratch, plan, batch, n, k, group_size,
           activation_dtype, stream, format);
}

void arc_w4a16_forward_rmsnorm(std::uintptr_t activations_ptr, std::uintptr_t norm_weight_ptr,
                               float eps, std::uintptr_t packets_ptr, std::uintptr_t output_ptr,
                               std::uintptr_t workspace_ptr, std::size_t workspace_bytes, int batch,
                               int n, int k, int group_size, int packet_format,
                               int activation_dtype, int split_k_slices, std::uintptr_t stream_ptr) {
  validate_dimensions(batch, n, k, group_size);
  const fk::PacketFormat format = to_packet_format(packet_format, false);
  validate_activation_dtype(activation_dtype);
  validate_forward_buffers(activations_ptr, packets_ptr, output_ptr);
  validate_pointer(norm_weight_ptr, 16, "norm_weight");
  if (!(eps >= 0.0f)) {
    throw_invalid("eps must be >= 0");
  }
  if (split_k_slices < 0) {
    throw_invalid("split_k_slices must be >= 0 (0 = automatic)");
  }
  const ArcW4A16Plan plan = plan_w4a16_rmsnorm(batch, n, k, group_size, activation_dtype,
                                               split_k_slices, 0, packet_format);
  if (plan.workspace_bytes > 0) {
    validate_pointer(workspace_ptr, kCounterRegionAlign, "workspace");
    if (workspace_bytes < plan.workspace_bytes) {
      std::ostringstream oss;
      oss << "workspace_bytes=" << workspace_bytes << " is smaller than the " << plan.workspace_bytes
          << " bytes this launch needs";
      throw_invalid(oss.str());
    }
  }
  run_gemv(activations_ptr, packets_ptr, output_ptr, reinterpret_cast<void*>(workspace_ptr), plan,
           batch, n, k, group_size, activation_dtype, reinterpret_cast<hipStream_t>(stream_ptr),
           format, fk::GemvFuse::kRmsNorm, norm_weight_ptr, eps);
}

ArcW4A16Plan plan_w4a16_rmsnorm(int batch, int n, int k, int group_size, int activation_dtype,
                                int split_k_slices, int cu_count, int packet_format) {
  to_packet_format(packet_format, false);
  ArcW4A16Plan plan{};
  if (split_k_slices == 0 &&
      fused_stream_plan(plan, batch, n, k, group_size, /*silu=*/false, cu_count)) {
    return plan;
  }
  return plan_for_format_impl(batch, n, k, group_size, activation_dtype, split_k_slices, cu_count,
                              packet_format, kKernelDot2, /*plain=*/false);
}

void arc_w4a16_forward_silu_mul(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                                std::uintptr_t output_ptr, int batch, int n, int k, int group_size,
                                int packet_format, int activation_dtype,
                                std::uintptr_t stream_ptr, std::uintptr_t norm_weight_ptr,
                                float eps) {
  validate_dimensions(batch, n, k, group_size);
  if (n % (2 * fk::kTileCols) != 0) {
    throw_invalid("n (gate and up rows together) must be divisible by 256");
  }
  const fk::PacketFormat format = to_packet_format(packet_format, false);
  validate_activation_dtype(activation_dtype);
  validate_forward_buffers(activations_ptr, packets_ptr, output_ptr);
  const bool norm = norm_weight_ptr != 0;
  if (norm && !(eps >= 0.0f)) {
    throw_invalid("eps must be >= 0");
  }
  if (norm) {
    validate_pointer(norm_weight_ptr, 16, "norm_weight");
  }
  // One row: the stream kernel over whole (gate slice, up slice) pairs where they divide over the
  // CUs (fused_stream_plan). Otherwise one workgroup per pair over all of K. No fix-up, no
  // workspace either way.
  ArcW4A16Plan plan{};
  if (!fused_stream_plan(plan, batch, n, k, group_size, /*silu=*/true, 0)) {
    plan.m_tile = fk::gemv_partials_m_tile_for_batch(batch);
    plan.slice_cols = fk::kSliceCols;
    plan.groups_per_workgroup = k / group_size;
    plan.max_tile_contributors = 1;
    plan.workspace_bytes = 0;
  }
  run_gemv(activations_ptr, packets_ptr, output_ptr, nullptr, plan, batch, n, k, group_size,
           activation_dtype, reinterpret_cast<hipStream_t>(stream_ptr), format,
           norm ? fk::GemvFuse::kRmsNormSiluMul : fk::GemvFuse::kSiluMul, norm_weight_ptr, eps);
}

}  // namespace fast_kernels::decode_quant_linear
