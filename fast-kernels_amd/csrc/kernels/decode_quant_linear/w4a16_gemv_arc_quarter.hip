// W4A16 GEMV over the reference packets for one activation row, by 32-column quarters of the
// packets, on the persistent stream schedule of the native-slab kernel (w4a16_gemv_stream.hip).
//
// The drop-in entry points (fk_arc_w4a16_forward*, arc_w4a16.cu:687-707) take the reference
// packet: per 128-column tile and group, G/8 word rows of 512 bytes (word w of column c at byte
// 4 (128 w + c)), then 128 fp16 alphas and 128 fp16 betas, the groups of a tile consecutive. This
// kernel's unit is the quarter (32 columns, "slice" s = 4 tile + q) of one packet: the 128 bytes
// of columns 32 q .. 32 q + 31 in each word row and their 64 bytes of alphas and of betas. Measured
// on MI355X, streaming reads alone (graph launches, 70B layer shapes): quarters of packets,
// 128-byte runs at a 512-byte stride, stream at 6.5 TB/s (gate_up's 249.6 MB in 38.3 us, o's
// 35.7 MB in 7.2 us), so the drop-in format runs on the native kernel's schedule with no
// conversion:
//
//  * slices are dealt as in the native stream kernel (w4a16_stream_common.h): stream_whole whole
//    slices per workgroup, one workgroup per CU, plus with kPieces the left-over slices as equal
//    block ranges handed off through the workspace by a control wave;
//  * wave w takes groups w, w + 8, .. of its slices (D units in flight, 4 KB of codes per wave);
//    lane l reads word rows R (l / 8) .. R (l / 8) + R - 1 (R = G / 64) of the columns
//    32 q + 4 (l % 8) .. + 3, 16 bytes per word row, and the alphas (l / 8 even) or the betas
//    (odd) of those columns, the other half coming from lane l ^ 8 by DPP;
//  * each wave stages its own groups' activations in LDS, re-paired, with per-(group, row group)
//    sums {-1024 S_even - 64 S_odd, S_even + S_odd} (the accumulator seed and the beta term), and
//    per group the bf16 staging scale; the first pass before the first block, one more after each
//    block (all of them first with pieces);
//  * math per word: the (1024 + q) / (64 + q) unpack and v_dot2 into fp32 seeded with the group's
//    offset term, then y += alpha * acc + beta * S: the reference-packet kernel's
//    (w4a16_gemv_kernels.h), beta any fp16;
//  * at the end of a slice the eight row groups of a column (lanes l, l ^ 8, l ^ 16, l ^ 32) are
//    added, the wave's 32 totals go to an LDS ring slot, and every four slices (and after the
//    last) a barrier lets the workgroup add the waves' totals in wave order and write them.
//
// kCols = 16 (G = 128, no pieces, short K): the unit is a packet's 16-column eighth (64-byte runs
// at the 512-byte stride), so that shapes with at most half as many quarters as CUs use every CU
// (7B and 8B o: 256 eighths). Lane l then reads word row l / 4, columns 16 e + 4 (l % 4) .. + 3;
// the 16 row groups alternate alphas and betas (the partner by DPP row_ror:4), and the fold adds
// lanes l ^ 4 .. l ^ 32.
//
// The slice of a unit comes from its linear (slice, group) index by a multiply-high with a
// reciprocal of K / G (GemvParams::ng_magic, exact over the launch's indices: see
// arc_quarter_magic_exact), no division in the loop.
#include "w4a16_gemv_native.h"
#include "w4a16_stream_common.h"

#include <type_traits>

namespace fk {
namespace {

constexpr int kQuarterWaves = 8;

// Unit geometry for kCols = 32 (a packet quarter) or 16 (an eighth, G = 128): kCols / 4 lanes
// cover a word row's kCols columns (16 bytes each), so a wave covers 64 / (kCols / 4) row groups
// of R word rows.
template <int G, int kCols>
struct QuarterGeom {
  static constexpr int kLanesPerRow = kCols / 4;
  static constexpr int kRowGroups = 64 / kLanesPerRow;
  static constexpr int kRows = (G / 8) / kRowGroups;  // word rows of the lane
  static_assert(kRows >= 1, "one word row per lane at least");
};

template <int G, int kCols>
struct QuarterUnit {
  static constexpr int kRows = QuarterGeom<G, kCols>::kRows;
  uint4 w[kRows];  // word rows R rg + k, columns 4 (l % (kCols / 4)) .. + 3 of the unit
  uint2 ab;  // the lane's four columns' alphas (row group even) or betas (odd); a lane of the
             // other parity and the same columns holds the other
};

// LDS: xs [(NG + 1) * G/8] re-paired words (group-major), sums [(NG + 1) * row groups] {seed, S}
// per (group, row group), scale [NG + 1] bf16 staging scales per group.
template <int G>
struct QuarterLds {
  uint4* xs;
  float2* sums;
  float* scale;
};

template <int G, int kCols>
__host__ __device__ constexpr size_t quarter_lds_bytes(int ng) {
  return static_cast<size_t>(ng + 1) *
         ((G / 8) * 16 + QuarterGeom<G, kCols>::kRowGroups * 8 + 4);
}

template <int G, Act A, int kStageSlots, bool kPieces, int kCols>
__global__ void __launch_bounds__(64 * (kQuarterWaves + (kPieces ? 1 : 0)), 1)
    w4a16_gemv_arc_quarter_kernel(GemvParams p) {
  constexpr int kW = kQuarterWaves;
  constexpr int D = G == 128 ? 2 : 4;  // units in flight per wave (4 KB of codes at kCols = 32)
  using Geom = QuarterGeom<G, kCols>;
  constexpr int R = Geom::kRows;
  constexpr int kLpr = Geom::kLanesPerRow;
  constexpr int kRg = Geom::kRowGroups;
  constexpr int kUnitsPerTile = kTileCols / kCols;
  constexpr int WR = G / 8;
  constexpr int Q = kW * D;  // groups per block
  constexpr int kRing = 4;
  extern __shared__ uint4 quarter_lds[];
  // Wave totals: slots 0 and 1 for the pieces, then two rounds of kRing whole slices.
  __shared__ float red[2 + 2 * kRing][kW][kCols];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg8 = lane / kLpr;  // the lane's row group
  const int c8 = lane % kLpr;   // the lane's columns 4 c8 .. 4 c8 + 3 of the unit
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, PacketFormat::kArc));
  const int grid = p.grid;
  int b = static_cast<int>(blockIdx.x);
  b = p.xcd_remap != 0 ? (b & 7) * p.xcd_remap + (b >> 3) : b;
  const int ng = p.NG;
  const int nbs = ng / Q;  // blocks per slice
  const int slices = p.N / kCols;  // units
  constexpr int kOut = kCols;

  if constexpr (kPieces) {
    if (wave == kW) {
      // Control wave: the pieces' totals (a barrier each), their hand-offs, then the whole
      // slices' barriers.
      const StreamRange rg = stream_range(b, grid, p.stream_whole, slices, nbs, true);
      float v[2][1];
      int slot = 0;
      const bool has[2] = {rg.head_len > 0, rg.tail_len > 0};
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        if (has[pc]) {
          lds_barrier();
          float s = 0.0f;
          if (lane < kOut) {
#pragma unroll
            for (int w = 0; w < kW; ++w) {
              s += red[slot][w][lane];
            }
          }
          v[pc][0] = s;
          slot ^= 1;
        }
      }
      if (has[0]) {
        stream_hand_off<A, 1>(p, b, 0, rg.head_slice, grid, p.stream_whole, slices, nbs, kOut,
                              kOut, v[0], lane);
      }
      if (has[1]) {
        stream_hand_off<A, 1>(p, b, 1, rg.tail_slice, grid, p.stream_whole, slices, nbs, kOut,
                              kOut, v[1], lane);
      }
      for (int r = 0; r < (rg.whole + kRing - 1) / kRing; ++r) {
        lds_barrier();
      }
      return;
    }
  }

  // Activations: every pass's loads first. Pass i stages word row l % WR of group
  // wave + kW (i * 64 / WR + l / WR).
  constexpr int kGroupsPerPass = 64 / WR;
  const int n_pass = (nbs * D + kGroupsPerPass - 1) / kGroupsPerPass;
  uint4 raw[kStageSlots];
#pragma unroll
  for (int i = 0; i < kStageSlots; ++i) {
    const int g = min(wave + kW * (i * kGroupsPerPass + lane / WR), ng - 1);
    raw[i] = *reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(g) * G + (lane % WR) * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  const StreamRange rg = stream_range(b, grid, p.stream_whole, slices, nbs, kPieces);

  QuarterLds<G> sm;
  sm.xs = quarter_lds;
  sm.sums = reinterpret_cast<float2*>(sm.xs + static_cast<size_t>(ng + 1) * WR);
  sm.scale = reinterpret_cast<float*>(sm.sums + static_cast<size_t>(ng + 1) * kRg);

  // The wave's units, in order: the head piece's, the tail piece's, then the whole slices' (as
  // in the native stream kernel, linear index slice * NG + group). Past its last unit a wave
  // re-reads it, so every load is unconditional and inside the buffer.
  const int n_h = rg.head_len * D;
  const int n_t = rg.tail_len * D;
  const int n_w = n_h + n_t + rg.whole * nbs * D;
  const int j_last = n_w - 1;
  const int off_w = rg.whole_slice0 * ng + wave - (n_h + n_t) * kW;
  const int off_t = rg.tail_slice * ng + wave - n_h * kW;
  const int off_h = rg.head_slice * ng + rg.head_blk0 * Q + wave;
  const uint32_t magic = p.ng_magic;
  const int lane_off = R * rg8 * kWordRowBytes + c8 * 16;
  const int scale_off = kTileCols * G / 2 + (rg8 & 1) * (kTileCols * 2) + c8 * 8;
  const bool has_alpha = (rg8 & 1) == 0;
  auto load_unit = [&](QuarterUnit<G, kCols>& u, int i) __attribute__((always_inline)) {
    const int c = min(i, j_last);
    int off = off_w;
    if constexpr (kPieces) {
      // 0/1 flags made opaque to the compiler (readfirstlane), which otherwise turns the choice
      // into a lookup table in scratch memory
      int in_t = c < n_h + n_t ? 1 : 0;
      int in_h = c < n_h ? 1 : 0;
      in_t = __builtin_amdgcn_readfirstlane(in_t);
      in_h = __builtin_amdgcn_readfirstlane(in_h);
      off += in_t * (off_t - off_w) + in_h * (off_h - off_t);
    }
    const uint32_t lin = static_cast<uint32_t>(c * kW + off);
    const uint32_t s = __umulhi(lin, magic);
    const uint32_t g = lin - s * static_cast<uint32_t>(ng);
    const uint32_t pkt = (s / kUnitsPerTile) * static_cast<uint32_t>(ng) + g;
    const uint8_t* pk = p.packets + static_cast<size_t>(pkt) * stride;
    const uint8_t* codes = pk + (s % kUnitsPerTile) * (kCols * 4) + lane_off;
#pragma unroll
    for (int k = 0; k < R; ++k) {
      u.w[k] = stream_load16(codes + k * kWordRowBytes);
    }
    // one 8-byte load per lane for the scales: alphas on even row groups, betas on odd ones
    u.ab = stream_load8(pk + scale_off + (s % kUnitsPerTile) * (kCols * 2));
  };

  QuarterUnit<G, kCols> buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_unit(buf[d], d);
    __builtin_amdgcn_sched_barrier(0);  // the same issue order as the refills in the loop
  }

  int staged = 0;
  // Stages the next pass from raw[0] and shifts the slots down (register moves; a runtime slot
  // index would put them in scratch memory). Groups past the row go to the spare slot NG.
  auto stage_one = [&]() {
    const int g = min(wave + kW * (staged * kGroupsPerPass + lane / WR), ng);
    const int w = lane % WR;
    uint4 r = raw[0];
    float undo = 1.0f;
    if constexpr (A == Act::kBF16) {
      const uint32_t e = group_max<WR>(bf16_max_mag(r)) >> 7;
      const int shift = bf16_stage_shift(e);
      const float sc = __builtin_bit_cast(float, static_cast<uint32_t>(127 - shift) << 23);
      undo = __builtin_bit_cast(float, static_cast<uint32_t>(127 + shift) << 23);
      r.x = bf16_pair_to_half_pair(r.x, sc);
      r.y = bf16_pair_to_half_pair(r.y, sc);
      r.z = bf16_pair_to_half_pair(r.z, sc);
      r.w = bf16_pair_to_half_pair(r.w, sc);
    }
    const uint4 xp = pair_activations(r);
    constexpr uint32_t kOnes = 0x3c003c00u;
    float se = dot2<Act::kF16>(xp.z, kOnes, dot2<Act::kF16>(xp.x, kOnes, 0.0f));
    float so = dot2<Act::kF16>(xp.w, kOnes, dot2<Act::kF16>(xp.y, kOnes, 0.0f));
    if constexpr (R > 1) {
      se = group_sum<R>(se);
      so = group_sum<R>(so);
    }
    sm.xs[static_cast<size_t>(g) * WR + w] = xp;
    // every lane of a row group holds the same values and writes them (no branch)
    sm.sums[static_cast<size_t>(g) * kRg + w / R] =
        make_float2(fmaf(-1024.0f, se, -64.0f * so), se + so);
    sm.scale[g] = undo;
#pragma unroll
    for (int i = 0; i + 1 < kStageSlots; ++i) {
      raw[i] = raw[i + 1];
    }
    ++staged;
    // The wave reads back only what it wrote (its LDS accesses complete in order); the fences
    // (no instruction) keep the compiler from hoisting the reads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  stage_one();
  if constexpr (kPieces) {
    while (staged < n_pass) {
      stage_one();
    }
  }

  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // A unit in two steps. Unpacked: its code words as the (1024 + q) / (64 + q) fp16 pairs and
  // its scales as floats, which frees the load buffer for the refill; then the arithmetic of
  // slice-local group g against the staged row.
  struct Unpacked {
    uint32_t e0[R][4], o0[R][4], e1[R][4], o1[R][4];
    float a[4], bt[4];
  };
  auto unpack = [&](const QuarterUnit<G, kCols>& u, Unpacked& up) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const uint32_t words[4] = {u.w[k].x, u.w[k].y, u.w[k].z, u.w[k].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wv = words[j];
        const uint32_t w8 = wv >> 8;
        up.e0[k][j] = (wv & mask_lo) | kBiasLow;   // 1024 + q: k0, k4
        up.o0[k][j] = (wv & mask_hi) | kBiasHigh;  // 64 + q: k1, k5
        up.e1[k][j] = (w8 & mask_lo) | kBiasLow;   // k2, k6
        up.o1[k][j] = (w8 & mask_hi) | kBiasHigh;  // k3, k7
      }
    }
    // the lane kLpr further in its 16-lane row (the other row-group parity, same columns) holds
    // the other half: DPP row_ror:kLpr
    const uint32_t ox = __builtin_amdgcn_mov_dpp(u.ab.x, 0x120 + kLpr, 0xf, 0xf, true);
    const uint32_t oy = __builtin_amdgcn_mov_dpp(u.ab.y, 0x120 + kLpr, 0xf, 0xf, true);
    const uint32_t ax = has_alpha ? u.ab.x : ox;
    const uint32_t ay = has_alpha ? u.ab.y : oy;
    const uint32_t bx = has_alpha ? ox : u.ab.x;
    const uint32_t by = has_alpha ? oy : u.ab.y;
    const uint32_t ab[4] = {ax, ax >> 16, ay, ay >> 16};
    const uint32_t bb[4] = {bx, bx >> 16, by, by >> 16};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      up.a[j] = half_bits_to_float(static_cast<uint16_t>(ab[j]));
      up.bt[j] = half_bits_to_float(static_cast<uint16_t>(bb[j]));
    }
  };
  auto compute = [&](const Unpacked& up, int g) __attribute__((always_inline)) {
    const float2 sp = sm.sums[static_cast<size_t>(g) * kRg + rg8];
    float acc[4][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[j][0] = sp.x;
      acc[j][1] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const uint4 xp = sm.xs[static_cast<size_t>(g) * WR + R * rg8 + k];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[j][0] = dot2<Act::kF16>(up.e0[k][j], xp.x, acc[j][0]);
        acc[j][1] = dot2<Act::kF16>(up.o0[k][j], xp.y, acc[j][1]);
        acc[j][0] = dot2<Act::kF16>(up.e1[k][j], xp.z, acc[j][0]);
        acc[j][1] = dot2<Act::kF16>(up.o1[k][j], xp.w, acc[j][1]);
      }
    }
    const float scale = A == Act::kBF16 ? sm.scale[g] : 1.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sum = acc[j][0] + acc[j][1];
      if constexpr (A == Act::kBF16) {
        y[j] = fmaf(fmaf(up.bt[j], sp.y, up.a[j] * sum), scale, y[j]);
      } else {
        y[j] = fmaf(up.bt[j], sp.y, fmaf(up.a[j], sum, y[j]));
      }
    }
  };
  int j = 0;  // the wave's next unit
  // A block of D units of slice-local groups gl0 + kW d; refill = false on the wave's last block
  // (its refills would only re-read its last unit and hold the wave one memory latency longer).
  // Each unit is unpacked out of its buffer before the refill is issued into it, so the load goes
  // out ahead of the unit's arithmetic (computing from the buffer kept the betas, which feed the
  // last fma, live to the end of the unit and the refill behind all of it).
  auto block_r = [&](int gl0, auto refill) __attribute__((always_inline)) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      Unpacked up;
      unpack(buf[d], up);
      if constexpr (decltype(refill)::value) {
        __builtin_amdgcn_sched_barrier(0);
        load_unit(buf[d], j + d + D);
        __builtin_amdgcn_sched_barrier(0);
      }
      compute(up, gl0 + kW * d);
      __builtin_amdgcn_sched_barrier(0);
    }
    j += D;
  };
  auto block = [&](int gl0) { block_r(gl0, std::true_type{}); };
  // The row groups of each column added, then the wave's kCols totals into LDS slot `slot`.
  auto fold = [&](int slot) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
      for (int o = kLpr; o < 64; o *= 2) {
        y[jj] += __shfl_xor(y[jj], o);
      }
    }
    if (lane < kLpr) {
      *reinterpret_cast<float4*>(&red[slot][wave][4 * c8]) = make_float4(y[0], y[1], y[2], y[3]);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      y[jj] = 0.0f;
    }
  };
  int n_red = 0;
  auto reduce = [&]() {
    fold(n_red & 1);
    lds_barrier();
    ++n_red;
  };

  if constexpr (kPieces) {
    for (int blk = 0; blk < rg.head_len; ++blk) {
      block((rg.head_blk0 + blk) * Q + wave);
    }
    if (rg.head_len > 0) {
      reduce();
    }
    for (int blk = 0; blk < rg.tail_len; ++blk) {
      block(blk * Q + wave);
    }
    if (rg.tail_len > 0) {
      reduce();
    }
  }
  for (int r = 0; r < rg.whole; ++r) {
    int blk = 0;
    const int n_loop = r == rg.whole - 1 ? nbs - 1 : nbs;
    if constexpr (!kPieces) {
      // blocks that each stage one more pass, then blocks that do not (no branch in either)
      const int n_staging = min(n_loop, n_pass - staged);
      for (; blk < n_staging; ++blk) {
        block(blk * Q + wave);
        stage_one();
      }
    }
    for (; blk < n_loop; ++blk) {
      block(blk * Q + wave);
    }
    if (r == rg.whole - 1) {
      if constexpr (!kPieces) {
        while (staged < n_pass) {
          stage_one();
        }
      }
      block_r((nbs - 1) * Q + wave, std::false_type{});
    }
    if constexpr (!kPieces) {
      while (staged < n_pass) {
        stage_one();
      }
    }
    // The wave's totals wait in the round's slot; a barrier every kRing slices (and after the
    // last) lets every thread write one output of the round, adding the waves in wave order.
    const int in_round = r % kRing;
    fold(2 + r % (2 * kRing));
    if (in_round == kRing - 1 || r == rg.whole - 1) {
      lds_barrier();
      const int r0 = r - in_round;
      for (int o = tid; o < (in_round + 1) * kCols; o += 64 * kW) {
        const int rr = r0 + o / kCols;
        const int c = o % kCols;
        const int slot = 2 + rr % (2 * kRing);
        float v = red[slot][0][c];
#pragma unroll
        for (int w = 1; w < kW; ++w) {
          v += red[slot][w][c];
        }
        p.out[static_cast<size_t>(rg.whole_slice0 + rr) * kCols + c] = float_to_act_bits<A>(v);
      }
    }
  }
  // Retire the loads of re-read tail slots before the workgroup ends.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

template <int G, Act A, int kStageSlots, int kCols>
hipError_t launch_arc_quarter_t(const GemvLaunch& l, hipStream_t stream) {
  int grid = 0;
  GemvParams p = native_params<G, 1>(l, &grid);
  p.pair = 0;
  grid = l.stream_grid;
  p.stream_whole = l.stream_whole;
  p.grid = grid;
  p.xcd_remap = grid % 8 == 0 ? grid / 8 : 0;
  p.ng_magic = l.ng_magic;
  const size_t lds = quarter_lds_bytes<G, kCols>(l.K / G);
  if constexpr (kCols == kSliceCols) {
    if (l.stream_pieces) {
      hipLaunchKernelGGL((w4a16_gemv_arc_quarter_kernel<G, A, kStageSlots, true, kCols>),
                         dim3(grid), dim3(64 * (kQuarterWaves + 1)), lds, stream, p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((w4a16_gemv_arc_quarter_kernel<G, A, kStageSlots, false, kCols>), dim3(grid),
                     dim3(64 * kQuarterWaves), lds, stream, p);
  return hipGetLastError();
}

template <int G, Act A, int kCols>
hipError_t arc_quarter_slots(const GemvLaunch& l, hipStream_t stream) {
  // passes of a wave: (K/G / 8 groups) / (64 / (G / 8) groups per pass)
  constexpr int kGroupsPerPass = 64 / (G / 8);
  const int passes = (l.K / G / kQuarterWaves + kGroupsPerPass - 1) / kGroupsPerPass;
  if (passes <= 2) {
    return launch_arc_quarter_t<G, A, 2, kCols>(l, stream);
  }
  // eighths: short K only (K/G <= 64 at G = 128)
  if constexpr (kCols == kSliceCols) {
    if (passes <= 8) {
      return launch_arc_quarter_t<G, A, 8, kCols>(l, stream);
    }
  }
  return hipErrorInvalidValue;
}

}  // namespace

size_t arc_quarter_lds(int group_size, int k, int cols) {
  if (group_size == 64) {
    return quarter_lds_bytes<64, kSliceCols>(k / 64);
  }
  return cols == kSliceCols / 2 ? quarter_lds_bytes<128, kSliceCols / 2>(k / 128)
                                : quarter_lds_bytes<128, kSliceCols>(k / 128);
}

bool arc_quarter_magic_exact(int num_groups, long long slices) {
  // With magic = floor(2^32 / d) + 1 = (2^32 + e) / d, 0 < e <= d: mulhi(lin, magic) =
  // floor(lin / d + lin e / (d 2^32)), which is floor(lin / d) while lin e < 2^32. Here
  // lin < slices * d and e <= d.
  return num_groups > 0 && slices > 0 &&
         static_cast<unsigned long long>(slices) * num_groups * num_groups < (1ULL << 32);
}

uint32_t arc_quarter_magic(int num_groups) {
  return static_cast<uint32_t>((1ULL << 32) / static_cast<uint64_t>(num_groups) + 1);
}

hipError_t launch_w4a16_gemv_arc_quarter(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode != GemvMode::kStreamK || l.M != 1 || l.m_tile != 1 || l.format != PacketFormat::kArc ||
      l.fuse != GemvFuse::kNone || l.K > kStreamMaxK || l.stream_grid <= 0 ||
      l.stream_whole < 0 || (l.group_size != 64 && l.group_size != 128) ||
      (l.slice_cols != kSliceCols &&
       (l.slice_cols != kSliceCols / 2 || l.group_size != 128 || l.stream_pieces))) {
    return hipErrorInvalidValue;
  }
  const int ng = l.K / l.group_size;
  const int quantum = kQuarterWaves * (l.group_size == 128 ? 2 : 4);
  if (ng % quantum != 0 || l.ng_magic != arc_quarter_magic(ng)) {
    return hipErrorInvalidValue;
  }
  const long long nbs = ng / quantum;
  const long long slices = l.N / l.slice_cols;  // units
  const long long left = slices - static_cast<long long>(l.stream_grid) * l.stream_whole;
  if (l.stream_pieces) {
    // left-over slices fewer than the workgroups, at least one left-over block per workgroup
    if (l.counters == nullptr || l.partials == nullptr || slices > kStreamMaxSlices ||
        l.stream_whole < 0 || left <= 0 || left >= l.stream_grid || left * nbs < l.stream_grid ||
        left * nbs * l.stream_grid >= (1LL << 31)) {
      return hipErrorInvalidValue;
    }
  } else if (l.stream_whole <= 0 || left != 0) {
    return hipErrorInvalidValue;
  }
  if (!arc_quarter_magic_exact(ng, slices)) {
    return hipErrorInvalidValue;
  }
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? arc_quarter_slots<64, Act::kF16, kSliceCols>(l, stream)
                              : arc_quarter_slots<64, Act::kBF16, kSliceCols>(l, stream);
  }
  if (l.slice_cols == kSliceCols / 2) {
    return l.act == Act::kF16 ? arc_quarter_slots<128, Act::kF16, kSliceCols / 2>(l, stream)
                              : arc_quarter_slots<128, Act::kBF16, kSliceCols / 2>(l, stream);
  }
  return l.act == Act::kF16 ? arc_quarter_slots<128, Act::kF16, kSliceCols>(l, stream)
                            : arc_quarter_slots<128, Act::kBF16, kSliceCols>(l, stream);
}

}  // namespace fk
