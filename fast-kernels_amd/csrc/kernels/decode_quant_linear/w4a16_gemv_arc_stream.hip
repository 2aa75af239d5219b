// W4A16 GEMV over the reference packets for one activation row, on the persistent stream schedule.
//
// The drop-in entry points (fk_arc_w4a16_forward*, arc_w4a16.cu:687-707) take the reference
// packet [(N/128) * NG, 64 G + 512]: per 128-column tile and group, G/8 word rows of 512 bytes
// (128 columns x one uint32 of 8 codes), then 128 fp16 alphas and 128 fp16 betas; the groups of a
// tile are consecutive, so a run of whole tiles is one contiguous byte range. This kernel streams
// them the way the native-slab stream kernel (w4a16_gemv_stream.hip) streams its slabs:
//
//  * one workgroup per CU streams stream_whole whole tiles b * whole .. as one contiguous range,
//    and the tiles left over (fewer than the workgroups) are dealt as equal block ranges, a head
//    and a tail piece per workgroup, handed off through the workspace by a control wave
//    (w4a16_stream_common.h; a "slice" there is a 128-column tile here);
//  * a unit is one quarter of a packet's word rows (G/32 rows: 2 KB of codes at G = 128, 1 KB at
//    G = 64) plus the alphas and betas of the lane's four columns; wave w always takes quarter
//    w mod 4 of the groups w / 4 mod 2, its i-th unit being packet (w / 4) + 2 i of its range,
//    with D units in flight (4 KB of codes per wave, the native kernel's), full 512-byte word rows
//    per load (lane l: four columns 4 (l mod 32) .., word rows of parity l / 32);
//  * each wave stages, converts and sums only the activations of its own (group, quarter) units,
//    so no barrier separates staging from streaming; the bf16 staging scale is per (group,
//    quarter);
//  * the math per unit is the reference-packet kernel's (w4a16_gemv_kernels.h compute_group):
//    (1024 + q) / (64 + q) unpack, v_dot2 into fp32 seeded with -1024 S_e - 64 S_o, then
//    y += alpha * acc + beta * (S_e + S_o), beta any fp16;
//  * at the end of a tile or piece the two lane halves (word-row parities) are added, each wave
//    writes its 128 column totals to an LDS slot, and after a barrier the totals are added in wave
//    order (deterministic).
#include "w4a16_gemv_native.h"
#include "w4a16_stream_common.h"

#include <type_traits>

namespace fk {
namespace {

constexpr int kArcStreamWaves = 8;

template <int G>
struct ArcUnit {
  static constexpr int kRows = G / 32;          // word rows of a unit
  static constexpr int kLoads = kRows / 2;      // dwordx4 loads per lane (two parities per load)
  uint4 w[kLoads];
  uint2 alpha;  // the lane's four columns
  uint2 beta;
};

// LDS view: xs [(NG + 2) * G/8] re-paired words (group-major), sums [(NG + 2) * 4 quarters * 2
// parities] {seed, S}, scale [(NG + 2) * 4] bf16 staging scales per (group, quarter).
template <int G>
struct ArcStreamLds {
  uint4* xs;
  float2* sums;
  float* scale;
};

template <int G>
__host__ __device__ constexpr size_t arc_stream_lds_bytes(int ng) {
  return static_cast<size_t>(ng + 2) * ((G / 8) * 16 + 4 * 2 * 8 + 4 * 4);
}

template <int G, Act A, int kStageSlots, bool kPieces>
__global__ void __launch_bounds__(64 * (kArcStreamWaves + (kPieces ? 1 : 0)), 1)
    w4a16_gemv_arc_stream_kernel(GemvParams p) {
  constexpr int kW = kArcStreamWaves;
  constexpr int D = G == 128 ? 2 : 4;  // units in flight per wave (4 KB of codes)
  constexpr int UR = ArcUnit<G>::kRows;
  constexpr int WR = G / 8;
  constexpr int kGroupsPerBlock = 2 * D;  // a block: kW * D units = 2 D groups
  extern __shared__ uint4 arc_stream_lds[];
  // Wave totals: slots 0 and 1 for the pieces, 2 and 3 for whole tiles in turn.
  __shared__ float red[4][kW][kTileCols];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int par = lane >> 5;   // word-row parity of the lane
  const int c4 = lane & 31;    // the lane's columns 4 c4 .. 4 c4 + 3
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, PacketFormat::kArc));
  const int grid = p.grid;
  int b = static_cast<int>(blockIdx.x);
  b = p.xcd_remap != 0 ? (b & 7) * p.xcd_remap + (b >> 3) : b;
  const int ng = p.NG;
  const int nbt = ng / kGroupsPerBlock;  // blocks per tile
  const int tiles = p.N / kTileCols;

  if constexpr (kPieces) {
    if (wave == kW) {
      // Control wave: the pieces' totals (a barrier each), their hand-offs, then the whole
      // tiles' barriers.
      const StreamRange rg = stream_range(b, grid, p.stream_whole, tiles, nbt, true);
      float v[2][2];
      const bool has[2] = {rg.head_len > 0, rg.tail_len > 0};
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        if (has[pc]) {
          lds_barrier();
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int o = lane + 64 * i;
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < kW; ++w) {
              s += red[pc][w][o];
            }
            v[pc][i] = s;
          }
        }
      }
      if (has[0]) {
        stream_hand_off<A, 2, kTileCols>(p, b, 0, rg.head_slice, grid, p.stream_whole, tiles, nbt,
                                         kTileCols, kTileCols, v[0], lane);
      }
      if (has[1]) {
        stream_hand_off<A, 2, kTileCols>(p, b, 1, rg.tail_slice, grid, p.stream_whole, tiles, nbt,
                                         kTileCols, kTileCols, v[1], lane);
      }
      for (int r = 0; r < rg.whole; ++r) {
        lds_barrier();
      }
      return;
    }
  }

  // The wave's quarter and group parity; its units are (group (w / 4) + 2 i, quarter q).
  const int q = wave & 3;
  const int gpar = (wave >> 2) & 1;
  // Activations: this wave's (group, quarter) units, 64 / UR groups per pass, loads first.
  constexpr int kGroupsPerPass = 64 / UR;
  const int n_pass = (ng / 2 + kGroupsPerPass - 1) / kGroupsPerPass;
  const int r_u = lane % UR;  // word row of the unit this lane stages
  uint4 raw[kStageSlots];
#pragma unroll
  for (int i = 0; i < kStageSlots; ++i) {
    const int g = min(gpar + 2 * (i * kGroupsPerPass + lane / UR), ng - 1);
    raw[i] = *reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(g) * G +
                                             (q * UR + r_u) * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  const StreamRange rg = stream_range(b, grid, p.stream_whole, tiles, nbt, kPieces);

  ArcStreamLds<G> sm;
  sm.xs = arc_stream_lds;
  sm.sums = reinterpret_cast<float2*>(sm.xs + static_cast<size_t>(ng + 2) * WR);
  sm.scale = reinterpret_cast<float*>(sm.sums + static_cast<size_t>(ng + 2) * 8);

  // The wave's units: head piece, tail piece, then the whole tiles (one contiguous range); unit i
  // of a part is packet base + 2 i. Past its last unit a wave re-reads it (loads unconditional).
  const int n_h = rg.head_len * D;
  const int n_t = rg.tail_len * D;
  const int n_u = n_h + n_t + rg.whole * nbt * D;
  const int j_last = n_u - 1;
  const int off_w = rg.whole_slice0 * ng + gpar - 2 * (n_h + n_t);
  const int off_t = rg.tail_slice * ng + gpar - 2 * n_h;
  const int off_h = rg.head_slice * ng + rg.head_blk0 * kGroupsPerBlock + gpar;
  auto packet = [&](int i) -> const uint8_t* {
    const int c = min(i, j_last);
    int off = off_w;
    if constexpr (kPieces) {
      int in_t = c < n_h + n_t ? 1 : 0;
      int in_h = c < n_h ? 1 : 0;
      in_t = __builtin_amdgcn_readfirstlane(in_t);
      in_h = __builtin_amdgcn_readfirstlane(in_h);
      off += in_t * (off_t - off_w) + in_h * (off_h - off_t);
    }
    return p.packets + static_cast<size_t>(static_cast<uint32_t>(2 * c + off)) * stride;
  };
  const int code_off = (q * UR + par) * kWordRowBytes + c4 * 16;
  const int scale_off = kTileCols * G / 2 + c4 * 8;
  auto load_unit = [&](ArcUnit<G>& u, int i) {
    const uint8_t* pk = packet(i);
#pragma unroll
    for (int l = 0; l < ArcUnit<G>::kLoads; ++l) {
      u.w[l] = stream_load16(pk + code_off + 2 * l * kWordRowBytes);
    }
    // plain loads: the four quarter-waves of a packet read the same scales, which non-temporal
    // loads would fetch from HBM four times
    u.alpha = *reinterpret_cast<const uint2*>(pk + scale_off);
    u.beta = *reinterpret_cast<const uint2*>(pk + scale_off + kTileCols * 2);
  };

  ArcUnit<G> buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_unit(buf[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  // Stage every pass (the weights' first loads are in flight meanwhile). Groups past the row go
  // to a spare slot.
#pragma unroll
  for (int s = 0; s < kStageSlots; ++s) {
    if (s < n_pass) {
      const int g_raw = gpar + 2 * (s * kGroupsPerPass + lane / UR);
      const int g = min(g_raw, ng + 1);
      uint4 r = raw[s];
      float undo = 1.0f;
      if constexpr (A == Act::kBF16) {
        const uint32_t e = group_max<UR>(bf16_max_mag(r)) >> 7;
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
      if constexpr (UR == 4) {
        // the unit's rows of one parity: r_u and r_u ^ 2
        se += dpp::move<dpp::kQuadXor2>(se);
        so += dpp::move<dpp::kQuadXor2>(so);
      }
      sm.xs[static_cast<size_t>(g) * WR + q * UR + r_u] = xp;
      sm.sums[(static_cast<size_t>(g) * 4 + q) * 2 + (r_u & 1)] =
          make_float2(fmaf(-1024.0f, se, -64.0f * so), se + so);
      sm.scale[static_cast<size_t>(g) * 4 + q] = undo;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // One unit of group g (tile-local): its words against the staged row, then the scales.
  auto compute = [&](const ArcUnit<G>& u, int g) __attribute__((always_inline)) {
    const float2 sp = sm.sums[(static_cast<size_t>(g) * 4 + q) * 2 + par];
    float acc[4][2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[j][0] = sp.x;
      acc[j][1] = 0.0f;
    }
#pragma unroll
    for (int l = 0; l < ArcUnit<G>::kLoads; ++l) {
      const uint4 xp = sm.xs[static_cast<size_t>(g) * WR + q * UR + 2 * l + par];
      const uint32_t words[4] = {u.w[l].x, u.w[l].y, u.w[l].z, u.w[l].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wv = words[j];
        const uint32_t w8 = wv >> 8;
        acc[j][0] = dot2<Act::kF16>((wv & mask_lo) | kBiasLow, xp.x, acc[j][0]);
        acc[j][1] = dot2<Act::kF16>((wv & mask_hi) | kBiasHigh, xp.y, acc[j][1]);
        acc[j][0] = dot2<Act::kF16>((w8 & mask_lo) | kBiasLow, xp.z, acc[j][0]);
        acc[j][1] = dot2<Act::kF16>((w8 & mask_hi) | kBiasHigh, xp.w, acc[j][1]);
      }
    }
    const uint32_t ab[4] = {u.alpha.x, u.alpha.x >> 16, u.alpha.y, u.alpha.y >> 16};
    const uint32_t bb[4] = {u.beta.x, u.beta.x >> 16, u.beta.y, u.beta.y >> 16};
    const float scale = A == Act::kBF16 ? sm.scale[static_cast<size_t>(g) * 4 + q] : 1.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = half_bits_to_float(static_cast<uint16_t>(ab[j]));
      const float bt = half_bits_to_float(static_cast<uint16_t>(bb[j]));
      const float sum = acc[j][0] + acc[j][1];
      if constexpr (A == Act::kBF16) {
        y[j] = fmaf(fmaf(bt, sp.y, a * sum), scale, y[j]);
      } else {
        y[j] = fmaf(bt, sp.y, fmaf(a, sum, y[j]));
      }
    }
  };
  int j = 0;  // the wave's next unit
  // A block of D units, groups gl0 + 2 d (tile-local); refill = false on the wave's last block.
  auto block_r = [&](int gl0, auto refill) __attribute__((always_inline)) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      compute(buf[d], gl0 + 2 * d);
      if constexpr (decltype(refill)::value) {
        load_unit(buf[d], j + d + D);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    j += D;
  };
  auto block = [&](int gl0) { block_r(gl0, std::true_type{}); };
  // The lane halves (parities) added, then the wave's 128 column totals into LDS slot `slot`.
  auto fold = [&](int slot) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      y[jj] += __shfl_xor(y[jj], 32);
    }
    if (lane < 32) {
      *reinterpret_cast<float4*>(&red[slot][wave][4 * c4]) = make_float4(y[0], y[1], y[2], y[3]);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      y[jj] = 0.0f;
    }
  };

  if constexpr (kPieces) {
    for (int blk = 0; blk < rg.head_len; ++blk) {
      block((rg.head_blk0 + blk) * kGroupsPerBlock + gpar);
    }
    if (rg.head_len > 0) {
      fold(0);
      lds_barrier();
    }
    for (int blk = 0; blk < rg.tail_len; ++blk) {
      block(blk * kGroupsPerBlock + gpar);
    }
    if (rg.tail_len > 0) {
      fold(1);
      lds_barrier();
    }
  }
  for (int r = 0; r < rg.whole; ++r) {
    const int n_loop = r == rg.whole - 1 ? nbt - 1 : nbt;
    for (int blk = 0; blk < n_loop; ++blk) {
      block(blk * kGroupsPerBlock + gpar);
    }
    if (r == rg.whole - 1) {
      block_r((nbt - 1) * kGroupsPerBlock + gpar, std::false_type{});
    }
    const int slot = 2 + (r & 1);
    fold(slot);
    lds_barrier();
    if (tid < kTileCols) {
      float v = red[slot][0][tid];
#pragma unroll
      for (int w = 1; w < kW; ++w) {
        v += red[slot][w][tid];
      }
      p.out[static_cast<size_t>(rg.whole_slice0 + r) * kTileCols + tid] = float_to_act_bits<A>(v);
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

template <int G, Act A, int kStageSlots>
hipError_t launch_arc_stream_t(const GemvLaunch& l, hipStream_t stream) {
  int grid = 0;
  GemvParams p = native_params<G, 1>(l, &grid);
  p.pair = 0;
  grid = l.stream_grid;
  p.stream_whole = l.stream_whole;
  p.grid = grid;
  p.xcd_remap = grid % 8 == 0 ? grid / 8 : 0;
  const size_t lds = arc_stream_lds_bytes<G>(l.K / G);
  if (l.stream_pieces) {
    hipLaunchKernelGGL((w4a16_gemv_arc_stream_kernel<G, A, kStageSlots, true>), dim3(grid),
                       dim3(64 * (kArcStreamWaves + 1)), lds, stream, p);
  } else {
    hipLaunchKernelGGL((w4a16_gemv_arc_stream_kernel<G, A, kStageSlots, false>), dim3(grid),
                       dim3(64 * kArcStreamWaves), lds, stream, p);
  }
  return hipGetLastError();
}

template <int G, Act A>
hipError_t arc_stream_slots(const GemvLaunch& l, hipStream_t stream) {
  // passes of a wave: (NG / 2 groups) / (64 / (G / 32) groups per pass)
  const int passes = (l.K / G / 2 + 64 / (G / 32) - 1) / (64 / (G / 32));
  if (passes <= 2) {
    return launch_arc_stream_t<G, A, 2>(l, stream);
  }
  if (passes <= 8) {
    return launch_arc_stream_t<G, A, 8>(l, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

size_t arc_stream_lds(int group_size, int k) {
  return group_size == 64 ? arc_stream_lds_bytes<64>(k / 64) : arc_stream_lds_bytes<128>(k / 128);
}

hipError_t launch_w4a16_gemv_arc_stream(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode != GemvMode::kStreamK || l.M != 1 || l.m_tile != 1 || l.format != PacketFormat::kArc ||
      l.fuse != GemvFuse::kNone || l.K > kStreamMaxK || l.stream_grid <= 0 ||
      l.stream_whole < 0 || (l.group_size != 64 && l.group_size != 128)) {
    return hipErrorInvalidValue;
  }
  const int ng = l.K / l.group_size;
  const int per_block = 2 * (l.group_size == 128 ? 2 : 4);
  if (ng % per_block != 0) {
    return hipErrorInvalidValue;
  }
  const long long nbt = ng / per_block;
  const long long tiles = l.N / kTileCols;
  const long long left = tiles - static_cast<long long>(l.stream_grid) * l.stream_whole;
  if (l.stream_pieces) {
    if (l.counters == nullptr || l.partials == nullptr || tiles > kStreamMaxSlices || left <= 0 ||
        left >= l.stream_grid || left * nbt < l.stream_grid ||
        left * nbt * l.stream_grid >= (1LL << 31)) {
      return hipErrorInvalidValue;
    }
  } else if (l.stream_whole <= 0 || left != 0) {
    return hipErrorInvalidValue;
  }
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? arc_stream_slots<64, Act::kF16>(l, stream)
                              : arc_stream_slots<64, Act::kBF16>(l, stream);
  }
  return l.act == Act::kF16 ? arc_stream_slots<128, Act::kF16>(l, stream)
                            : arc_stream_slots<128, Act::kBF16>(l, stream);
}

}  // namespace fk
