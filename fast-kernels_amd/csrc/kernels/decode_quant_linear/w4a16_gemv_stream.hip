// W4A16 GEMV over native slabs for one activation row: the persistent "stream" schedule.
//
// The native slabs of a buffer are laid out [slice][group] (w4a16_device.h), so a run of slices is
// one contiguous byte range. With one workgroup per CU, workgroup b streams the stream_whole
// slices b * stream_whole .. as one range. The slices left over when they do not divide evenly
// (fewer than the workgroups) are cut into blocks of kW * D groups (one slab in each of a wave's D
// register buffers) and dealt to the workgroups as equal contiguous block ranges ("stream-K"), so
// every CU streams the same number of bytes whatever the shape. Such a range is shorter than a
// slice: at most a head piece (the end of a slice an earlier workgroup starts) and a tail piece
// (the start of a slice a later workgroup finishes).
//
//  * The activation rows are staged in LDS once per workgroup (dynamic LDS: K/G groups of
//    re-paired fp16 values and per-quarter sums per row, as native_stage_unit writes them). Wave w
//    only ever computes groups g = w (mod kW), so each wave stages its own groups and no
//    workgroup barrier separates staging from streaming. Without pieces the staging is spread
//    over the first slice (one pass of the wave's groups before its first block, one more after
//    each block), so that the first weights are consumed as soon as they arrive; with pieces all
//    passes are staged first (a piece may start anywhere in K).
//  * The staging loads are issued before the first weight loads, so the conversion overlaps the
//    weights' HBM latency (the load counter retires in order, so waiting for the activations does
//    not wait for the weights behind them).
//  * Wave w takes slabs w, w + kW, w + 2 kW, ... of each part (pieces first, then the whole
//    slices) through D register buffers, and the pipeline runs across part and slice boundaries: the loads of the next slabs are in flight
//    while a slice is reduced, so the stream never drains before the workgroup's last slab. The
//    slab address is a uniform select between the three parts' bases, so the pipelined loops have
//    no branch.
//  * At the end of a slice or piece each wave folds its lane partials over the column's four
//    quarters into an LDS slot of its own. A piece's totals then meet the control wave at a
//    barrier. Whole slices' totals wait in a ring of slots: a barrier every four slices (and
//    after the last) lets every thread of the workgroup write one output of those slices, adding
//    the waves' totals in wave order, so the waves do not meet once per slice (7B qkv, three
//    half-slices per CU: 7.4 -> 7.0 us). The loads of the next slabs stay in flight throughout.
//  * The pieces are streamed first (head, then tail) and handed to a ninth, control wave (kPieces)
//    so that their hand-off is off the critical path: the control wave adds the waves' totals,
//    stores the piece's partial sums to the workspace (one slot per workgroup and piece) and
//    bumps the slice's arrival counter once they are acknowledged; the workgroup that arrives
//    last adds the slice's parts in workgroup order, so the result does not depend on arrival
//    order, writes the outputs and resets the counter for the next call. The streaming waves go
//    on meanwhile; the control wave meets them at every later barrier (s_barrier counts waves).
//  * With the logical-to-hardware workgroup remap consecutive ranges, and so the parts of a split
//    slice, run on one XCD, whose L2 then serves the partials the last part reads.
//  * kHalf (one row, G = 128): the slices' 16-column halves are the units (the first or second KB
//    of every slab). Workgroup b streams half-slices b * whole .. (slice hs / 2, half hs & 1):
//    with at most half as many slices as CUs one each, so every CU streams and no slice is split
//    over K; with twice the slices a multiple of the CUs (8B gate_up: 1792 halves, 7 per CU) an
//    even share of halves, where whole slices would not divide.
//
// Math per group is native_compute_group's (w4a16_gemv_native.h); results equal the per-slice
// kernel's up to fp32 summation order across waves.
#include "w4a16_gemv_native.h"
#include "w4a16_stream_common.h"

#include <type_traits>

namespace fk {
namespace {

// LDS view of the staged activation rows: xs [MT][NG + 1][G/8] re-paired fp16 words, sums
// [MT][NG + 1][4] per-quarter offset terms, scale [MT][NG + 1] bf16 staging scales (the layout of
// NativeSmem for every group of K, plus a spare group slot per row for branch-free staging).
template <int G>
struct StreamLds {
  uint4* xs;
  float2* sums;
  float* scale;
  int slots;  // NG + 1

  __device__ int at(int m, int gl) const { return m * slots + gl; }
  __device__ uint4 x_at(int m, int gl, int i) const { return xs[at(m, gl) * (G / 8) + i]; }
  __device__ float2 sums_at(int m, int gl, int t) const { return sums[at(m, gl) * 4 + t]; }
  __device__ float scale_at(int m, int gl) const { return scale[at(m, gl)]; }
  __device__ void set_x(int m, int gl, int i, uint4 v) { xs[at(m, gl) * (G / 8) + i] = v; }
  __device__ void set_sums(int m, int gl, int t, float2 v) { sums[at(m, gl) * 4 + t] = v; }
  __device__ void set_scale(int m, int gl, float v) { scale[at(m, gl)] = v; }
};

// kW streaming waves per workgroup (plus the control wave with kPieces), D register buffers
// (slabs in flight) per wave, MT activation rows; one workgroup per CU. kStageSlots passes of
// 64 / (G / 8) groups per wave stage K <= kStageSlots * 64 * kW * 8 activations.
//
// kFuse (one row, whole slices, no pieces): kRmsNorm stages round(gamma * round(x * inv_rms))
// with inv_rms = 1 / sqrt(mean(x^2) + eps) of the row, formed per workgroup from the staging
// loads it issues anyway (each wave's sum over its own groups, one barrier). kSiluMul: the weight
// is [W_gate; W_up] stacked along N, and workgroup b streams the gate slices b * whole .. and then
// the same up slices (slice + N / 64), keeps all their totals in the LDS ring, and writes
// round(round(silu(round(g))) * round(u)) to out[N / 2] (the unfused GEMV, SiLU and product, each
// rounded to the activation dtype). kRmsNormSiluMul: both.
template <int G, Act A, PacketFormat F, int kStageSlots, int kW, int D, int MT, bool kPieces,
          bool kHalf, bool kRagged = false, GemvFuse kFuse = GemvFuse::kNone>
__global__ void __launch_bounds__(64 * (kW + (kPieces ? 1 : 0)), 1)
    w4a16_gemv_stream_kernel(GemvParams p) {
  static_assert(!kHalf || (MT == 1 && !kPieces && G == 128), "half slices: one row, no pieces");
  static_assert(!kRagged || kHalf, "a partial last block: half slices only");
  constexpr bool kNorm = kFuse == GemvFuse::kRmsNorm || kFuse == GemvFuse::kRmsNormSiluMul;
  constexpr bool kSilu = kFuse == GemvFuse::kSiluMul || kFuse == GemvFuse::kRmsNormSiluMul;
  static_assert(kFuse == GemvFuse::kNone || (MT == 1 && !kPieces && !kHalf),
                "fused: one row over whole slices");
  extern __shared__ uint4 stream_lds[];
  // Wave totals: slots 0 and 1 for the pieces, then two rounds of kRing whole slices.
  constexpr int kRing = 4;
  __shared__ float red[2 + 2 * kRing][kW][MT * kSliceCols];
  __shared__ float rms_part[kW];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = lane / 16;
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  const int grid = p.grid;
  int b = static_cast<int>(blockIdx.x);
  // Consecutive logical workgroups on one XCD (the hardware deals workgroup b to XCD b % 8).
  b = p.xcd_remap != 0 ? (b & 7) * p.xcd_remap + (b >> 3) : b;
  const int ng = p.NG;
  constexpr int Q = kW * D;  // groups per block
  // Blocks per slice. kRagged (half slices whose group count is not a multiple of Q): the last
  // block's groups past the slice re-read its last slab and compute against the spare group slot
  // of the staged row, which holds zeros, so they add nothing. The clamps this takes cost the
  // other shapes 0.1-0.6 us, so they are compiled in only there.
  const int nbs = kRagged ? (ng + Q - 1) / Q : ng / Q;
  // slice-local group g clamped into the slice (kRagged), for the weights and the staged row
  auto clamp_w = [&](int g) { return kRagged ? min(g, ng - 1) : g; };
  auto clamp_x = [&](int g) { return kRagged ? min(g, ng) : g; };
  constexpr int kOut = MT * kSliceCols;  // outputs of a slice
  constexpr int kOutPerLane = (kOut + 63) / 64;

  const int slices = p.N / kSliceCols;
  if constexpr (kPieces) {
    if (wave == kW) {
      const StreamRange rg = stream_range(b, grid, p.stream_whole, slices, nbs, true);
      // Control wave. Totals of the pieces first (a barrier each), then their hand-offs, then the
      // whole slices' barriers.
      float v[2][kOutPerLane];
      int slot = 0;
      const bool has[2] = {rg.head_len > 0, rg.tail_len > 0};
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        if (has[pc]) {
          lds_barrier();
#pragma unroll
          for (int i = 0; i < kOutPerLane; ++i) {
            const int o = lane + 64 * i;
            float s = 0.0f;
            if (o < kOut) {
#pragma unroll
              for (int w = 0; w < kW; ++w) {
                s += red[slot][w][o];
              }
            }
            v[pc][i] = s;
          }
          slot ^= 1;
        }
      }
      if (has[0]) {
        stream_hand_off<A, kOutPerLane>(p, b, 0, rg.head_slice, grid, p.stream_whole, slices, nbs,
                                        kOut, kOut, v[0], lane);
      }
      if (has[1]) {
        stream_hand_off<A, kOutPerLane>(p, b, 1, rg.tail_slice, grid, p.stream_whole, slices, nbs,
                                        kOut, kOut, v[1], lane);
      }
      for (int r = 0; r < (rg.whole + kRing - 1) / kRing; ++r) {
        lds_barrier();
      }
      return;
    }
  }

  // Activations: every pass's loads first, ahead of the range arithmetic (with pieces some hundred
  // scalar instructions of divisions). Pass i stages groups wave + kW (i * 64 / WR + l / WR) (lane
  // l, word row l % WR) of every row.
  constexpr int WR = G / 8;
  constexpr int kGroupsPerPass = 64 / WR;
  const int n_pass = (nbs * D + kGroupsPerPass - 1) / kGroupsPerPass;
  uint4 raw[kStageSlots][MT];
#pragma unroll
  for (int i = 0; i < kStageSlots; ++i) {
    // clamped and unconditional (a load under a branch waits for the one before it); slots past
    // the wave's passes and groups past the row are never staged
    const int g = min(wave + kW * (i * kGroupsPerPass + lane / WR), ng - 1);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      raw[i][m] = *reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(m) * p.K +
                                                  static_cast<size_t>(g) * G + (lane % WR) * 8);
    }
  }
  // (no use of the loaded registers here: that would wait for the first load before the weights'
  // loads go out)
  __builtin_amdgcn_sched_barrier(0);
  StreamRange rg = stream_range(b, grid, p.stream_whole, slices, nbs, kPieces);
  if constexpr (kSilu) {
    rg.whole_slice0 = b * (p.stream_whole / 2);  // gate slices (whole / 2 of them), then up
  }
  // kHalf: half-slices hs0 .. hs0 + whole - 1, half-slice hs being half hs & 1 of slice hs / 2.
  const int hs0 = kHalf ? b * p.stream_whole : 0;
  int half = 0;

  StreamLds<G> sm;
  sm.slots = ng + 1;
  sm.xs = stream_lds;
  sm.sums = reinterpret_cast<float2*>(stream_lds + static_cast<size_t>(MT) * sm.slots * (G / 8));
  sm.scale = reinterpret_cast<float*>(sm.sums + static_cast<size_t>(MT) * sm.slots * 4);

  // The wave's slabs, in order: the head piece's, the tail piece's, then the whole slices' (one
  // contiguous range). Past its last slab a wave re-reads that slab, so every buffer slot is
  // loaded unconditionally (and never past the buffer).
  const int n_h = rg.head_len * D;
  const int n_t = rg.tail_len * D;
  const int n_w = n_h + n_t + rg.whole * nbs * D;
  const int j_last = n_w - 1;
  // Slab index of the wave's i-th slab: i * kW plus a per-part offset (uniform 32-bit arithmetic;
  // selects of 64-bit addresses compile to branches).
  const int off_w = rg.whole_slice0 * ng + wave - (n_h + n_t) * kW;
  // kSilu: the first half of the range is the gate slices, the second the same up slices
  const int n_gate = kSilu ? rg.whole / 2 * nbs * D : 0;
  const int off_up = (rg.whole_slice0 + slices / 2) * ng + wave - n_gate * kW;
  const int off_t = rg.tail_slice * ng + wave - n_h * kW;
  const int off_h = rg.head_slice * ng + rg.head_blk0 * Q + wave;
  auto slab = [&](int i) -> const uint8_t* {
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
    if constexpr (kSilu) {
      const int in_up = __builtin_amdgcn_readfirstlane(c >= n_gate ? 1 : 0);
      off += in_up * (off_up - off_w);
    }
    return p.packets + static_cast<size_t>(static_cast<uint32_t>(c * kW + off)) * stride;
  };
  // kHalf: the wave's slab i is slab jj of half-slice r (spr slabs a half-slice), uniform 32-bit
  // arithmetic.
  const int spr = nbs * D;
  auto load_slab = [&](NativeLoad<G>& ld, int i) {
    if constexpr (kHalf) {
      const int c = __builtin_amdgcn_readfirstlane(min(i, j_last));
      const int r = static_cast<int>(static_cast<uint32_t>(c) / static_cast<uint32_t>(spr));
      const int hs = hs0 + r;
      const int jj = c - r * spr;
      native_load_half<G, F>(
          ld, p.packets + static_cast<size_t>(static_cast<uint32_t>((hs >> 1) * ng +
                                                                    clamp_w(wave + kW * jj))) *
                              stride,
          lane, hs & 1);
    } else {
      native_load<G, F>(ld, slab(i), lane);
    }
  };

  // kNorm: gamma of the same units (one row of K for all rows)
  uint4 gam[kNorm ? kStageSlots : 1];
  if constexpr (kNorm) {
#pragma unroll
    for (int i = 0; i < kStageSlots; ++i) {
      const int g = min(wave + kW * (i * kGroupsPerPass + lane / WR), ng - 1);
      gam[i] = *reinterpret_cast<const uint4*>(p.norm_weight + static_cast<size_t>(g) * G +
                                               (lane % WR) * 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  NativeLoad<G> buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_slab(buf[d], d);
    __builtin_amdgcn_sched_barrier(0);  // the same issue order as the refills in the loop
  }
  // kNorm: 1 / sqrt(mean(x^2) + eps) of the row (fp32 sums). Every unit of the row is in exactly
  // one lane's staging registers (slots of the wave's passes, groups inside the row), so the
  // waves' sums add up to the row's; the weights' loads are in flight meanwhile.
  float inv_rms = 1.0f;
  if constexpr (kNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kStageSlots; ++i) {
      const bool live = i < n_pass && wave + kW * (i * kGroupsPerPass + lane / WR) < ng;
      float si = 0.0f;
      si = sum_sq_word<A>(raw[i][0].x, si);
      si = sum_sq_word<A>(raw[i][0].y, si);
      si = sum_sq_word<A>(raw[i][0].z, si);
      si = sum_sq_word<A>(raw[i][0].w, si);
      ss += live ? si : 0.0f;
    }
    // the wave's total: DPP within each 16-lane row, then the four rows' lanes 0 read out (a
    // shuffle per step would be an LDS round trip)
    ss = group_sum<16>(ss);
    ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ss), 48));
    if (lane == 0) {
      rms_part[wave] = ss;
    }
    lds_barrier();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      total += rms_part[w];
    }
    inv_rms = 1.0f / sqrtf(total / static_cast<float>(p.K) + p.eps);
  }
  int staged = 0;
  // Stages the next pass from raw[0] and shifts the slots down (register moves; a runtime slot
  // index would put the slots in scratch memory).
  auto stage_one = [&]() {
    // Groups past the row (the wave's last pass may be partial) go to the spare group
    // slot past the row's (zeros with kRagged, which reads it), so the staging has no branch.
    const int g_raw = wave + kW * (staged * kGroupsPerPass + lane / WR);
    const int g = min(g_raw, ng);
    const uint32_t keep = !kRagged || g_raw < ng ? 0xffffffffu : 0u;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      uint4 v = raw[0][m];
      if constexpr (kRagged) {
        v = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
      }
      if constexpr (kNorm) {
        const uint4 gw = gam[0];
        v = make_uint4(norm_pair<A>(v.x, gw.x, inv_rms), norm_pair<A>(v.y, gw.y, inv_rms),
                       norm_pair<A>(v.z, gw.z, inv_rms), norm_pair<A>(v.w, gw.w, inv_rms));
      }
      native_stage_unit<G, A, F>(sm, v, m, g, lane % WR);
    }
#pragma unroll
    for (int i = 0; i + 1 < kStageSlots; ++i) {
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        raw[i][m] = raw[i + 1][m];
      }
      if constexpr (kNorm) {
        gam[i] = gam[i + 1];
      }
    }
    ++staged;
    // The wave reads back only what it wrote: its LDS accesses complete in order, so a
    // wave-scope fence (no instruction) is all that keeps the compiler from hoisting the reads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  stage_one();
  if constexpr (kPieces) {
    while (staged < n_pass) {
      stage_one();
    }
  }

  float y[MT][2];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    y[m][0] = 0.0f;
    y[m][1] = 0.0f;
  }
  int j = 0;  // the wave's next slab to compute
  // A block of D slabs of slice-local groups gl0 .., kW apart. Every part is whole blocks (the
  // host plans K/G as a multiple of kW * D), so the block loops have no branch: the compiler's
  // wait for a buffer is then the in-order count of the loads issued after it, not a drain of the
  // pipeline.
  // refill = false: the wave's last block, whose refills would only re-read its last slab and
  // hold the wave (the end waits for every load) one memory latency after its last arithmetic.
  // One row: the next slab's staged operands are read from LDS while the current slab computes
  // (in pairs of slabs, the operand registers alternating), so the LDS latency is off the path.
  // Measured on MI355X (alternating runs): 8B gate_up -0.1-0.3 us, 7B down (half slices with a
  // partial last block) 6.8 -> 6.5 us; whole-block half slices were slower with it (8B down
  // +0.3 us) and keep reading their operands per slab.
  auto step = [&](int d, int gl0, const RowOps<G>& cur, RowOps<G>& nxt, auto refill)
      __attribute__((always_inline)) {
    if (d + 1 < D) {
      native_load_ops<G, A>(sm, clamp_x(gl0 + kW * (d + 1)), t, nxt);
    }
    native_compute_ops<G, A, F, kHalf ? 1 : 2>(cur, buf[d], mask_lo, mask_hi, y, half);
    if constexpr (decltype(refill)::value) {
      load_slab(buf[d], j + d + D);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto block_r = [&](int gl0, auto refill) __attribute__((always_inline)) {
    if constexpr (MT == 1 && D % 2 == 0 && (!kHalf || kRagged)) {
      RowOps<G> op0;
      RowOps<G> op1;
      native_load_ops<G, A>(sm, clamp_x(gl0), t, op0);
#pragma unroll
      for (int d = 0; d < D; d += 2) {
        step(d, gl0, op0, op1, refill);
        step(d + 1, gl0, op1, op0, refill);
      }
    } else {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        native_compute_group<G, A, MT, F, StreamLds<G>, kHalf ? 1 : 2>(sm, buf[d],
                                                                       clamp_x(gl0 + kW * d), t,
                                                                       mask_lo, mask_hi, y, half);
        if constexpr (decltype(refill)::value) {
          load_slab(buf[d], j + d + D);
        }
        // Issue the refill here, not after the block's later slabs: the scheduler would
        // otherwise sink every load below the block's arithmetic and drain the pipeline once per
        // block.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    j += D;
  };
  auto block = [&](int gl0) { block_r(gl0, std::true_type{}); };
  int n_red = 0;  // piece reductions so far: LDS slot 0 (head) or 1 (tail)
  // Folds the lane partials over the column's four quarters (lanes n, n+16, n+32, n+48) into LDS
  // slot `slot` and clears them.
  auto fold = [&](int slot) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float y0 = y[m][0];
      float y1 = y[m][1];
      y0 += __shfl_xor(y0, 16);
      y0 += __shfl_xor(y0, 32);
      if constexpr (!kHalf) {
        y1 += __shfl_xor(y1, 16);
        y1 += __shfl_xor(y1, 32);
      }
      y[m][0] = 0.0f;
      y[m][1] = 0.0f;
      if (lane < 16) {
        red[slot][wave][m * kSliceCols + lane] = y0;
        if constexpr (!kHalf) {
          red[slot][wave][m * kSliceCols + lane + 16] = y1;
        }
      }
    }
  };
  // A piece's totals meet the control wave at a barrier (the loads of the next slabs stay in
  // flight).
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
    if constexpr (kHalf) {
      half = (hs0 + r) & 1;
    }
    // Without pieces: blocks that each stage one more pass, then blocks that do not: two loops,
    // no branch in either.
    int blk = 0;
    // the last slice's last block is the wave's last: no refills
    const int n_loop = r == rg.whole - 1 ? nbs - 1 : nbs;
    if constexpr (!kPieces) {
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
        while (staged < n_pass) {  // the passes the last block reads, if still due
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
    // The wave's totals wait in the round's LDS slot; a barrier every kRing slices (and after
    // the last) lets all waves write the round's outputs at once, adding the waves' totals in wave
    // order. Rounds alternate between two sets of slots: a wave writes a set again only after the
    // next round's barrier, which every wave reaches after reading it.
    if constexpr (kSilu) {
      // every slice's totals stay in the ring (2 * whole <= 2 * kRing slots); one barrier after
      // the last, then the gate and up totals of each output
      fold(2 + r);
      if (r == rg.whole - 1) {
        lds_barrier();
        const int pairs = rg.whole / 2;
        for (int o = tid; o < pairs * kSliceCols; o += 64 * kW) {
          const int rr = o / kSliceCols;
          const int c = o % kSliceCols;
          float gv = red[2 + rr][0][c];
          float uv = red[2 + pairs + rr][0][c];
#pragma unroll
          for (int w = 1; w < kW; ++w) {
            gv += red[2 + rr][w][c];
            uv += red[2 + pairs + rr][w][c];
          }
          const float gr = act_bits_to_float<A>(float_to_act_bits<A>(gv));
          const float ur = act_bits_to_float<A>(float_to_act_bits<A>(uv));
          const float sg = act_bits_to_float<A>(float_to_act_bits<A>(gr / (1.0f + expf(-gr))));
          p.out[static_cast<size_t>(rg.whole_slice0 + rr) * kSliceCols + c] =
              float_to_act_bits<A>(sg * ur);
        }
      }
      continue;
    }
    const int in_round = r % kRing;
    fold(2 + r % (2 * kRing));
    if (in_round == kRing - 1 || r == rg.whole - 1) {
      lds_barrier();
      constexpr int kCols = kHalf ? kSliceCols / 2 : kSliceCols;
      constexpr int kPerSlice = MT * kCols;
      const int r0 = r - in_round;
      for (int o = tid; o < (in_round + 1) * kPerSlice; o += 64 * kW) {
        const int rr = r0 + o / kPerSlice;
        const int m = (o % kPerSlice) / kCols;
        const int c = o % kCols;
        const int slot = 2 + rr % (2 * kRing);
        if (m < p.M) {
          float v = red[slot][0][m * kSliceCols + c];
#pragma unroll
          for (int w = 1; w < kW; ++w) {
            v += red[slot][w][m * kSliceCols + c];
          }
          const int slice = kHalf ? (hs0 + rr) >> 1 : rg.whole_slice0 + rr;
          const int col = kHalf ? 16 * ((hs0 + rr) & 1) + c : c;
          p.out[static_cast<size_t>(m) * p.N + static_cast<size_t>(slice) * kSliceCols + col] =
              float_to_act_bits<A>(v);
        }
      }
    }
  }
  // Retire the loads of re-read tail slots before the workgroup ends.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

template <int G, Act A, PacketFormat F, int kStageSlots, int kW, int D, int MT>
hipError_t launch_stream_t(const GemvLaunch& l, hipStream_t stream) {
  int grid = 0;
  GemvParams p = native_params<G, MT>(l, &grid);
  p.pair = 0;
  grid = l.stream_grid;
  p.stream_whole = l.stream_whole;
  p.grid = grid;
  p.xcd_remap = grid % 8 == 0 ? grid / 8 : 0;
  const size_t lds = static_cast<size_t>(MT) * stream_lds_bytes(G, l.K / G + 1);
  if (l.fuse != GemvFuse::kNone) {
    if constexpr (MT == 1 && D == stream_depth_for_kb(G, kStreamKB)) {
      if (l.stream_pieces || l.stream_half) {
        return hipErrorInvalidValue;
      }
      switch (l.fuse) {
        case GemvFuse::kRmsNorm:
          hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, 1, false, false,
                                                       false, GemvFuse::kRmsNorm>),
                             dim3(grid), dim3(64 * kW), lds, stream, p);
          break;
        case GemvFuse::kSiluMul:
          hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, 1, false, false,
                                                       false, GemvFuse::kSiluMul>),
                             dim3(grid), dim3(64 * kW), lds, stream, p);
          break;
        default:
          hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, 1, false, false,
                                                       false, GemvFuse::kRmsNormSiluMul>),
                             dim3(grid), dim3(64 * kW), lds, stream, p);
          break;
      }
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
  if constexpr (D != stream_depth_for_kb(G, kStreamKB)) {
    // the deeper pipeline serves half slices only (a half-slab is half the bytes)
    if constexpr (G == 128 && MT == 1) {
      if (!l.stream_half || l.stream_pieces) {
        return hipErrorInvalidValue;
      }
      if ((l.K / G) % (kW * D) != 0) {
        hipLaunchKernelGGL(
            (w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, 1, false, true, true>),
            dim3(grid), dim3(64 * kW), lds, stream, p);
      } else {
        hipLaunchKernelGGL(
            (w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, 1, false, true>),
            dim3(grid), dim3(64 * kW), lds, stream, p);
      }
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
  if (l.stream_pieces) {
    hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, MT, true, false>),
                       dim3(grid), dim3(64 * (kW + 1)), lds, stream, p);
  } else if (l.stream_half) {
    if constexpr (G == 128 && MT == 1) {
      if ((l.K / G) % (kW * D) != 0) {
        hipLaunchKernelGGL(
            (w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, 1, false, true, true>),
            dim3(grid), dim3(64 * kW), lds, stream, p);
      } else {
        hipLaunchKernelGGL(
            (w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, 1, false, true>),
            dim3(grid), dim3(64 * kW), lds, stream, p);
      }
    } else {
      return hipErrorInvalidValue;
    }
  } else {
    hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, MT, false, false>),
                       dim3(grid), dim3(64 * kW), lds, stream, p);
  }
  return hipGetLastError();
}

template <int G, Act A, PacketFormat F, int kW, int D, int MT>
hipError_t stream_dispatch_slots(const GemvLaunch& l, hipStream_t stream) {
  constexpr int kPerPass = 64 * kW * 8;  // activations staged per slot
  if (l.K <= kPerPass * (16 / kW)) {
    return launch_stream_t<G, A, F, 16 / kW, kW, D, MT>(l, stream);
  }
  if (l.K <= kPerPass * (64 / kW)) {
    return launch_stream_t<G, A, F, 64 / kW, kW, D, MT>(l, stream);
  }
  return hipErrorInvalidValue;
}

template <int G, Act A, PacketFormat F>
hipError_t stream_dispatch_rows(const GemvLaunch& l, hipStream_t stream) {
  constexpr int D = stream_depth_for_kb(G, kStreamKB);
  if (l.stream_waves != kStreamWaves ||
      (l.stream_depth != D && !(l.stream_half && l.stream_depth == 2 * D))) {
    return hipErrorInvalidValue;
  }
  if constexpr (G == 128) {
    // half slices with the weights' bytes in flight of whole slices
    if (l.stream_half && l.stream_depth == 2 * D && l.M == 1) {
      return stream_dispatch_slots<G, A, F, kStreamWaves, 2 * D, 1>(l, stream);
    }
  }
  // MT > 1 (several rows per slab) builds, but measured slower than the per-slice runs on MI355X
  // (benchmark configuration 3, 14336 x 4096, G = 64: two rows 9.7 -> 10.5 us, four rows 12.9 ->
  // 13.7 us; the dot2 arithmetic of four rows per slab at two waves per SIMD does not keep up),
  // so only one row is dispatched.
  if (l.M != 1) {
    return hipErrorInvalidValue;
  }
  return stream_dispatch_slots<G, A, F, kStreamWaves, D, 1>(l, stream);
}

template <PacketFormat F>
hipError_t stream_dispatch(const GemvLaunch& l, hipStream_t stream) {
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? stream_dispatch_rows<64, Act::kF16, F>(l, stream)
                              : stream_dispatch_rows<64, Act::kBF16, F>(l, stream);
  }
  return l.act == Act::kF16 ? stream_dispatch_rows<128, Act::kF16, F>(l, stream)
                            : stream_dispatch_rows<128, Act::kBF16, F>(l, stream);
}

}  // namespace

hipError_t launch_w4a16_gemv_stream(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode != GemvMode::kStreamK || l.m_tile != l.M || l.slice_cols != kSliceCols ||
      l.slice_pair || l.K > kStreamMaxK || l.stream_depth <= 0 || l.stream_grid <= 0) {
    return hipErrorInvalidValue;
  }
  // Whole blocks of waves * depth groups per slice, except half slices (whose last block may be
  // partial). Half slices: G = 128, one row, two workgroups per slice. Pieces: the workspace to
  // finish the split slices. Else whole slices, the same count per workgroup; with the SiLU
  // epilogue, gate and up slices in pairs (whole / 2 of each, up to the ring's 8 slots).
  const int ng = l.K / l.group_size;
  const int quantum = l.stream_waves * l.stream_depth;
  if (ng % quantum != 0 && !l.stream_half) {
    return hipErrorInvalidValue;
  }
  const long long slices = l.N / kSliceCols;
  if (l.fuse != GemvFuse::kNone) {
    const bool norm = l.fuse == GemvFuse::kRmsNorm || l.fuse == GemvFuse::kRmsNormSiluMul;
    const bool silu = l.fuse == GemvFuse::kSiluMul || l.fuse == GemvFuse::kRmsNormSiluMul;
    if (l.M != 1 || l.stream_half || l.stream_pieces || (norm && l.norm_weight == nullptr) ||
        l.stream_whole <= 0 || (silu && (slices % 2 != 0 || l.stream_whole % 2 != 0 ||
                                          l.stream_whole > 8))) {
      return hipErrorInvalidValue;
    }
  }
  if (l.stream_half) {
    if (l.group_size != 128 || l.M != 1 || l.stream_pieces || l.stream_whole <= 0 ||
        static_cast<long long>(l.stream_grid) * l.stream_whole != 2 * slices) {
      return hipErrorInvalidValue;
    }
  } else if (l.stream_pieces) {
    // left-over slices fewer than the workgroups (so a range is shorter than a slice), and at
    // least one left-over block per workgroup
    const long long left = slices - static_cast<long long>(l.stream_grid) * l.stream_whole;
    if (l.counters == nullptr || l.partials == nullptr || slices > kStreamMaxSlices ||
        l.stream_whole < 0 || left <= 0 || left >= l.stream_grid ||
        left * (ng / quantum) < l.stream_grid ||
        left * (ng / quantum) * l.stream_grid >= (1LL << 31)) {
      return hipErrorInvalidValue;
    }
  } else if (l.stream_whole <= 0 ||
             static_cast<long long>(l.stream_whole) * l.stream_grid != slices) {
    return hipErrorInvalidValue;
  }
  switch (l.format) {
    case PacketFormat::kNativeSym: return stream_dispatch<PacketFormat::kNativeSym>(l, stream);
    case PacketFormat::kNativeAsym: return stream_dispatch<PacketFormat::kNativeAsym>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fk
