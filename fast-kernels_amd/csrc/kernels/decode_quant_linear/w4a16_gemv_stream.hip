// W4A16 GEMV over native slabs for one activation row: the persistent "stream" schedule.
//
// The native slabs of a buffer are laid out [slice][group] (w4a16_device.h), so the slices
// b * whole .. (b + 1) * whole - 1 are one contiguous byte range. When the 32-column slices divide
// evenly over one workgroup per CU (Llama-70B o, gate_up and down: 256, 1792 and 256 slices on
// 256 CUs), workgroup b streams that range without a break:
//
//  * The whole activation row is staged in LDS once per workgroup (dynamic LDS: K/G groups of
//    re-paired fp16 values and per-quarter sums, as native_stage_unit writes them) instead of
//    once per slice and chunk. Wave w only ever computes groups g = w (mod 8), so each wave
//    stages its own groups and no workgroup barrier separates staging from streaming. Staging
//    is spread over the first slice: one pass of the wave's groups before its first block, one
//    more after each block, so that the first weights are consumed as soon as they arrive.
//  * The staging loads are issued before the first weight loads, so the conversion overlaps
//    the weights' HBM latency (the load counter retires in order, so waiting for the activations
//    does not wait for the weights behind them).
//  * Wave w takes slabs w, w + 8, w + 16, ... of the range through D register buffers, and the
//    pipeline runs across slice boundaries: the loads of the next slice's first slabs are in
//    flight while a slice is reduced, so the stream does not drain at each slice as it does when
//    every slice is its own workgroup run.
//  * At a slice boundary each wave folds its lane partials over the column's four quarters,
//    writes them to one of two LDS slots and meets the others at a barrier (its loads stay in
//    flight); one wave, rotating with the slice, adds the eight waves' totals in wave order and
//    writes the 32 outputs. No slice is shared, so there is no fix-up and no workspace.
//
// Slices that do not divide evenly (Llama-70B qkv: 320 slices on 256 CUs) leave stream_grid *
// stream_whole slices to the whole ranges and cut each remaining "tail" slice into stream_parts
// pieces of stream_tail groups, one piece per workgroup (kTail): 1.25 slices per CU instead of
// one round of 256 slices and a second of 64. A workgroup streams its piece first, then its whole
// slices, so the hand-off of the piece is off the critical path:
//
//  * The piece's activations are staged first (one extra pass; the piece lies inside one pass).
//  * After the piece, the eight streaming waves write their totals to LDS and meet a ninth,
//    control wave at the barrier, and go on streaming. The control wave adds the totals, stores
//    the piece's 32 partial sums to the workspace, and bumps the tail slice's arrival counter
//    once they are acknowledged (agent scope); the workgroup that arrives last adds the parts' partials
//    in part order, so the result does not depend on arrival order, writes the 32 outputs and
//    resets the counter to zero for the next call. The control wave's waits (the store, the
//    counter's return, the partials' loads) stall no weight stream.
//  * With the logical-to-hardware workgroup remap the parts of one tail slice run on one XCD,
//    whose L2 then holds the partials the last part reads.
//
// Math per group is native_compute_group's (w4a16_gemv_native.h); results equal the per-slice
// kernel's up to fp32 summation order across waves.
#include "w4a16_gemv_native.h"

namespace fk {
namespace {

// LDS view of a whole staged activation row: xs [NG][G/8] re-paired fp16 words, sums [NG][4]
// per-quarter offset terms, scale [NG] bf16 staging scales (the layout of NativeSmem for one row
// and every group of K).
template <int G>
struct StreamLds {
  uint4* xs;
  float2* sums;
  float* scale;

  __device__ uint4 x_at(int, int gl, int i) const { return xs[gl * (G / 8) + i]; }
  __device__ float2 sums_at(int, int gl, int t) const { return sums[gl * 4 + t]; }
  __device__ float scale_at(int, int gl) const { return scale[gl]; }
  __device__ void set_x(int, int gl, int i, uint4 v) { xs[gl * (G / 8) + i] = v; }
  __device__ void set_sums(int, int gl, int t, float2 v) { sums[gl * 4 + t] = v; }
  __device__ void set_scale(int, int gl, float v) { scale[gl] = v; }
};

// kW waves per workgroup, D register buffers (slabs in flight) per wave: kW * D slabs of 2 KB
// (G = 128) or 1 KB (G = 64) in flight per workgroup, one workgroup per CU. kStageSlots passes
// of 64 / (G / 8) groups per wave stage K <= kStageSlots * 64 * kW * 8 activations.
template <int G, Act A, PacketFormat F, int kStageSlots, int kW, int D, bool kTail, bool kHalf>
__global__ void __launch_bounds__(64 * (kW + (kTail ? 1 : 0)), 1)
    w4a16_gemv_stream_kernel(GemvParams p) {
  extern __shared__ uint4 stream_lds[];
  __shared__ float red[2][kW][kSliceCols];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = lane / 16;
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  const int grid = static_cast<int>(gridDim.x);
  int b = static_cast<int>(blockIdx.x);
  // Consecutive logical workgroups on one XCD (the hardware deals workgroup b to XCD b % 8).
  if (p.xcd_remap) {
    b = (b & 7) * (grid >> 3) + (b >> 3);
  }
  const uint32_t ng = static_cast<uint32_t>(p.NG);
  const int whole = p.stream_whole;
  // The tail piece: groups gt0 .. gt0 + stream_tail - 1 of tail slice `tail_slice`.
  const int parts = kTail ? p.stream_parts : 1;
  const int tail_local = b / parts;
  const int part = b - tail_local * parts;
  const int tail_slice = grid * whole + tail_local;
  const int gt0 = part * p.stream_tail;
  if constexpr (kTail) {
    if (wave == kW) {
      // Control wave: finishes the tail piece, then meets the streaming waves at every slice's
      // barrier (s_barrier counts waves, not code locations).
      lds_barrier();
      if (lane < kSliceCols) {
        float v = red[0][0][lane];
#pragma unroll
        for (int w = 1; w < kW; ++w) {
          v += red[0][w][lane];
        }
        float* ws = p.partials + static_cast<size_t>(tail_local) * parts * kSliceCols;
        __hip_atomic_store(&ws[part * kSliceCols + lane], v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      // Hand-off without cache-wide fences (an agent-scope release writes back the whole L2 and
      // costs microseconds): the partials are agent-scope stores, which gfx950 writes through the
      // XCD's L2 to the memory-side coherence point; s_waitcnt vmcnt(0) holds the wave until all
      // of them are acknowledged there, and only then is the counter bumped. The last part's
      // loads are agent-scope too, so they miss the L2 and read the coherence point, after its
      // counter bump has returned the final count. Every part does the same, so whichever
      // arrives last sees all parts' partials.
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      uint32_t prev = 0;
      if (lane == 0) {
        prev = __hip_atomic_fetch_add(&p.counters[tail_local], 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
      }
      prev = __builtin_amdgcn_readfirstlane(prev);
      if (prev == static_cast<uint32_t>(parts - 1)) {
        if (lane < kSliceCols) {
          const float* ws = p.partials + static_cast<size_t>(tail_local) * parts * kSliceCols;
          float v = 0.0f;
          for (int q = 0; q < parts; ++q) {
            v += __hip_atomic_load(&ws[q * kSliceCols + lane], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          }
          p.out[static_cast<size_t>(tail_slice) * kSliceCols + lane] = float_to_act_bits<A>(v);
        }
        if (lane == 0) {
          __hip_atomic_store(&p.counters[tail_local], 0u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      for (int r = 0; r < whole; ++r) {
        lds_barrier();
      }
      return;
    }
  }

  StreamLds<G> sm;
  sm.xs = stream_lds;
  // K/G groups and one spare group slot (stage_one)
  sm.sums = reinterpret_cast<float2*>(stream_lds + static_cast<size_t>(p.NG + 1) * (G / 8));
  sm.scale = reinterpret_cast<float*>(sm.sums + static_cast<size_t>(p.NG + 1) * 4);

  // This wave's slabs: u0 + wave + kW j, j < n_w. Past its last slab a wave re-reads that slab,
  // so every buffer slot is loaded unconditionally (and never past the range).
  // kHalf: workgroup b streams half (b & 1) of slice b / 2 (one half-slice per workgroup).
  const int half = kHalf ? (b & 1) : 0;
  const uint32_t u0 = (kHalf ? static_cast<uint32_t>(b >> 1)
                             : static_cast<uint32_t>(b) * static_cast<uint32_t>(whole)) * ng;
  const int n_blk = static_cast<int>(ng) / (kW * D);  // blocks of D slabs per wave and slice
  const int n_t = kTail ? p.stream_tail / kW : 0;     // the wave's slabs of the tail piece
  const int n_w = n_t + whole * n_blk * D;
  const int j_last = n_w - 1;
  const uint8_t* base = p.packets + static_cast<size_t>(u0 + wave) * stride;
  const uint8_t* tail_base =
      p.packets + (static_cast<size_t>(tail_slice) * ng + gt0 + wave) * stride;
  const size_t step = static_cast<size_t>(kW) * stride;
  // The wave's slab i (clamped to its last): the tail piece's first, then the whole range. The
  // choice is uniform (a scalar select), so the pipeline has no branch.
  auto slab = [&](int i) -> const uint8_t* {
    const int c = min(i, j_last);
    if constexpr (kTail) {
      return c < n_t ? tail_base + static_cast<size_t>(c) * step
                     : base + static_cast<size_t>(c - n_t) * step;
    } else {
      return base + static_cast<size_t>(c) * step;
    }
  };
  auto load_slab = [&](NativeLoad<G>& ld, const uint8_t* ptr) {
    if constexpr (kHalf) {
      native_load_half<G, F>(ld, ptr, lane, half);
    } else {
      native_load<G, F>(ld, ptr, lane);
    }
  };

  // Activations: every pass's loads first. Pass i stages groups wave + kW (i * 64 / WR + l / WR)
  // (lane l, word row l % WR); pass 0 before the first block, one more after each block of the
  // first slice (pass i covers the wave's slabs 64 / WR * i .. of a slice, and a block needs D of
  // them), and any left after it.
  constexpr int WR = G / 8;
  constexpr int kGroupsPerPass = 64 / WR;
  const int n_pass = (p.NG / kW + kGroupsPerPass - 1) / kGroupsPerPass;
  uint4 raw[kStageSlots];
#pragma unroll
  for (int i = 0; i < kStageSlots; ++i) {
    // clamped and unconditional (a load under a branch waits for the one before it); slots past
    // the wave's passes and groups past the row are never staged
    const int g = min(wave + kW * (i * kGroupsPerPass + lane / WR), p.NG - 1);
    raw[i] = *reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(g) * G + (lane % WR) * 8);
  }
  // The pass holding the tail piece's groups, loaded once more into a register of its own (picking
  // it out of raw[] by a runtime index would put raw[] in scratch memory).
  uint4 raw_tail = make_uint4(0u, 0u, 0u, 0u);
  int g_tail = 0;
  if constexpr (kTail) {
    const int q = (gt0 / kW) / kGroupsPerPass;
    g_tail = min(wave + kW * (q * kGroupsPerPass + lane / WR), p.NG);
    raw_tail = *reinterpret_cast<const uint4*>(p.x + static_cast<size_t>(min(g_tail, p.NG - 1)) * G +
                                               (lane % WR) * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  NativeLoad<G> buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_slab(buf[d], slab(d));
    __builtin_amdgcn_sched_barrier(0);  // the same issue order as the refills in the loop
  }
  int staged = 0;
  // Stages the next pass from raw[0] and shifts the slots down (register moves; a runtime slot
  // index would put the slots in scratch memory).
  auto stage_one = [&]() {
    // Groups past the row (the wave's last pass may be partial) are staged into a spare group
    // slot past the row's, so the staging has no branch.
    const int g = min(wave + kW * (staged * kGroupsPerPass + lane / WR), p.NG);
    native_stage_unit<G, A, F>(sm, raw[0], 0, g, lane % WR);
#pragma unroll
    for (int i = 0; i + 1 < kStageSlots; ++i) {
      raw[i] = raw[i + 1];
    }
    ++staged;
    // The wave reads back only what it wrote: its LDS accesses complete in order, so a
    // wave-scope fence (no instruction) is all that keeps the compiler from hoisting the reads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  float y[1][2] = {{0.0f, 0.0f}};
  int j = 0;  // the wave's next slab to compute
  // A block of D slabs of slice-local groups gl0 .., kW apart. Each slice gives every wave n_blk
  // whole blocks (the host plans K/G as a multiple of kW * D), so the block loops have no branch:
  // the compiler's wait for a buffer is then the in-order count of the loads issued after it,
  // not a drain of the pipeline.
  auto block = [&](int gl0) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      native_compute_group<G, A, 1, F, StreamLds<G>, kHalf ? 1 : 2>(sm, buf[d], gl0 + kW * d, t,
                                                                    mask_lo, mask_hi, y, half);
      load_slab(buf[d], slab(j + d + D));
      // Issue the refill here, not after the block's later slabs: the scheduler would otherwise
      // sink every load below the block's arithmetic and drain the pipeline once per block.
      __builtin_amdgcn_sched_barrier(0);
    }
    j += D;
  };
  // Folds the lane partials over the column's four quarters (lanes n, n+16, n+32, n+48) into LDS
  // slot `slot` and meets the other waves; the loads of the next slabs stay in flight.
  auto reduce_slice = [&](int slot) {
    float y0 = y[0][0];
    float y1 = y[0][1];
    y0 += __shfl_xor(y0, 16);
    y0 += __shfl_xor(y0, 32);
    if constexpr (!kHalf) {
      y1 += __shfl_xor(y1, 16);
      y1 += __shfl_xor(y1, 32);
    }
    y[0][0] = 0.0f;
    y[0][1] = 0.0f;
    if (lane < 16) {
      red[slot][wave][lane] = y0;
      if constexpr (!kHalf) {
        red[slot][wave][lane + 16] = y1;
      }
    }
    lds_barrier();
  };
  if constexpr (kTail) {
    // Stage the pass holding the piece's groups, stream the piece, hand its totals to the control
    // wave. The regular passes later stage this one again, with the same values.
    native_stage_unit<G, A, F>(sm, raw_tail, 0, g_tail, lane % WR);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int blk = 0; blk < n_t / D; ++blk) {
      block(gt0 + wave + kW * D * blk);
    }
    reduce_slice(0);
  }
  stage_one();
  for (int r = 0; r < whole; ++r) {
    // Blocks that each stage one more pass, then blocks that do not: two loops, no branch in
    // either.
    const int n_staging = min(n_blk, n_pass - staged);
    int blk = 0;
    for (; blk < n_staging; ++blk) {
      block(wave + kW * D * blk);
      stage_one();
    }
    for (; blk < n_blk; ++blk) {
      block(wave + kW * D * blk);
    }
    while (staged < n_pass) {
      stage_one();
    }

    // Slot reuse is safe: a slot is written again only after the next slice's barrier, which the
    // wave reading it (below, or the control wave for the tail piece) reaches after reading.
    const int slot = (r + (kTail ? 1 : 0)) & 1;
    reduce_slice(slot);
    // One wave, rotating with the slice, writes it.
    constexpr int kCols = kHalf ? kSliceCols / 2 : kSliceCols;
    if (wave == (r & (kW - 1)) && lane < kCols) {
      float v = red[slot][0][lane];
#pragma unroll
      for (int w = 1; w < kW; ++w) {
        v += red[slot][w][lane];
      }
      const size_t col = kHalf ? static_cast<size_t>(b >> 1) * kSliceCols + 16 * half + lane
                               : (static_cast<size_t>(b) * whole + r) * kSliceCols + lane;
      p.out[col] = float_to_act_bits<A>(v);
    }
  }
  // Retire the loads of re-read tail slots before the workgroup ends.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

template <int G, Act A, PacketFormat F, int kStageSlots, int kW, int D>
hipError_t launch_stream_t(const GemvLaunch& l, hipStream_t stream) {
  int grid = 0;
  GemvParams p = native_params<G, 1>(l, &grid);
  p.pair = 0;
  p.stream_whole = l.stream_whole;
  p.stream_tail = l.stream_tail;
  p.stream_parts = l.stream_parts;
  grid = l.stream_grid;
  p.xcd_remap = grid % 8 == 0 ? 1 : 0;
  const size_t lds = stream_lds_bytes(G, l.K / G + 1);
  if (l.stream_tail > 0) {
    hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, true, false>),
                       dim3(grid), dim3(64 * (kW + 1)), lds, stream, p);
  } else if (l.stream_half) {
    if constexpr (G == 128) {
      hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, false, true>),
                         dim3(grid), dim3(64 * kW), lds, stream, p);
    } else {
      return hipErrorInvalidValue;
    }
  } else {
    hipLaunchKernelGGL((w4a16_gemv_stream_kernel<G, A, F, kStageSlots, kW, D, false, false>),
                       dim3(grid), dim3(64 * kW), lds, stream, p);
  }
  return hipGetLastError();
}

template <int G, Act A, PacketFormat F, int kW, int D>
hipError_t stream_dispatch_slots(const GemvLaunch& l, hipStream_t stream) {
  constexpr int kPerPass = 64 * kW * 8;  // activations staged per slot
  if (l.K <= kPerPass * (16 / kW)) {
    return launch_stream_t<G, A, F, 16 / kW, kW, D>(l, stream);
  }
  if (l.K <= kPerPass * (64 / kW)) {
    return launch_stream_t<G, A, F, 64 / kW, kW, D>(l, stream);
  }
  return hipErrorInvalidValue;
}

// Waves and depth: units_per_workgroup and K / G are multiples of stream_waves * stream_depth
// (the host plans them so).
template <int G, Act A, PacketFormat F>
hipError_t stream_dispatch_waves(const GemvLaunch& l, hipStream_t stream) {
  constexpr int kUnitKB = G == 128 ? 2 : 1;
  if (l.stream_waves != kStreamWaves) {
    return hipErrorInvalidValue;
  }
  switch (l.stream_depth * kUnitKB) {
    case 4: return stream_dispatch_slots<G, A, F, kStreamWaves, 4 / kUnitKB>(l, stream);
    case 8: return stream_dispatch_slots<G, A, F, kStreamWaves, 8 / kUnitKB>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

template <PacketFormat F>
hipError_t stream_dispatch(const GemvLaunch& l, hipStream_t stream) {
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? stream_dispatch_waves<64, Act::kF16, F>(l, stream)
                              : stream_dispatch_waves<64, Act::kBF16, F>(l, stream);
  }
  return l.act == Act::kF16 ? stream_dispatch_waves<128, Act::kF16, F>(l, stream)
                            : stream_dispatch_waves<128, Act::kBF16, F>(l, stream);
}

}  // namespace

hipError_t launch_w4a16_gemv_stream(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode != GemvMode::kStreamK || l.m_tile != 1 || l.M != 1 || l.fuse != GemvFuse::kNone ||
      l.slice_cols != kSliceCols || l.slice_pair || l.K > kStreamMaxK || l.stream_depth <= 0 ||
      l.stream_grid <= 0) {
    return hipErrorInvalidValue;
  }
  // Whole slices, the same count per workgroup, in blocks of waves * depth units; with a tail,
  // one piece per workgroup of the slices left over, lying inside one staging pass of the wave's
  // groups (64 / (G / 8) of them), with the workspace to finish them.
  const int ng = l.K / l.group_size;
  const int quantum = l.stream_waves * l.stream_depth;
  if (l.stream_whole < 0 || ng % quantum != 0) {
    return hipErrorInvalidValue;
  }
  const long long slices = l.N / kSliceCols;
  const long long whole_slices = static_cast<long long>(l.stream_whole) * l.stream_grid;
  if (l.stream_half) {
    // one half-slice (16 columns of a G = 128 slice) per workgroup
    if (l.group_size != 128 || l.stream_tail != 0 || l.stream_whole != 1 ||
        l.stream_grid != 2 * slices) {
      return hipErrorInvalidValue;
    }
  } else if (l.stream_tail == 0) {
    if (l.stream_whole == 0 || whole_slices != slices) {
      return hipErrorInvalidValue;
    }
  } else {
    const int pass_groups = l.stream_waves * (64 / (l.group_size / 8));
    if (l.stream_parts <= 0 || l.stream_grid % l.stream_parts != 0 ||
        l.stream_tail * l.stream_parts != ng || l.stream_tail % quantum != 0 ||
        pass_groups % l.stream_tail != 0 ||
        whole_slices + l.stream_grid / l.stream_parts != slices || l.counters == nullptr ||
        l.partials == nullptr) {
      return hipErrorInvalidValue;
    }
  }
  switch (l.format) {
    case PacketFormat::kNativeSym: return stream_dispatch<PacketFormat::kNativeSym>(l, stream);
    case PacketFormat::kNativeAsym: return stream_dispatch<PacketFormat::kNativeAsym>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fk
