// Work split and piece hand-off shared by the persistent stream kernels over native slabs
// (w4a16_gemv_stream.hip: one row on the dot2 path; w4a16_gemm_mfma_stream.hip: up to 16 rows on
// the matrix cores).
//
// With one workgroup per CU, workgroup b streams the stream_whole slices b * stream_whole .. as
// one contiguous range (the slabs are [slice][group]). The slices left over past grid *
// stream_whole (fewer than the workgroups) are cut into blocks of (waves x slabs in flight) groups
// and dealt as equal contiguous block ranges, each shorter than a slice: a head piece (the end of
// a slice an earlier workgroup starts) and a tail piece (the start of a slice a later workgroup
// finishes). A piece's partial sums go to the workspace (slot 2 b + piece); the slice's last
// part to arrive adds all parts in workgroup order and writes the outputs.
#pragma once

#include "w4a16_gemv_kernels.h"

namespace fk {

struct StreamRange {
  int head_slice, head_blk0, head_len;  // head piece: blocks head_blk0 .. of head_slice
  int tail_slice, tail_len;             // tail piece: the first tail_len blocks of tail_slice
  int whole_slice0, whole;              // whole slices whole_slice0 ..
};

// First left-over block of workgroup b (left-over blocks numbered from 0). 32-bit arithmetic: the
// host bounds grid * total below 2^31 (a 64-bit division costs hundreds of instructions).
__device__ __forceinline__ int range_start(int b, int total, int grid) {
  return static_cast<int>(static_cast<uint32_t>(b * total) / static_cast<uint32_t>(grid));
}

// Workgroup owning left-over block x: the last b with range_start(b) <= x.
__device__ __forceinline__ int range_owner(int x, int total, int grid) {
  return static_cast<int>(static_cast<uint32_t>((x + 1) * grid - 1) / static_cast<uint32_t>(total));
}

// The pieces of workgroup b's left-over range; slice s0 is the first left-over slice.
__device__ __forceinline__ void stream_pieces(StreamRange& r, int b, int total, int grid, int nbs,
                                              int s0) {
  const int blk0 = range_start(b, total, grid);
  const int blk1 = range_start(b + 1, total, grid);
  const int q0 = blk0 / nbs;
  const int off0 = blk0 - q0 * nbs;
  r.head_slice = s0 + q0;
  r.head_blk0 = off0;
  r.head_len = off0 != 0 ? min(blk1, blk0 - off0 + nbs) - blk0 : 0;
  const int c = blk0 + r.head_len;  // a slice start, or blk1
  // the range is shorter than a slice, so what follows the head piece is the start of one slice
  r.tail_slice = s0 + c / nbs;
  r.tail_len = blk1 - c;
}

// Workgroup b's parts: whole slices, and with pieces its share of the left-over slices.
__device__ __forceinline__ StreamRange stream_range(int b, int grid, int whole, int slices,
                                                    int nbs, bool pieces) {
  StreamRange r;
  r.head_slice = 0;
  r.head_blk0 = 0;
  r.head_len = 0;
  r.tail_slice = 0;
  r.tail_len = 0;
  r.whole_slice0 = b * whole;
  r.whole = whole;
  if (pieces) {
    const int s_left = grid * whole;
    stream_pieces(r, b, (slices - s_left) * nbs, grid, nbs, s_left);
  }
  return r;
}

// Hands off piece pc (0 head, 1 tail) of workgroup b, slice `slice` (kCols columns: a 32-column
// slice of native slabs, or a 128-column tile of reference packets): kPer values per lane, value
// i being output o = lane + 64 i of the slice's rows x kCols outputs (o < n_out; output o is row
// o / kCols, column o % kCols). Called by one wave. Slot size: slot_floats per (workgroup, piece).
//
// Hand-off without cache-wide fences (an agent-scope release writes back the whole L2 and costs
// microseconds): the partials are agent-scope stores, which gfx950 writes through the XCD's L2 to
// the memory-side coherence point; s_waitcnt vmcnt(0) holds the wave until all of them are
// acknowledged there, and only then is the counter bumped. The last part's loads are agent-scope
// too, so they miss the L2 and read the coherence point, after its counter bump has returned the
// final count. Every part does the same, so whichever arrives last sees all parts' partials.
template <Act A, int kPer, int kCols = kSliceCols>
__device__ __forceinline__ void stream_hand_off(const GemvParams& p, int b, int pc, int slice,
                                                int grid, int whole, int slices, int nbs,
                                                int n_out, int slot_floats, const float (&v)[kPer],
                                                int lane) {
  float* mine = p.partials + (static_cast<size_t>(b) * 2 + pc) * slot_floats;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int o = lane + 64 * i;
    if (o < n_out) {
      __hip_atomic_store(&mine[o], v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  // The waitcnt builtin is no compiler barrier: a signal fence (no instruction) keeps the
  // compiler from moving the partial stores past the counter bump below.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // Parts of the slice: the workgroups owning its first and last left-over block.
  const int s_left = grid * whole;
  const int left_blocks = (slices - s_left) * nbs;
  const int s0 = (slice - s_left) * nbs;
  const int b_first = range_owner(s0, left_blocks, grid);
  const int b_last = range_owner(s0 + nbs - 1, left_blocks, grid);
  uint32_t prev = 0;
  if (lane == 0) {
    prev = __hip_atomic_fetch_add(&p.counters[slice], 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  }
  prev = __builtin_amdgcn_readfirstlane(prev);
  if (prev != static_cast<uint32_t>(b_last - b_first)) {
    return;
  }
  // and the partial loads of the last part ahead of its counter bump
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  float acc[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    acc[i] = 0.0f;
  }
  for (int bb = b_first; bb <= b_last; ++bb) {
    // The slice is the head piece of a workgroup whose range starts inside it.
    const int pp = range_start(bb, left_blocks, grid) > s0 ? 0 : 1;
    const float* part = p.partials + (static_cast<size_t>(bb) * 2 + pp) * slot_floats;
    // unconditional loads from clamped offsets (a load under a branch waits for the one before)
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int o = min(lane + 64 * i, n_out - 1);
      acc[i] += __hip_atomic_load(&part[o], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int o = lane + 64 * i;
    if (o < n_out) {
      p.out[static_cast<size_t>(o / kCols) * p.N + static_cast<size_t>(slice) * kCols +
            o % kCols] = float_to_act_bits<A>(acc[i]);
    }
  }
  if (lane == 0) {
    __hip_atomic_store(&p.counters[slice], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace fk
