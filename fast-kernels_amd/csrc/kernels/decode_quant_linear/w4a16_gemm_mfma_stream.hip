// W4A16 small-batch GEMM (2-16 activation rows) over native slabs or the reference packets on the
// gfx950 matrix cores, on the persistent stream schedule.
//
// The work split is the one-row stream kernel's (w4a16_stream_common.h): one workgroup per CU
// streams its whole 32-column slices as one contiguous range, plus pieces of the slices left
// over, handed off by a control wave. What changes is the arithmetic per slab:
//
//  * One v_mfma_f32_16x16x32_f16 multiplies A = 16 activation rows x 32 k by B = 32 k x 16
//    columns. A slab gives lane l = 16 t + n the U = G/32 code words of quarter t of columns n
//    and n + 16; MFMA window j takes word j of every lane (k-chunks {j, U + j, 2U + j, 3U + j}
//    of the group), so a slab is 2 U MFMAs: two 16-column halves times U windows, the halves
//    sharing each window's A operand. B is the unpacked words, 1024 + q (even k) and 64 + q (odd
//    k) in the slot order (0,4)(1,5)(2,6)(3,7); A is the activations paired in that order.
//  * The activation rows are staged once per workgroup in LDS (MT rows of K, MT = 4, 8 or 16;
//    rows past the batch are zeros), each wave staging the groups it computes (g = w mod 8), so no
//    barrier separates staging from streaming. All of a wave's staging loads are issued before
//    its first weight loads, and converted while those are in flight. The A operand of a window
//    is one ds_read_b128 per lane for all 16 rows, whatever the batch: the LDS traffic per slab is
//    U KB per wave (the dot2 kernel reads the activations once per row).
//  * Every MFMA chain starts from the group's seed, C = -1024 S_e - 64 S_o (kNativeSym: minus
//    8 (S_e + S_o) more, folding beta = -8 alpha), which cancels the unpack bias; the epilogue is
//    y += alpha D (+ beta S for kNativeAsym), with the bf16 staging scale where it applies. The
//    16 x 16 D tile gives lane l rows 4 t .. 4 t + 3 of column n of its half.
//  * At the end of a slice or piece each wave writes its partial tile (rows < M) to LDS and meets
//    the others; one wave (rotating with the slice, or the control wave for pieces) adds the
//    eight partials in wave order and writes the slice, and a second barrier frees the one LDS
//    slot (the activations of 16 rows leave no room for a second).
//  * Over the reference packets (kArc) the slices are the packets' 32-column quarters (slice
//    4 tile + q, so the output columns and the work split are the same): lane l = 16 t + n reads,
//    for window j, the 8 bytes of columns 32 q + 2 n and + 1 in word row 4 j + t (four 128-byte
//    runs per load) and those columns' alphas and betas; the two chains are the two columns, A
//    the staged k-chunk 4 j + t, and the epilogue y += alpha D + beta S with the packet's betas.
//  * kParts (rows too long to stage whole): K in stream_parts equal parts; workgroup b takes part
//    b / (grid / parts) of its whole slices, stages only that part's activations, and writes its
//    fp32 partial tiles to partials [parts, M, N]; add_parts_kernel then adds the parts in part
//    order and rounds once (no counters, no hand-off).
#include "w4a16_gemv_native.h"
#include "w4a16_stream_common.h"

#include <type_traits>

namespace fk {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// LDS of the MFMA stream kernel: xs [NG][G/8][MT] paired activation words (row fastest, the row
// slot swizzled by the word row: see xs_slot),
// sums [NG][MT] {-1024 S_e - 64 S_o, S_e + S_o}, scale [NG][MT] bf16 staging scales, then the
// reduction slot red [kW][MT][32].
template <int G, int MT>
struct MfmaStreamLds {
  uint4* xs;
  float2* sums;
  float* scale;
  float* red;
};

template <int G, int MT>
__host__ __device__ constexpr size_t mfma_stream_lds_bytes(int ng, int waves) {
  return static_cast<size_t>(ng) * MT * ((G / 8) * 16 + 8 + 4) +
         static_cast<size_t>(waves) * MT * kSliceCols * 4;
}

// Slot of row m in word row wr of xs. The staging's consecutive lanes store one row's
// consecutive word rows, MT * 16 bytes apart, which with MT slots per word row put 4-8 of every
// 8 lanes' 16-byte stores in the same banks; the row xor a function of the word row spreads
// them over distinct 16-byte slots of each 128 bytes (MT >= 8: wr mod 8; MT = 4: two word rows
// per 128 bytes, so (wr / 2) mod 4). The compute's reads (16 rows of one word row per 16 lanes)
// stay conflict-free: xor is a permutation of the word row's slots.
template <int MT>
__device__ __forceinline__ int xs_slot(int wr, int m) {
  return m ^ (MT >= 8 ? (wr & 7) : ((wr >> 1) & (MT - 1)));
}

// Code word -> 8 fp16 values in the slot order (k0,k4)(k1,k5)(k2,k6)(k3,k7): 1024 + q for even
// k, 64 + q for odd k. One shift, four and-or.
__device__ __forceinline__ half8_t unpack_word8(uint32_t w, uint32_t mask_lo, uint32_t mask_hi) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const uint32_t w8 = w >> 8;
  u32x4 v;
  v.x = (w & mask_lo) | kBiasLow;
  v.y = (w & mask_hi) | kBiasHigh;
  v.z = (w8 & mask_lo) | kBiasLow;
  v.w = (w8 & mask_hi) | kBiasHigh;
  return __builtin_bit_cast(half8_t, v);
}

// Word j of half i of the lane's unit (native_word_offset's layout).
template <int G>
__device__ __forceinline__ uint32_t slab_word(const NativeLoad<G>& ld, int i, int j) {
  if constexpr (G == 128) {
    const uint4 v = ld.w[i];
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
  } else {
    const uint4 v = ld.w[0];
    return i == 0 ? (j == 0 ? v.x : v.y) : (j == 0 ? v.z : v.w);
  }
}

// One 32-column quarter q of a reference packet (kArc) for the matrix cores: lane l = 16 t + n
// holds, for window j, the words of columns 32 q + 2 n and 32 q + 2 n + 1 in word row 4 j + t
// (8 bytes), and those two columns' alphas and betas.
template <int G>
struct ArcMfmaLoad {
  static constexpr int kWindows = G / 32;
  uint2 w[kWindows];
  uint32_t alpha;
  uint32_t beta;
};

template <int G>
__device__ __forceinline__ void arc_mfma_load(ArcMfmaLoad<G>& ld, const uint8_t* packet, int q,
                                              int t, int n) {
  const uint8_t* codes = packet + q * (kSliceCols * 4) + 8 * n;
#pragma unroll
  for (int j = 0; j < ArcMfmaLoad<G>::kWindows; ++j) {
    ld.w[j] = stream_load8(codes + (4 * j + t) * kWordRowBytes);
  }
  const uint8_t* scales = packet + kTileCols * G / 2 + q * (kSliceCols * 2) + 4 * n;
  ld.alpha = stream_load4(scales);
  ld.beta = stream_load4(scales + kTileCols * 2);
}

// Most staging loads per lane (a wave's groups x MT rows x G/8 word rows / 64 lanes): MT. The
// host keeps launches within it.
constexpr int max_stage_per_lane(int mt) { return mt; }

template <int G, Act A, PacketFormat F, int kW, int D, int MT, bool kPieces, bool kParts = false>
__global__ void __launch_bounds__(64 * (kW + (kPieces ? 1 : 0)), 1)
    w4a16_gemm_mfma_stream_kernel(GemvParams p) {
  static_assert(!(kPieces && kParts), "pieces or K parts, not both");
  extern __shared__ uint4 mfma_stream_lds[];
  constexpr int WR = G / 8;
  constexpr int U = native_unit_words(G);
  constexpr int Q = kW * D;           // groups per block
  constexpr int kOutMax = 16 * kSliceCols;
  constexpr int kPer = MT * kSliceCols / 64;  // outputs per lane of a slice (MT rows)
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = lane / 16;
  const int n = lane % 16;
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  const int grid = p.grid;
  int b = static_cast<int>(blockIdx.x);
  b = p.xcd_remap != 0 ? (b & 7) * p.xcd_remap + (b >> 3) : b;
  const int ng = p.NG;
  // kParts: workgroup b streams K part `part` (groups g0 .. g0 + ngs - 1 of every slice) of its
  // slices; the slice groups of one part are grid / parts consecutive workgroups.
  const int parts = kParts ? p.stream_parts : 1;
  const int ngs = ng / parts;  // groups staged, and streamed per slice
  int part = 0;
  if constexpr (kParts) {
    const int per_part = grid / parts;
    part = b / per_part;
    b -= part * per_part;
  }
  const int g0 = part * ngs;
  const int nbs = ngs / Q;
  const int slices = p.N / kSliceCols;
  const int rows = p.M;  // rows < MT are real, the rest zeros
  const int n_out = rows * kSliceCols;
  const StreamRange rg = stream_range(b, grid, p.stream_whole, slices, nbs, kPieces);
  constexpr bool kArcPk = F == PacketFormat::kArc;
  using Load = std::conditional_t<kArcPk, ArcMfmaLoad<G>, NativeLoad<G>>;

  MfmaStreamLds<G, MT> sm;
  sm.xs = mfma_stream_lds;
  sm.sums = reinterpret_cast<float2*>(sm.xs + static_cast<size_t>(ngs) * WR * MT);
  sm.scale = reinterpret_cast<float*>(sm.sums + static_cast<size_t>(ngs) * MT);
  sm.red = sm.scale + static_cast<size_t>(ngs) * MT;

  // Adds the waves' partial tiles of output o in wave order.
  auto total = [&](int o) __attribute__((always_inline)) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      s += sm.red[w * MT * kSliceCols + o];
    }
    return s;
  };

  if constexpr (kPieces) {
    if (wave == kW) {
      // Control wave: the pieces' totals first (two barriers each, the slot is then free), then
      // their hand-offs, then the whole slices' barriers.
      float v[2][kPer];
      const bool has[2] = {rg.head_len > 0, rg.tail_len > 0};
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        if (has[pc]) {
          lds_barrier();
#pragma unroll
          for (int i = 0; i < kPer; ++i) {
            const int o = lane + 64 * i;
            v[pc][i] = o < n_out ? total(o) : 0.0f;
          }
          lds_barrier();
        }
      }
      if (has[0]) {
        stream_hand_off<A, kPer>(p, b, 0, rg.head_slice, grid, p.stream_whole, slices, nbs,
                                 n_out, kOutMax, v[0], lane);
      }
      if (has[1]) {
        stream_hand_off<A, kPer>(p, b, 1, rg.tail_slice, grid, p.stream_whole, slices, nbs,
                                 n_out, kOutMax, v[1], lane);
      }
      for (int r = 0; r < rg.whole; ++r) {
        lds_barrier();
        lds_barrier();
      }
      return;
    }
  }

  // The wave's slabs: the head piece's, the tail piece's, then the whole slices' range (as in the
  // one-row stream kernel; re-reads past the last slab keep every load unconditional).
  const int n_h = rg.head_len * D;
  const int n_t = rg.tail_len * D;
  const int n_w = n_h + n_t + rg.whole * nbs * D;
  const int j_last = n_w - 1;
  const int off_w = rg.whole_slice0 * ng + wave - (n_h + n_t) * kW;
  const int off_t = rg.tail_slice * ng + wave - n_h * kW;
  const int off_h = rg.head_slice * ng + rg.head_blk0 * Q + wave;
  auto slab = [&](int i) __attribute__((always_inline)) -> const uint8_t* {
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
    return p.packets + static_cast<size_t>(static_cast<uint32_t>(c * kW + off)) * stride;
  };
  // kArc: the slab index slice * NG + group gives the slice by a multiply-high with a reciprocal
  // of NG (exact over the launch's indices, checked by the host), then packet (slice / 4) * NG +
  // group and quarter slice % 4.
  // kParts: the wave's slab i is group g0 + wave + kW gi of slice whole_slice0 + r (spw slabs of
  // the wave per slice), uniform 32-bit arithmetic.
  const int spw = ngs / kW;
  auto load_slab = [&](Load& ld, int i) __attribute__((always_inline)) {
    if constexpr (kParts) {
      const int c = __builtin_amdgcn_readfirstlane(min(i, j_last));
      const int r = static_cast<int>(static_cast<uint32_t>(c) / static_cast<uint32_t>(spw));
      const int gi = c - r * spw;
      const uint32_t sl = static_cast<uint32_t>(rg.whole_slice0 + r);
      const uint32_t g = static_cast<uint32_t>(g0 + wave + kW * gi);
      if constexpr (kArcPk) {
        const uint8_t* pk =
            p.packets + static_cast<size_t>((sl >> 2) * static_cast<uint32_t>(ng) + g) * stride;
        arc_mfma_load<G>(ld, pk, static_cast<int>(sl & 3), t, n);
      } else {
        native_load<G, F>(ld, p.packets + static_cast<size_t>(sl * ng + g) * stride, lane);
      }
    } else if constexpr (kArcPk) {
      const int c = min(i, j_last);
      int off = off_w;
      if constexpr (kPieces) {
        int in_t = c < n_h + n_t ? 1 : 0;
        int in_h = c < n_h ? 1 : 0;
        in_t = __builtin_amdgcn_readfirstlane(in_t);
        in_h = __builtin_amdgcn_readfirstlane(in_h);
        off += in_t * (off_t - off_w) + in_h * (off_h - off_t);
      }
      const uint32_t lin = static_cast<uint32_t>(c * kW + off);
      const uint32_t sl = __umulhi(lin, p.ng_magic);
      const uint32_t g = lin - sl * static_cast<uint32_t>(ng);
      const uint8_t* pk =
          p.packets + static_cast<size_t>((sl >> 2) * static_cast<uint32_t>(ng) + g) * stride;
      arc_mfma_load<G>(ld, pk, static_cast<int>(sl & 3), t, n);
    } else {
      native_load<G, F>(ld, slab(i), lane);
    }
  };

  // Staging: the wave's (group, row, word row) units, 64 a pass, groups g = wave + kW gi; a
  // group's MT * WR units are P consecutive lanes' worth (row and word row fastest), so a group's
  // WR word rows of one row are WR consecutive lanes (the per-(group, row) sums are xor-shuffles).
  // With P >= 64 a pass lies inside one group and its group and first row are compile-time
  // constants of the (unrolled) pass; with P = 32 a pass holds two groups, one per half-wave.
  // Either way a unit's address is a lane constant plus a uniform offset (the general division
  // form put some 600 instructions ahead of the first weight load).
  constexpr int P = MT * WR;
  constexpr int L = P < 64 ? P : 64;  // lanes per group in a pass
  constexpr int kGroupsPerPass = 64 / L;
  const int gsub = lane / L;
  const int m_l = (lane % L) / WR;
  const int wr = lane % WR;
  const int g_last = ngs / kW - 1;  // the wave's last group index
  // Group index and row of this lane's unit in pass i (i a compile-time constant). Passes past
  // the wave's last group stage that group again (the same values; the host bounds the passes).
  auto pass_group = [&](int i) __attribute__((always_inline)) {
    return P >= 64 ? min((i * 64) / P, g_last) : min(i * kGroupsPerPass + gsub, g_last);
  };
  auto pass_row = [&](int i) __attribute__((always_inline)) { return (P >= 64 ? ((i * 64) % P) / WR : 0) + m_l; };
  constexpr int kStage = max_stage_per_lane(MT);
  uint4 raw[kStage];
#pragma unroll
  for (int i = 0; i < kStage; ++i) {
    // every pass loads (a load under a branch waits for the one before it, and an early exit
    // spills raw[] to scratch)
    const int g = wave + kW * pass_group(i);
    const int m = min(pass_row(i), rows - 1);  // rows past the batch: read a real row, stage 0
    raw[i] = *reinterpret_cast<const uint4*>(p.x + (m * p.K + (g0 + g) * G + wr * 8));
  }
  __builtin_amdgcn_sched_barrier(0);
  Load buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_slab(buf[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  // Convert and store: rows past the batch stage zeros (a mask, not a branch); a pass past the
  // wave's last group stores that group's values again.
#pragma unroll
  for (int i = 0; i < kStage; ++i) {
    const int g = wave + kW * pass_group(i);
    const int m = pass_row(i);
    const uint32_t keep = m < rows ? 0xffffffffu : 0u;
    uint4 v = make_uint4(raw[i].x & keep, raw[i].y & keep, raw[i].z & keep, raw[i].w & keep);
    float undo = 1.0f;
    if constexpr (A == Act::kBF16) {
      const uint32_t e = group_max<WR>(bf16_max_mag(v)) >> 7;
      const int shift = bf16_stage_shift(e);
      const float sc = __builtin_bit_cast(float, static_cast<uint32_t>(127 - shift) << 23);
      undo = __builtin_bit_cast(float, static_cast<uint32_t>(127 + shift) << 23);
      v.x = bf16_pair_to_half_pair(v.x, sc);
      v.y = bf16_pair_to_half_pair(v.y, sc);
      v.z = bf16_pair_to_half_pair(v.z, sc);
      v.w = bf16_pair_to_half_pair(v.w, sc);
    }
    const uint4 xp = pair_activations(v);
    // even k: x0 x2 x4 x6 (xp.x, xp.z), odd k: x1 x3 x5 x7 (xp.y, xp.w)
    constexpr uint32_t kOnes = 0x3c003c00u;
    float se = dot2<Act::kF16>(xp.z, kOnes, dot2<Act::kF16>(xp.x, kOnes, 0.0f));
    float so = dot2<Act::kF16>(xp.w, kOnes, dot2<Act::kF16>(xp.y, kOnes, 0.0f));
    se = group_sum<WR>(se);
    so = group_sum<WR>(so);
    sm.xs[(g * WR + wr) * MT + xs_slot<MT>(wr, m)] = xp;
    // every lane of the (group, row) holds the same values and writes them (no branch)
    sm.sums[g * MT + m] = make_float2(fmaf(-1024.0f, se, -64.0f * so), se + so);
    if constexpr (A == Act::kBF16) {
      sm.scale[g * MT + m] = undo;
    }
  }
  // The wave reads back only what it wrote (its LDS accesses complete in order); the fences keep
  // the compiler from hoisting the reads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  float y[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      y[i][r] = 0.0f;
    }
  }
  const int r0 = 4 * t;  // D rows of this lane
  // The staged operands of slice-local group gl: the A windows, the chain seeds and the offset
  // sums of the lane's rows, and (bf16) their staging scales. A block reads the next slab's
  // while the current one's chains run, so the LDS latency is not on the slab's path.
  struct Op {
    half8_t a[U];
    float4_t seed;
    float s[4];
    float sc[4];
  };
  auto load_op = [&](int gl, Op& o) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < U; ++j) {
      // the k-chunk of window j for lane quarter t: U t + j (native slabs), 4 j + t (kArc)
      const int wr_j = kArcPk ? 4 * j + t : U * t + j;
      const uint4 xv = sm.xs[(static_cast<size_t>(gl) * WR + wr_j) * MT +
                             xs_slot<MT>(wr_j, min(n, MT - 1))];
      o.a[j] = __builtin_bit_cast(half8_t, n < MT ? xv : make_uint4(0u, 0u, 0u, 0u));
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = min(r0 + r, MT - 1);
      const float2 v = sm.sums[gl * MT + row];
      const bool live = r0 + r < MT;
      o.s[r] = live ? v.y : 0.0f;
      const float c = F == PacketFormat::kNativeSym ? fmaf(-8.0f, v.y, v.x) : v.x;
      o.seed[r] = live ? c : 0.0f;
      o.sc[r] = A == Act::kBF16 ? sm.scale[gl * MT + row] : 1.0f;
    }
  };
  // Slab of one group: 2 U MFMAs and the epilogue.
  // kArc: the two chains are the lane's columns 2 n and 2 n + 1, with the packet's betas.
  constexpr bool kBeta = F != PacketFormat::kNativeSym;
  auto compute = [&](const Load& ld, const Op& o) __attribute__((always_inline)) {
    const auto& a = o.a;
    const float4_t seed = o.seed;
    const auto& s = o.s;
    const auto& sc = o.sc;
    uint32_t beta_pair = 0;
    if constexpr (kArcPk) {
      beta_pair = ld.beta;
    } else if constexpr (F == PacketFormat::kNativeAsym) {
      beta_pair = __builtin_bit_cast(
          uint32_t, __builtin_bit_cast(half2_t, ld.alpha) * __builtin_bit_cast(half2_t, ld.zp));
    }
    float4_t dd[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dd[i] = seed;
#pragma unroll
      for (int j = 0; j < U; ++j) {
        uint32_t word;
        if constexpr (kArcPk) {
          word = i == 0 ? ld.w[j].x : ld.w[j].y;
        } else {
          word = slab_word<G>(ld, i, j);
        }
        dd[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], unpack_word8(word, mask_lo, mask_hi),
                                                       dd[i], 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float alpha = half_bits_to_float(static_cast<uint16_t>(ld.alpha >> (16 * i)));
      const float beta = half_bits_to_float(static_cast<uint16_t>(beta_pair >> (16 * i)));
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (A == Act::kBF16) {
          float tt = alpha * dd[i][r];
          if constexpr (kBeta) {
            tt = fmaf(beta, s[r], tt);
          }
          y[i][r] = fmaf(tt, sc[r], y[i][r]);
        } else {
          y[i][r] = fmaf(alpha, dd[i][r], y[i][r]);
          if constexpr (kBeta) {
            y[i][r] = fmaf(beta, s[r], y[i][r]);
          }
        }
      }
    }
  };
  int j = 0;
  // refill = false: the wave's last block (refills past it would only re-read its last slab and
  // hold the wave one memory latency past its last arithmetic).
  // One slab of a block: compute with `cur` (its operands), then read the next slab's into `nxt`
  // ahead of the refill.
  auto step = [&](int d, int gl0, const Op& cur, Op& nxt, auto refill)
      __attribute__((always_inline)) {
    if (d + 1 < D) {
      load_op(gl0 + kW * (d + 1), nxt);
    }
    compute(buf[d], cur);
    if constexpr (decltype(refill)::value) {
      load_slab(buf[d], j + d + D);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(D % 2 == 0, "slabs in pairs: the operand registers alternate");
  auto block_r = [&](int gl0, auto refill) __attribute__((always_inline)) {
    if constexpr (kPieces) {
      // (with pieces the prefetch registers push the kernel into scratch memory)
#pragma unroll
      for (int d = 0; d < D; ++d) {
        Op op;
        load_op(gl0 + kW * d, op);
        compute(buf[d], op);
        if constexpr (decltype(refill)::value) {
          load_slab(buf[d], j + d + D);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      Op op0;
      Op op1;
      load_op(gl0, op0);
#pragma unroll
      for (int d = 0; d < D; d += 2) {
        step(d, gl0, op0, op1, refill);
        step(d + 1, gl0, op1, op0, refill);
      }
    }
    j += D;
  };
  auto block = [&](int gl0) __attribute__((always_inline)) { block_r(gl0, std::true_type{}); };
  // The wave's partial tile (rows < M) into the slot, then the first barrier.
  auto reduce = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (r0 + r < MT) {
          sm.red[(wave * MT + r0 + r) * kSliceCols + (kArcPk ? 2 * n + i : 16 * i + n)] = y[i][r];
        }
        y[i][r] = 0.0f;
      }
    }
    lds_barrier();
  };

  if constexpr (kPieces) {
    for (int blk = 0; blk < rg.head_len; ++blk) {
      block((rg.head_blk0 + blk) * Q + wave);
    }
    if (rg.head_len > 0) {
      reduce();
      lds_barrier();  // the control wave has read the slot
    }
    for (int blk = 0; blk < rg.tail_len; ++blk) {
      block(blk * Q + wave);
    }
    if (rg.tail_len > 0) {
      reduce();
      lds_barrier();
    }
  }
  for (int r = 0; r < rg.whole; ++r) {
    const int n_loop = r == rg.whole - 1 ? nbs - 1 : nbs;
    for (int blk = 0; blk < n_loop; ++blk) {
      block(blk * Q + wave);
    }
    if (r == rg.whole - 1) {
      block_r((nbs - 1) * Q + wave, std::false_type{});
    }
    reduce();
    if (wave == (r & (kW - 1))) {
      const size_t slice = static_cast<size_t>(rg.whole_slice0) + r;
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int o = lane + 64 * i;
        if (o < n_out) {
          const size_t at =
              static_cast<size_t>(o / kSliceCols) * p.N + slice * kSliceCols + o % kSliceCols;
          if constexpr (kParts) {
            p.partials[static_cast<size_t>(part) * p.M * p.N + at] = total(o);
          } else {
            p.out[at] = float_to_act_bits<A>(total(o));
          }
        }
      }
    }
    lds_barrier();  // the slot is free again
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
}

// The K parts' partial sums added in part order and rounded once: out[i] = act(sum_p parts[p][i]).
template <Act A>
__global__ void __launch_bounds__(256) add_parts_kernel(const float* __restrict__ parts,
                                                        uint16_t* __restrict__ out, int total,
                                                        int n_parts) {
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i >= total) {
    return;
  }
  float v = 0.0f;
  for (int q = 0; q < n_parts; ++q) {
    v += parts[static_cast<size_t>(q) * total + i];
  }
  out[i] = float_to_act_bits<A>(v);
}

template <int G, Act A, PacketFormat F, int MT>
hipError_t launch_mfma_stream_t(const GemvLaunch& l, hipStream_t stream) {
  constexpr int D = stream_depth_for_kb(G, kStreamKB);
  int grid = 0;
  GemvParams p = native_params<G, 1>(l, &grid);
  p.pair = 0;
  p.stream_whole = l.stream_whole;
  grid = l.stream_grid;
  p.grid = grid;
  p.xcd_remap = grid % 8 == 0 ? grid / 8 : 0;
  p.ng_magic = l.ng_magic;
  p.stream_parts = l.stream_parts;
  const size_t lds = mfma_stream_lds_bytes<G, MT>(l.K / G / l.stream_parts, kStreamWaves);
  if (l.stream_parts > 1) {
    hipLaunchKernelGGL((w4a16_gemm_mfma_stream_kernel<G, A, F, kStreamWaves, D, MT, false, true>),
                       dim3(grid), dim3(64 * kStreamWaves), lds, stream, p);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
      return err;
    }
    const int total = l.M * l.N;
    hipLaunchKernelGGL(add_parts_kernel<A>, dim3((total + 255) / 256), dim3(256), 0, stream,
                       static_cast<const float*>(l.partials), static_cast<uint16_t*>(l.out), total,
                       l.stream_parts);
    return hipGetLastError();
  }
  if (l.stream_pieces) {
    // (over the reference packets the pieces' registers spill: whole slices only)
    if constexpr (F != PacketFormat::kArc) {
      hipLaunchKernelGGL((w4a16_gemm_mfma_stream_kernel<G, A, F, kStreamWaves, D, MT, true>),
                         dim3(grid), dim3(64 * (kStreamWaves + 1)), lds, stream, p);
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((w4a16_gemm_mfma_stream_kernel<G, A, F, kStreamWaves, D, MT, false>),
                     dim3(grid), dim3(64 * kStreamWaves), lds, stream, p);
  return hipGetLastError();
}

template <int G, Act A, PacketFormat F>
hipError_t mfma_stream_rows(const GemvLaunch& l, hipStream_t stream) {
  if (l.M <= 4) return launch_mfma_stream_t<G, A, F, 4>(l, stream);
  if (l.M <= 8) return launch_mfma_stream_t<G, A, F, 8>(l, stream);
  return launch_mfma_stream_t<G, A, F, 16>(l, stream);
}

template <PacketFormat F>
hipError_t mfma_stream_dispatch(const GemvLaunch& l, hipStream_t stream) {
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? mfma_stream_rows<64, Act::kF16, F>(l, stream)
                              : mfma_stream_rows<64, Act::kBF16, F>(l, stream);
  }
  return l.act == Act::kF16 ? mfma_stream_rows<128, Act::kF16, F>(l, stream)
                            : mfma_stream_rows<128, Act::kBF16, F>(l, stream);
}

}  // namespace

int mfma_stream_rows_for_batch(int batch) { return batch <= 4 ? 4 : batch <= 8 ? 8 : 16; }

size_t mfma_stream_lds(int group_size, int k, int batch) {
  const int mt = mfma_stream_rows_for_batch(batch);
  const int ng = k / group_size;
  const int wr = group_size / 8;
  return static_cast<size_t>(ng) * mt * (wr * 16 + 8 + 4) +
         static_cast<size_t>(kStreamWaves) * mt * kSliceCols * 4;
}

bool mfma_stream_fits(int group_size, int k, int batch) {
  const int mt = mfma_stream_rows_for_batch(batch);
  const int units_per_lane = ((k / group_size / kStreamWaves) * mt * (group_size / 8) + 63) / 64;
  return (k / group_size) % kStreamWaves == 0 && units_per_lane <= max_stage_per_lane(mt);
}

hipError_t launch_w4a16_gemm_mfma_stream(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode != GemvMode::kStreamK || !l.stream || l.m_tile != kMfmaRows || l.M < 1 ||
      l.M > kMfmaRows || l.fuse != GemvFuse::kNone || l.slice_cols != kSliceCols ||
      l.stream_half || l.stream_grid <= 0 || l.stream_parts < 1 ||
      (l.stream_parts == 1 && !mfma_stream_fits(l.group_size, l.K, l.M))) {
    return hipErrorInvalidValue;
  }
  const int ng = l.K / l.group_size;
  const int quantum = l.stream_waves * l.stream_depth;
  if (l.stream_waves != kStreamWaves ||
      l.stream_depth != stream_depth_for_kb(l.group_size, kStreamKB) || ng % quantum != 0) {
    return hipErrorInvalidValue;
  }
  const long long slices = l.N / kSliceCols;
  if (l.stream_parts > 1) {
    // K parts: whole blocks per part, the part's rows fit the staging, every part has the same
    // slice groups, and the partials [parts, M, N] in the workspace
    const int ngs = ng / l.stream_parts;
    if (l.stream_pieces || ng % l.stream_parts != 0 || ngs % quantum != 0 ||
        !mfma_stream_fits(l.group_size, ngs * l.group_size, l.M) ||
        l.stream_grid % l.stream_parts != 0 || l.stream_whole <= 0 ||
        static_cast<long long>(l.stream_grid / l.stream_parts) * l.stream_whole != slices ||
        l.partials == nullptr || static_cast<long long>(l.M) * l.N >= (1LL << 31)) {
      return hipErrorInvalidValue;
    }
    switch (l.format) {
      case PacketFormat::kNativeSym: return mfma_stream_dispatch<PacketFormat::kNativeSym>(l, stream);
      case PacketFormat::kNativeAsym: return mfma_stream_dispatch<PacketFormat::kNativeAsym>(l, stream);
      case PacketFormat::kArc: return mfma_stream_dispatch<PacketFormat::kArc>(l, stream);
      default: return hipErrorInvalidValue;
    }
  }
  if (l.stream_parts != 1) {
    return hipErrorInvalidValue;
  }
  if (l.format == PacketFormat::kArc &&
      (l.ng_magic != arc_quarter_magic(ng) || !arc_quarter_magic_exact(ng, slices))) {
    return hipErrorInvalidValue;
  }
  if (l.stream_pieces) {
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
    case PacketFormat::kNativeSym: return mfma_stream_dispatch<PacketFormat::kNativeSym>(l, stream);
    case PacketFormat::kNativeAsym: return mfma_stream_dispatch<PacketFormat::kNativeAsym>(l, stream);
    case PacketFormat::kArc: return mfma_stream_dispatch<PacketFormat::kArc>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fk
