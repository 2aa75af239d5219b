// W4A16 small-batch GEMM (8-16 activation rows) on the gfx950 matrix cores.
//
// Same math and packet formats as w4a16_gemv.hip; with 8 or more rows the dot2 loop there is bound
// by VALU issue (four v_dot2 per code word per row), so here the products run on
// v_mfma_f32_16x16x32_f16 and the VALU only unpacks nibbles:
//
//  * One MFMA multiplies A = 16 activation rows x 32 k by B = 32 k x 16 output columns. Lane l
//    supplies A row l % 16 and B column l % 16, both for k = 8*(l / 16) .. +7, i.e. one code word
//    per lane. A wave-wide dwordx4 load gives lane l the words of 4 consecutive columns
//    (4*(l % 16) + j, j = 0..3) of word row l / 16, so 4 MFMAs (one per j) cover 64 columns x
//    4 word rows; MFMA j's output column c maps to packet column 4*c + j.
//  * A code word unpacks into the fp16 values 1024 + q (even k) and 64 + q (odd k) in the k
//    order (0,4)(1,5)(2,6)(3,7), one shift and four and-or; the staged activations are paired in
//    that order, so A and B agree slot by slot.
//  * Every block's MFMA chain starts from C = -1024 S_e - 64 S_o (S_e, S_o: the group's even- and
//    odd-k activation sums), which cancels the unpack bias, so the group's scale and offset are
//    applied once per (group, row, column) as y += alpha * D + beta * (S_e + S_o); kNativeSym
//    (beta = -8 alpha) also folds -8 (S_e + S_o) into C and is left with y += alpha * D.
//  * Work split, XCD remap and the cross-workgroup fix-up are those of the GEMV kernel
//    (stream-K over (tile, group) units, last contributor finishes the tile).
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "w4a16_device.h"
#include "w4a16_gemv.h"

namespace fk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = kMfmaRows;  // activation rows per m-tile (MFMA M)
constexpr int kWordRowBytes = kTileCols * 4;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

template <int G>
struct MfmaSmem {
  static constexpr int kWordRows = G / 8;
  static constexpr int kChunk = 1024 / G;  // groups staged per barrier (16 KB of activations)
  // Paired fp16 activations, row fastest; one spare row per word row staggers the LDS banks of
  // the staging stores (consecutive lanes store consecutive word rows of one activation row).
  uint4 xs[kChunk][kWordRows][kRows + 1];
  // per (group, row) of the staged activations: {-1024 S_even - 64 S_odd, S_even + S_odd}
  float2 sums[kChunk][kRows];
  float scale[kChunk][kRows];              // power of two undoing the bf16 staging scale
  float red[kWaves][kRows][kTileCols];     // cross-wave reduction
  int last;
};

struct MfmaParams {
  const uint16_t* x;
  const uint8_t* packets;
  uint16_t* out;
  float* partials;
  uint32_t* counters;
  int M, N, K, NG, tiles, mtiles, per, max_contrib;
  int grid;       // workgroups of the launch (gridDim would be a second, dependent argument load)
  int xcd_remap;  // grid / 8 when consecutive logical workgroups are kept on one XCD, else 0
};

template <int G>
struct MfmaStage {
  static constexpr int kUnits = MfmaSmem<G>::kChunk * (G / 8) * kRows;
  static constexpr int kPerThread = kUnits / kThreads;
  uint4 raw[kPerThread];
  bool ok[kPerThread];  // the unit lies inside the chunk and the batch (else it stages zeros)
};

// Unit u = ((row * kChunk) + gl) * WR + w: word rows of one (row, group) are consecutive, so the
// global loads are contiguous and the per-(row, group) reductions are xor-shuffles within WR lanes.
template <int G>
__device__ __forceinline__ void mfma_stage_load(MfmaStage<G>& st, const MfmaParams& p, int row0,
                                                int g0, int n_chunk) {
  constexpr int WR = G / 8;
  constexpr int kChunk = MfmaSmem<G>::kChunk;
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < MfmaStage<G>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunk;
    const int r = u / (WR * kChunk);
    // unconditional loads from clamped addresses (a branch per load serialises them); units
    // outside the chunk or the batch are zeroed in mfma_stage_store
    st.ok[it] = gl < n_chunk && row0 + r < p.M;
    st.raw[it] = *reinterpret_cast<const uint4*>(
        p.x + static_cast<size_t>(min(row0 + r, p.M - 1)) * p.K +
        static_cast<size_t>(g0 + min(gl, n_chunk - 1)) * G + w * 8);
  }
}

template <int G, Act A>
__device__ __forceinline__ void mfma_stage_store(MfmaSmem<G>& sm, MfmaStage<G>& st, int n_chunk) {
  constexpr int WR = G / 8;
  constexpr int kChunk = MfmaSmem<G>::kChunk;
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < MfmaStage<G>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunk;
    const int r = u / (WR * kChunk);
    if (gl >= n_chunk) {
      continue;  // past a short chunk: never read
    }
    if (!st.ok[it]) {
      // A row past the batch: zeros, without the conversions (a group's WR lanes share r and gl,
      // so the cross-lane sums below only ever combine live lanes).
      sm.xs[gl][w][r] = make_uint4(0u, 0u, 0u, 0u);
      if (w == 0) {
        sm.sums[gl][r] = make_float2(0.0f, 0.0f);
        sm.scale[gl][r] = 1.0f;
      }
      continue;
    }
    uint4 v = st.raw[it];
    float undo = 1.0f;
    if constexpr (A == Act::kBF16) {
      const uint32_t e = group_max<WR>(bf16_max_mag(v)) >> 7;
      const int shift = bf16_stage_shift(e);
      const float s = __builtin_bit_cast(float, static_cast<uint32_t>(127 - shift) << 23);
      undo = __builtin_bit_cast(float, static_cast<uint32_t>(127 + shift) << 23);
      v.x = bf16_pair_to_half_pair(v.x, s);
      v.y = bf16_pair_to_half_pair(v.y, s);
      v.z = bf16_pair_to_half_pair(v.z, s);
      v.w = bf16_pair_to_half_pair(v.w, s);
    }
    // even k: low halves, odd k: high halves
    float se = 0.0f;
    float so = 0.0f;
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      se += half_bits_to_float(static_cast<uint16_t>(words[q]));
      so += half_bits_to_float(static_cast<uint16_t>(words[q] >> 16));
    }
    se = group_sum<WR>(se);
    so = group_sum<WR>(so);
    {
      // Staged as they are: the high-nibble unpack is 64 + q (see unpack_word).
      const uint4 xp = pair_activations(v);
      sm.xs[gl][w][r] = xp;
      if (w == 0) {
        sm.sums[gl][r] = make_float2(fmaf(-1024.0f, se, -64.0f * so), se + so);
        sm.scale[gl][r] = undo;
      }
    }
  }
}

template <int G>
struct MfmaGroupLoad {
  static constexpr int KB = G / 32;  // MFMA k-blocks per group
  uint4 w[2][KB];                    // [half of the tile][k-block]
  uint2 alpha[2];
  uint2 beta[2];  // kArc: 4 fp16 offsets; kNativeAsym: (-zp) fp16 pairs of slabs 2h (.x), 2h+1 (.y)
};

// packet: the group's reference packet (kArc), or its slab of slice 0 (native formats: the slab
// of slice s is slice_step bytes further on).
template <int G, PacketFormat F>
__device__ __forceinline__ void mfma_load_group(MfmaGroupLoad<G>& gl, const uint8_t* packet,
                                                size_t slice_step, int lane) {
  const int col4 = 4 * (lane % 16);
  if constexpr (is_native(F)) {
    // Slab s (slice s of the tile) gives this lane the quarter t = lane / 16 of its columns
    // n = lane % 16 and n + 16: G = 128 two 16-byte units (w[s/2][2*(s%2) + i]), G = 64 one
    // 16-byte vector holding both units (w[s/2][s%2]).
    (void)col4;
#pragma unroll
    for (int s = 0; s < kSlicesPerTile; ++s) {
      const uint8_t* slab = packet + static_cast<size_t>(s) * slice_step;
      const uint8_t* record = slab + native_record_offset(G) + native_record_bytes(F) * (lane % 16);
      uint32_t pair = 0;
      if constexpr (F == PacketFormat::kNativeAsym) {
        const uint2 r = stream_load8(record);
        pair = r.x;
        if (s % 2 == 0) {
          gl.beta[s / 2].x = r.y;
        } else {
          gl.beta[s / 2].y = r.y;
        }
      } else {
        pair = stream_load4(record);
      }
      if (s % 2 == 0) {
        gl.alpha[s / 2].x = pair;
      } else {
        gl.alpha[s / 2].y = pair;
      }
      if constexpr (G == 128) {
        gl.w[s / 2][2 * (s % 2)] = stream_load16(slab + lane * 16);
        gl.w[s / 2][2 * (s % 2) + 1] = stream_load16(slab + 1024 + lane * 16);
      } else {
        gl.w[s / 2][s % 2] = stream_load16(slab + lane * 16);
      }
    }
  } else {
    constexpr int QB = kTileCols * G / 2;
    const int code = (lane / 16) * kWordRowBytes + col4 * 4;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      gl.alpha[h] = stream_load8(packet + QB + (h * 64 + col4) * 2);
      gl.beta[h] = stream_load8(packet + QB + kTileCols * 2 + (h * 64 + col4) * 2);
#pragma unroll
      for (int kb = 0; kb < MfmaGroupLoad<G>::KB; ++kb) {
        gl.w[h][kb] = stream_load16(packet + code + kb * 4 * kWordRowBytes + h * 256);
      }
    }
  }
}

// Code word -> 8 fp16 values in the slot order (k0,k4)(k1,k5)(k2,k6)(k3,k7): 1024 + q for even
// k, 64 + q for odd k. One shift, four and-or.
__device__ __forceinline__ half8_t unpack_word(uint32_t w, uint32_t mask_lo, uint32_t mask_hi) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const uint32_t w8 = w >> 8;
  u32x4 v;
  v.x = (w & mask_lo) | kBiasLow;
  v.y = (w & mask_hi) | kBiasHigh;
  v.z = (w8 & mask_lo) | kBiasLow;
  v.w = (w8 & mask_hi) | kBiasHigh;
  return __builtin_bit_cast(half8_t, v);
}

template <int G, Act A, PacketFormat F>
__device__ __forceinline__ void mfma_compute_group(const MfmaSmem<G>& sm, const MfmaGroupLoad<G>& ld,
                                                   int gl, int lane, uint32_t mask_lo,
                                                   uint32_t mask_hi, float (&y)[2][4][4]) {
  constexpr int KB = MfmaGroupLoad<G>::KB;
  const int r0 = 4 * (lane / 16);  // output rows r0 .. r0+3 of this lane
  float4 sc4 = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
  if constexpr (A == Act::kBF16) {
    sc4 = *reinterpret_cast<const float4*>(&sm.scale[gl][r0]);
  }
  const float sc[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
  // Every block's MFMA chain starts from the rows' unpack bias (kNativeSym: and its offset
  // beta = -8 alpha, i.e. -1032 S_e - 72 S_o), so the epilogue is alpha * D (+ beta * S).
  float s[4];
  float4_t seed;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float2 v = sm.sums[gl][r0 + r];
    s[r] = v.y;
    seed[r] = F == PacketFormat::kNativeSym ? fmaf(-8.0f, v.y, v.x) : v.x;
  }
  // y += sc * (alpha * d + beta * s): the offset term is absent for kNativeSym.
  auto apply = [&](float& acc, float alpha, float beta, float d, int r) {
    if constexpr (A == Act::kBF16) {
      float t = alpha * d;
      if constexpr (F != PacketFormat::kNativeSym) {
        t = fmaf(beta, s[r], t);
      }
      acc = fmaf(t, sc[r], acc);
    } else {
      acc = fmaf(alpha, d, acc);
      if constexpr (F != PacketFormat::kNativeSym) {
        acc = fmaf(beta, s[r], acc);
      }
    }
  };
  if constexpr (is_native(F)) {
    // Block (slab s, half i) = columns 32 s + 16 i + (lane % 16); its U MFMAs j multiply the
    // lane's unit word j (k-chunk lane / 16 of the window {j, U + j, 2U + j, 3U + j}) by the
    // activations of word U * (lane / 16) + j, all into one accumulator.
    constexpr int U = native_unit_words(G);
    half8_t a[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      a[j] = __builtin_bit_cast(half8_t, sm.xs[gl][U * (lane / 16) + j][lane % 16]);
    }
    // Scales of the lane's two columns of each slab; kNativeAsym beta = half_rn(-alpha * zp) for
    // both columns with one packed fp16 multiply of the alphas by the stored (-zp) pair.
    float bs[kSlicesPerTile][2];
    float as[kSlicesPerTile][2];
#pragma unroll
    for (int sl = 0; sl < kSlicesPerTile; ++sl) {
      const uint32_t pair = (sl % 2 == 0) ? ld.alpha[sl / 2].x : ld.alpha[sl / 2].y;
      uint32_t beta_pair = 0;
      if constexpr (F == PacketFormat::kNativeAsym) {
        const uint32_t neg_zp = (sl % 2 == 0) ? ld.beta[sl / 2].x : ld.beta[sl / 2].y;
        beta_pair = __builtin_bit_cast(
            uint32_t, __builtin_bit_cast(half2_t, pair) * __builtin_bit_cast(half2_t, neg_zp));
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        as[sl][i] = half_bits_to_float(static_cast<uint16_t>(pair >> (16 * i)));
        bs[sl][i] = half_bits_to_float(static_cast<uint16_t>(beta_pair >> (16 * i)));
      }
    }
    // The MFMA chains of kPass blocks, then their epilogues, so that the matrix core's latency is
    // not waited out block by block. G = 128 takes four blocks per pass: all eight would need
    // more than 256 registers and halve the workgroups per CU.
    constexpr int kPass = G == 64 ? 8 : 4;
#pragma unroll
    for (int b0 = 0; b0 < 8; b0 += kPass) {
      float4_t d[kPass];
#pragma unroll
      for (int bi = 0; bi < kPass; ++bi) {
        const int blk = b0 + bi;
        const int sl = blk / 2;  // slab
        const int i = blk % 2;   // half of the slab
        uint32_t words[U];
        if constexpr (G == 128) {
          const uint4 v = ld.w[sl / 2][2 * (sl % 2) + i];
          words[0] = v.x;
          words[1] = v.y;
          words[2] = v.z;
          words[3] = v.w;
        } else {
          const uint4 v = ld.w[sl / 2][sl % 2];
          words[0] = i == 0 ? v.x : v.z;
          words[1] = i == 0 ? v.y : v.w;
        }
        d[bi] = seed;
#pragma unroll
        for (int j = 0; j < U; ++j) {
          d[bi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              a[j], unpack_word(words[j], mask_lo, mask_hi), d[bi], 0, 0, 0);
        }
      }
#pragma unroll
      for (int bi = 0; bi < kPass; ++bi) {
        const int blk = b0 + bi;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          apply(y[blk / 4][blk % 4][r], as[blk / 2][blk % 2], bs[blk / 2][blk % 2], d[bi][r], r);
        }
      }
    }
    return;
  }
  half8_t a[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    a[kb] = __builtin_bit_cast(half8_t, sm.xs[gl][kb * 4 + lane / 16][lane % 16]);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float4_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      d[j] = seed;
    }
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const uint32_t words[4] = {ld.w[h][kb].x, ld.w[h][kb].y, ld.w[h][kb].z, ld.w[h][kb].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        d[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            a[kb], unpack_word(words[j], mask_lo, mask_hi), d[j], 0, 0, 0);
      }
    }
    const uint16_t ab[4] = {static_cast<uint16_t>(ld.alpha[h].x), static_cast<uint16_t>(ld.alpha[h].x >> 16),
                            static_cast<uint16_t>(ld.alpha[h].y), static_cast<uint16_t>(ld.alpha[h].y >> 16)};
    const uint16_t bb[4] = {static_cast<uint16_t>(ld.beta[h].x), static_cast<uint16_t>(ld.beta[h].x >> 16),
                            static_cast<uint16_t>(ld.beta[h].y), static_cast<uint16_t>(ld.beta[h].y >> 16)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float alpha = half_bits_to_float(ab[j]);
      const float beta = group_offset<F>(alpha, bb[j], (ld.beta[h].x >> (4 * j)) & 0xFu);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        apply(y[h][j][r], alpha, beta, d[j][r], r);
      }
    }
  }
}

template <int G, Act A, PacketFormat F>
__device__ __forceinline__ void mfma_stream_groups(MfmaSmem<G>& sm, const MfmaParams& p,
                                                   const uint8_t* tile_packets, int row0, int g_lo,
                                                   int g_hi, int lane, int wave, uint32_t mask_lo,
                                                   uint32_t mask_hi,
                                                   float (&y)[2][4][4]) {
  constexpr int kChunk = MfmaSmem<G>::kChunk;
  // Two groups in flight per wave: three or four measured slower at 14336 x 4096 on MI355X.
  constexpr int kDepth = 2;
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  for (int g0 = g_lo; g0 < g_hi; g0 += kChunk) {
    const int n_chunk = min(kChunk, g_hi - g0);
    if (g0 != g_lo) {
      lds_barrier();
    }
    MfmaStage<G> st;
    mfma_stage_load<G>(st, p, row0, g0, n_chunk);
    // This wave's groups: gl = wave + 4t, t < n_w, through kDepth register buffers; loads are
    // unconditional (a wave past its last group re-reads that group and does not compute it) so
    // the compiler can count the loads behind each buffer.
    const int n_w = n_chunk > wave ? (n_chunk - wave + kWaves - 1) / kWaves : 0;
    const int t_last = max(n_w - 1, 0);
    const int gl_base = n_w > 0 ? wave : n_chunk - 1;
    const uint8_t* gp = tile_packets + static_cast<size_t>(g0 + gl_base) * stride;
    const size_t step = static_cast<size_t>(kWaves) * stride;
    const size_t slice_step = static_cast<size_t>(p.NG) * stride;  // native formats
    MfmaGroupLoad<G> buf[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      mfma_load_group<G, F>(buf[d], gp + static_cast<size_t>(min(d, t_last)) * step, slice_step,
                            lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    mfma_stage_store<G, A>(sm, st, n_chunk);
    lds_barrier();
    const int n_blocks = (n_w + kDepth - 1) / kDepth;
    int t0 = 0;
    for (int blk = 0; blk + 1 < n_blocks; ++blk, t0 += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        mfma_compute_group<G, A, F>(sm, buf[d], wave + (t0 + d) * kWaves, lane, mask_lo, mask_hi,
                                    y);
        mfma_load_group<G, F>(buf[d],
                              gp + static_cast<size_t>(min(t0 + kDepth + d, t_last)) * step,
                              slice_step, lane);
      }
    }
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      if (t0 + d < n_w) {
        mfma_compute_group<G, A, F>(sm, buf[d], wave + (t0 + d) * kWaves, lane, mask_lo, mask_hi,
                                    y);
      }
    }
    // The loads of skipped tail slots are never consumed; retire them here, or the compiler's
    // wait for their registers lands between the next chunk's first loads and serialises them.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  }
}

template <int G, Act A, PacketFormat F>
__global__ void __launch_bounds__(kThreads, 2) w4a16_gemm_mfma_kernel(MfmaParams p) {
  constexpr int kOut = kRows * kTileCols;
  __shared__ MfmaSmem<G> sm;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  const int grid = p.grid;
  int b = static_cast<int>(blockIdx.x);
  b = p.xcd_remap != 0 ? (b & 7) * p.xcd_remap + (b >> 3) : b;
  // 32-bit unit arithmetic (the host keeps the unit count below 2^31): 64-bit divisions put
  // about 180 instructions ahead of the first weight load.
  const uint32_t ng = static_cast<uint32_t>(p.NG);
  const uint32_t total_units = static_cast<uint32_t>(p.tiles) * p.mtiles * p.NG;
  const uint32_t u_begin = static_cast<uint32_t>(b) * p.per;
  const uint32_t u_end = min(total_units, u_begin + p.per);
  uint32_t u = u_begin;
  while (u < u_end) {
    const uint32_t Tu = u / ng;
    const int T = static_cast<int>(Tu);
    const int g_lo = static_cast<int>(u - Tu * ng);
    const int g_hi = static_cast<int>(min(ng, g_lo + (u_end - u)));
    const uint32_t mt = Tu / static_cast<uint32_t>(p.tiles);
    const int tile = static_cast<int>(Tu - mt * p.tiles);
    const int row0 = static_cast<int>(mt) * kRows;
    const int col_base = tile * kTileCols;
    float y[2][4][4] = {};
    const uint8_t* tile_packets =
        p.packets + static_cast<size_t>(tile) * (is_native(F) ? kSlicesPerTile : 1) * p.NG * stride;
    mfma_stream_groups<G, A, F>(sm, p, tile_packets, row0, g_lo, g_hi, lane, wave, mask_lo,
                                mask_hi, y);
    if constexpr (is_native(F)) {
      // Lane l holds rows 4*(l/16)+r of column 32*s + 16*i + l%16 in y[s/2][2*(s%2)+i].
#pragma unroll
      for (int blk = 0; blk < 8; ++blk) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sm.red[wave][4 * (lane / 16) + r][16 * blk + lane % 16] = y[blk / 4][blk % 4][r];
        }
      }
    } else {
      // Lane l holds rows 4*(l/16)+r and columns h*64 + 4*(l%16) + j.
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          *reinterpret_cast<float4*>(&sm.red[wave][4 * (lane / 16) + r][h * 64 + 4 * (lane % 16)]) =
              make_float4(y[h][0][r], y[h][1][r], y[h][2][r], y[h][3][r]);
        }
      }
    }
    __syncthreads();
    auto red_sum = [&](int idx) {
      const int r = idx / kTileCols;
      const int c = idx % kTileCols;
      float v = sm.red[0][r][c];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) {
        v += sm.red[w][r][c];
      }
      return v;
    };
    const uint32_t tile_u0 = Tu * ng;
    const int first = static_cast<int>(tile_u0 / static_cast<uint32_t>(p.per));
    const int last = static_cast<int>((tile_u0 + ng - 1) / static_cast<uint32_t>(p.per));
    if (first == last) {
      for (int idx = tid; idx < kOut; idx += kThreads) {
        const int r = idx / kTileCols;
        if (row0 + r < p.M) {
          p.out[static_cast<size_t>(row0 + r) * p.N + col_base + idx % kTileCols] =
              float_to_act_bits<A>(red_sum(idx));
        }
      }
    } else {
      // Same hand-off as the GEMV kernel: relaxed agent-scope atomics, stores complete before the
      // barrier that precedes the counter increment, last arriver sums in workgroup order.
      const int contributors = last - first + 1;
      float* ws = p.partials + static_cast<size_t>(T) * p.max_contrib * kOut;
      for (int idx = tid; idx < kOut; idx += kThreads) {
        __hip_atomic_store(&ws[static_cast<size_t>(b - first) * kOut + idx], red_sum(idx),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
      if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&p.counters[T], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        sm.last = (prev == static_cast<uint32_t>(contributors - 1)) ? 1 : 0;
      }
      __syncthreads();
      if (sm.last) {
        constexpr int kPer = kOut / kThreads;
        float acc[kPer];
        sum_tile_partials<kPer, kThreads>(ws, kOut, contributors, tid, acc);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
          const int idx = tid + i * kThreads;
          const int r = idx / kTileCols;
          if (row0 + r < p.M) {
            p.out[static_cast<size_t>(row0 + r) * p.N + col_base + idx % kTileCols] =
                float_to_act_bits<A>(acc[i]);
          }
        }
        if (tid == 0) {
          __hip_atomic_store(&p.counters[T], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    __syncthreads();
    u += g_hi - g_lo;
  }
}

template <int G, Act A, PacketFormat F>
hipError_t launch_mfma_t(const GemvLaunch& l, hipStream_t stream) {
  MfmaParams p;
  p.x = static_cast<const uint16_t*>(l.x);
  p.packets = static_cast<const uint8_t*>(l.packets);
  p.out = static_cast<uint16_t*>(l.out);
  p.partials = static_cast<float*>(l.partials);
  p.counters = static_cast<uint32_t*>(l.counters);
  p.M = l.M;
  p.N = l.N;
  p.K = l.K;
  p.NG = l.K / G;
  p.tiles = l.N / kTileCols;
  p.mtiles = (l.M + kRows - 1) / kRows;
  p.per = l.units_per_workgroup;
  p.max_contrib = l.max_contributors;
  const long long total = static_cast<long long>(p.tiles) * p.mtiles * p.NG;
  const int grid = static_cast<int>((total + p.per - 1) / p.per);
  p.grid = grid;
  p.xcd_remap = grid % 8 == 0 ? grid / 8 : 0;
  hipLaunchKernelGGL((w4a16_gemm_mfma_kernel<G, A, F>), dim3(grid), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

template <int G, PacketFormat F>
hipError_t dispatch_act(const GemvLaunch& l, hipStream_t stream) {
  return l.act == Act::kF16 ? launch_mfma_t<G, Act::kF16, F>(l, stream)
                            : launch_mfma_t<G, Act::kBF16, F>(l, stream);
}

template <PacketFormat F>
hipError_t dispatch_group(const GemvLaunch& l, hipStream_t stream) {
  return l.group_size == 64 ? dispatch_act<64, F>(l, stream) : dispatch_act<128, F>(l, stream);
}

hipError_t dispatch_format(const GemvLaunch& l, hipStream_t stream) {
  switch (l.format) {
    case PacketFormat::kArc: return dispatch_group<PacketFormat::kArc>(l, stream);
    case PacketFormat::kNativeSym: return dispatch_group<PacketFormat::kNativeSym>(l, stream);
    case PacketFormat::kNativeAsym: return dispatch_group<PacketFormat::kNativeAsym>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_w4a16_gemm_mfma(const GemvLaunch& l, hipStream_t stream) {
  if (l.m_tile != kRows || l.mode != GemvMode::kStreamK || l.slice_cols != kTileCols) {
    return hipErrorInvalidValue;
  }
  return dispatch_format(l, stream);
}

}  // namespace fk
