// W4A16 GEMV / small-batch GEMM kernels (dot2 path) over the reference packets, hand-written for
// gfx950. Templates: w4a16_gemv.hip instantiates them; the native slab formats have their own
// kernel (w4a16_gemv_native.hip), which shares the staging, the work split and the fix-up here.
//
// Computes y[m,n] = round( sum_g sum_{k in g} (alpha[n,g]*q[n,k] + beta[n,g]) * x[m,k] ), fp32
// accumulation, output in the activation dtype (fp16 or bf16). Follows the math of the reference
// hot loop (arc_w4a16.cu:222-297, accumulate_arc_group_range) but not its structure:
//
//  * 128-bit loads over column slices. A packet (arc_w4a16.cu:87-122) stores word w of column c
//    at byte (w*128 + c)*4, so a word row is 512 contiguous bytes. A workgroup owns a slice of
//    CW in {128, 64, 32} columns of a 128-column tile; one 64-lane dwordx4 load covers 256/CW word
//    rows of the slice (CW*4 contiguous bytes each, whole 128-byte lines), and lane l holds the
//    four columns 4*(l % (CW/4)) .. +3 of word row l / (CW/4). Narrow slices give small-N shapes
//    enough workgroups to fill the chip without splitting K across workgroups.
//  * A wave streams its own groups of the slice through D register buffers of one group each
//    (16 dwordx4 loads per lane in flight for whole tiles, 8 for narrower slices), refilling
//    each buffer as soon as it is consumed.
//  * Register dequant with no per-element conversion: nibbles are OR-ed into fp16 mantissas
//    (see w4a16_device.h) and multiplied by v_dot2_f32_f16 (fp32 accumulation) against
//    activations re-paired once per workgroup in LDS. High nibbles unpack as 64 + q (fp16
//    0x5400 | q << 4), so both positions add into one fp32
//    accumulator: sum (1024 + q) x_e + (64 + q) x_o. The constant part is removed by seeding the
//    accumulator with -1024 S_e - 64 S_o from per-group activation sums, and the group's beta
//    term is beta * (S_e + S_o).
//  * bf16 activations are converted to fp16 when staged, after scaling each (row, group) by a
//    power of two that puts its largest magnitude in fp16's top binade (bf16_stage_shift); the
//    scale is re-applied to the group's fp32 partial. Every bf16 value within 2^-24 of its
//    group's largest converts exactly (bf16 has 8 significant bits, fp16 normals 11), so bf16
//    runs the same fp16 inner loop.
//  * Stream-K work split: the grid is sized to be resident on the chip at once and each
//    workgroup takes an equal run of (slice, group) units, crossing slice boundaries; slices
//    shared by several workgroups are finished in-kernel by their last contributor (see the
//    kernel).
//  * Logical workgroup order is remapped so that consecutive logical workgroups (the
//    contributors of one slice) run on the same XCD: the hardware dispatches workgroup b to
//    XCD b % 8.
#pragma once

#include <hip/hip_runtime.h>

#include "w4a16_gemv.h"

#include <cstddef>
#include <cstdint>

#include "w4a16_device.h"

namespace fk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kWordRowBytes = kTileCols * 4;


// Geometry of a CW-column slice of a G-group packet.
template <int G, int CW>
struct Slice {
  static constexpr int kLanesPerRow = CW / 4;             // lanes covering one word row
  static constexpr int kRowsPerLoad = 64 / kLanesPerRow;  // word rows per wave-wide load
  static constexpr int kWordRows = G / 8;                 // word rows per group
  static constexpr int kLoads = kWordRows / kRowsPerLoad;  // dwordx4 loads per group and lane
  // Register buffers (groups in flight per wave): 16 dwordx4 loads per lane for whole tiles,
  // 8 for 64- and 32-column slices (measured on MI355X: deeper pipelines over narrow slices
  // lower the achieved bandwidth, as for the native slabs).
  static constexpr int kDepth = (CW == kTileCols ? 16 : 8) / kLoads;
  static constexpr int kSlices = kTileCols / CW;
  static_assert(kLoads >= 1 && kWordRows % kRowsPerLoad == 0, "unsupported slice");
};

// Groups whose activations are staged in LDS at once. Wide slices run two workgroups per CU, so
// their staging area stays small; narrow slices are used when there are fewer slices than CUs
// (one workgroup per CU) and stage more of K per barrier.
//
// 32-column slices with G = 64 and 2-4 rows stage 1024 word rows (32 or 64 groups, the same
// register footprint as 16 groups at G = 128): fewer barriers and staging rounds per run, measured
// 1-1.5 us faster at 14336 x 4096 on MI355X. The same rule at G = 128 spills.
template <int G, int MT, int CW>
constexpr int chunk_groups() {
  if (CW == 32 && G == 64 && MT >= 2 && MT <= 4) {
    return 128 / MT;
  }
  return MT > 1 ? 16 : (CW == kTileCols ? 32 : 64);
}

template <int G, int MT, int CW>
struct Smem {
  static constexpr int kChunk = chunk_groups<G, MT, CW>();
  static constexpr int kWordRows = G / 8;
  static constexpr int kRowsPerLoad = Slice<G, CW>::kRowsPerLoad;
  uint4 xs[MT][kChunk][kWordRows];        // re-paired fp16 activations, 16 B per word row
  // per word-row class r mod kRowsPerLoad: {-1024 S_even - 64 S_odd, S_even + S_odd}
  float2 sums[MT][kChunk][kRowsPerLoad];
  float scale[MT][kChunk];                // power of two undoing the bf16 staging scale
  float red[kWaves][MT][CW];              // cross-wave reduction
  int last;                               // this workgroup finishes the slice
};

struct GemvParams {
  const uint16_t* x;       // [M, K] activations (fp16 or bf16 bits)
  const uint8_t* packets;  // [(N/128) * NG, S]
  uint16_t* out;           // [M, N] (unused in partials mode)
  float* partials;         // fix-up scratch or reference split-K partials [S_k, M, N]
  uint32_t* counters;      // fix-up arrival counters, one per (slice, m-tile)
  int M, N, K, NG;
  int tiles, mtiles, splits, gps;  // kPartials: fixed split of every tile
  int per;                          // stream-K: group units per workgroup
  int max_contrib;                  // stream-K: partial slots per slice in the scratch
  // Workgroups of the launch, read with the other arguments (gridDim is a kernel argument of its
  // own, and a second, dependent argument load at the start of every workgroup).
  int grid;
  int xcd_remap;  // grid / 8 when consecutive logical workgroups are kept on one XCD, else 0
  const uint16_t* norm_weight;      // RMSNorm prologue: gamma [K] (activation dtype), else null
  float eps;                        // RMSNorm prologue: epsilon
  int pair;                         // native slabs: each run streams two adjacent whole slices
  int stream_whole;                 // stream schedule: whole slices per workgroup
  uint32_t ng_magic;                // quarter schedule over reference packets: floor(2^32/NG) + 1
  int stream_parts;                 // matrix-core stream kernel: K in this many parts (1: whole)
};

template <int G, int MT, int CW>
struct StageRegs {
  static constexpr int kUnits = MT * chunk_groups<G, MT, CW>() * (G / 8);
  static constexpr int kPerThread = (kUnits + kThreads - 1) / kThreads;
  uint4 raw[kPerThread];
  bool ok[kPerThread];  // the unit lies inside the chunk and the batch (else it stages zeros)

  __device__ __forceinline__ uint4 unit(int it) const {
    return ok[it] ? raw[it] : make_uint4(0u, 0u, 0u, 0u);
  }
};

// Issue the global loads of one chunk's activations (16 B = one word row per unit). Every load is
// issued unconditionally from a clamped, in-bounds address and units outside the chunk or the
// batch are zeroed where they are consumed (StageRegs::unit): loads under a branch each wait for
// the one before, which serialised the start of every run.
template <int G, int MT, int CW>
__device__ __forceinline__ void stage_load(StageRegs<G, MT, CW>& st, const GemvParams& p, int row0,
                                           int g0, int n_chunk) {
  constexpr int WR = G / 8;
  constexpr int kChunk = chunk_groups<G, MT, CW>();
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < StageRegs<G, MT, CW>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunk;
    const int m = u / (WR * kChunk);
    st.ok[it] = u < StageRegs<G, MT, CW>::kUnits && gl < n_chunk && row0 + m < p.M;
    const int row = min(row0 + m, p.M - 1);
    const size_t off = static_cast<size_t>(row) * p.K +
                       static_cast<size_t>(g0 + min(gl, n_chunk - 1)) * G +
                       static_cast<size_t>(w) * 8;
    st.raw[it] = *reinterpret_cast<const uint4*>(p.x + off);
  }
}

// Convert (bf16) and re-pair the staged activations into LDS and reduce the per-(row, group,
// word row mod R) sums, R = word rows per load. Word rows of one (m, group) are WR consecutive,
// WR-aligned lanes, so xor-shuffles over R..WR/2 stay inside the group.
template <int G, Act A, int MT, int CW>
__device__ __forceinline__ void stage_store(Smem<G, MT, CW>& sm, StageRegs<G, MT, CW>& st,
                                            int n_chunk) {
  constexpr int WR = G / 8;
  constexpr int R = Slice<G, CW>::kRowsPerLoad;
  constexpr int kChunk = chunk_groups<G, MT, CW>();
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < StageRegs<G, MT, CW>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunk;
    const int m = u / (WR * kChunk);
    // Units past the chunk stage nothing; a group's WR lanes share gl (see the native staging).
    if (u >= StageRegs<G, MT, CW>::kUnits || gl >= n_chunk) {
      continue;
    }
    uint4 r = st.unit(it);
    float undo = 1.0f;
    if constexpr (A == Act::kBF16) {
      const uint32_t e = group_max<WR>(bf16_max_mag(r)) >> 7;
      const int shift = bf16_stage_shift(e);
      const float s = __builtin_bit_cast(float, static_cast<uint32_t>(127 - shift) << 23);
      undo = __builtin_bit_cast(float, static_cast<uint32_t>(127 + shift) << 23);
      r.x = bf16_pair_to_half_pair(r.x, s);
      r.y = bf16_pair_to_half_pair(r.y, s);
      r.z = bf16_pair_to_half_pair(r.z, s);
      r.w = bf16_pair_to_half_pair(r.w, s);
    }
    // even k: x0 x2 x4 x6 (low halves), odd k: x1 x3 x5 x7 (high halves)
    float se = half_bits_to_float(static_cast<uint16_t>(r.x)) +
               half_bits_to_float(static_cast<uint16_t>(r.y)) +
               half_bits_to_float(static_cast<uint16_t>(r.z)) +
               half_bits_to_float(static_cast<uint16_t>(r.w));
    float so = half_bits_to_float(static_cast<uint16_t>(r.x >> 16)) +
               half_bits_to_float(static_cast<uint16_t>(r.y >> 16)) +
               half_bits_to_float(static_cast<uint16_t>(r.z >> 16)) +
               half_bits_to_float(static_cast<uint16_t>(r.w >> 16));
    if constexpr (WR == 16 && R < WR) {
      // One 16-lane DPP row per (row, group): rotations by R, 2R, ... (one VALU op each).
      se = row_strided_sum<R>(se);
      so = row_strided_sum<R>(so);
    } else if constexpr (R == 2) {
      // Even and odd word rows of an 8-lane group: masked 8-lane DPP reductions.
      const bool odd = (w & 1) != 0;
      const float se_odd = group_sum<WR>(odd ? se : 0.0f);
      const float so_odd = group_sum<WR>(odd ? so : 0.0f);
      const float se_even = group_sum<WR>(odd ? 0.0f : se);
      const float so_even = group_sum<WR>(odd ? 0.0f : so);
      se = odd ? se_odd : se_even;
      so = odd ? so_odd : so_even;
    } else {
#pragma unroll
      for (int off = R; off < WR; off <<= 1) {
        se += __shfl_xor(se, off);
        so += __shfl_xor(so, off);
      }
    }
    {
      // Both nibble positions accumulate into one sum, (1024 + q) x_e + (64 + q) x_o (the high
      // nibbles unpack as 64 + q), so the activations are staged as they are.
      const uint4 xp = pair_activations(r);
      sm.xs[m][gl][w] = xp;
      if (w < R) {
        // the unpack bias, which seeds the accumulators, and the sum for the beta term
        sm.sums[m][gl][w] = make_float2(fmaf(-1024.0f, se, -64.0f * so), se + so);
      }
      if (w == 0) {
        sm.scale[m][gl] = undo;
      }
    }
  }
}


template <int G, int CW, PacketFormat F>
struct GroupLoad {
  static constexpr int NL = Slice<G, CW>::kLoads;
  uint4 w[NL];
  uint2 alpha;
  uint2 beta;  // 4 fp16 offsets
};

// Per-lane constant parts of a group's addresses inside its packet.
struct LaneAddr {
  int code;   // byte offset of the lane's first 16 B of codes
  int scale;  // byte offset of the lane's 4 alphas (the betas follow 256 bytes later)
};

template <int G, int CW>
__device__ __forceinline__ LaneAddr lane_addr(int lane, int slice) {
  constexpr int LPR = Slice<G, CW>::kLanesPerRow;
  const int col = slice * CW + 4 * (lane % LPR);
  LaneAddr a;
  a.code = (lane / LPR) * kWordRowBytes + col * 4;
  a.scale = kTileCols * G / 2 + col * 2;
  return a;
}

template <int G, int CW, PacketFormat F>
__device__ __forceinline__ void load_group(GroupLoad<G, CW, F>& gl, const uint8_t* packet,
                                           LaneAddr la) {
  static_assert(F == PacketFormat::kArc, "native slabs are read by w4a16_gemv_native.hip");
  constexpr int R = Slice<G, CW>::kRowsPerLoad;
  gl.alpha = stream_load8(packet + la.scale);
  gl.beta = stream_load8(packet + la.scale + kTileCols * 2);
#pragma unroll
  for (int i = 0; i < GroupLoad<G, CW, F>::NL; ++i) {
    gl.w[i] = stream_load16(packet + la.code + i * R * kWordRowBytes);
  }
}

// One group: multiply-accumulate its codes against the staged activations, then apply the
// group's scales: with the accumulator seeded by the unpack bias C = -1024 S_e - 64 S_o,
// y += alpha * acc + beta * (S_e + S_o).
template <int G, Act A, int MT, int CW, PacketFormat F>
__device__ __forceinline__ void compute_group(const Smem<G, MT, CW>& sm,
                                              const GroupLoad<G, CW, F>& ld, int gl, int sub,
                                              uint32_t mask_lo, uint32_t mask_hi,
                                              float (&y)[MT][4]) {
  constexpr int NL = GroupLoad<G, CW, F>::NL;
  constexpr int R = Slice<G, CW>::kRowsPerLoad;
  // One accumulator per (row, column); a single row keeps a second one so that its dependent
  // dot2 chains interleave in pairs.
  constexpr int kAcc = MT == 1 ? 2 : 1;
  float acc[MT][4][kAcc];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float seed = sm.sums[m][gl][sub].x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[m][j][0] = seed;
      if constexpr (kAcc == 2) {
        acc[m][j][kAcc - 1] = 0.0f;
      }
    }
  }

#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int wrow = i * R + sub;
    uint4 xp[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      xp[m] = sm.xs[m][gl][wrow];
    }
    const uint32_t words[4] = {ld.w[i].x, ld.w[i].y, ld.w[i].z, ld.w[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t wv = words[j];
      const uint32_t e0 = (wv & mask_lo) | kBiasLow;   // 1024+q for k0,k4
      const uint32_t o0 = (wv & mask_hi) | kBiasHigh;  // 64+q for k1,k5
      const uint32_t w8 = wv >> 8;
      const uint32_t e1 = (w8 & mask_lo) | kBiasLow;   // k2,k6
      const uint32_t o1 = (w8 & mask_hi) | kBiasHigh;  // k3,k7
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float& a0 = acc[m][j][0];
        float& a1 = acc[m][j][kAcc - 1];
        a0 = dot2<Act::kF16>(e0, xp[m].x, a0);
        a1 = dot2<Act::kF16>(o0, xp[m].y, a1);
        a0 = dot2<Act::kF16>(e1, xp[m].z, a0);
        a1 = dot2<Act::kF16>(o1, xp[m].w, a1);
      }
    }
  }

  const uint16_t a_bits[4] = {static_cast<uint16_t>(ld.alpha.x), static_cast<uint16_t>(ld.alpha.x >> 16),
                              static_cast<uint16_t>(ld.alpha.y), static_cast<uint16_t>(ld.alpha.y >> 16)};
  const uint16_t b_bits[4] = {static_cast<uint16_t>(ld.beta.x), static_cast<uint16_t>(ld.beta.x >> 16),
                              static_cast<uint16_t>(ld.beta.y), static_cast<uint16_t>(ld.beta.y >> 16)};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float a = half_bits_to_float(a_bits[j]);
    const float b = group_offset<F>(a, b_bits[j], (ld.beta.x >> (4 * j)) & 0xFu);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float sum = acc[m][j][0];
      if constexpr (kAcc == 2) {
        sum += acc[m][j][1];
      }
      const float s = sm.sums[m][gl][sub].y;
      if constexpr (A == Act::kBF16) {
        // the staged activations carry a power-of-two scale per (row, group)
        y[m][j] = fmaf(fmaf(b, s, a * sum), sm.scale[m][gl], y[m][j]);
      } else {
        y[m][j] = fmaf(b, s, fmaf(a, sum, y[m][j]));
      }
    }
  }
}

// Waves per SIMD the M=1 kernel must fit (caps its VGPRs at 512 / waves). Two is the measured
// optimum: the pipelined loop needs ~170-190 VGPRs, and capping lower spills registers.
template <int MT>
constexpr int min_waves_per_eu() {
  return MT == 1 ? 2 : 1;
}

// Accumulate groups [g_lo, g_hi) of one slice into y: stage the activations of up to kChunk
// groups in LDS, then each wave streams groups g_lo + wave, g_lo + wave + 4, ... through D
// register buffers.
template <int G, Act A, int MT, int CW, PacketFormat F>
__device__ __forceinline__ void stream_groups(Smem<G, MT, CW>& sm, const GemvParams& p,
                                              const uint8_t* tile_packets, LaneAddr la, int row0,
                                              int g_lo, int g_hi, int wave, int sub,
                                              uint32_t mask_lo, uint32_t mask_hi,
                                              float (&y)[MT][4]) {
  constexpr int kChunk = chunk_groups<G, MT, CW>();
  constexpr int D = Slice<G, CW>::kDepth;
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  for (int g0 = g_lo; g0 < g_hi; g0 += kChunk) {
    const int n_chunk = min(kChunk, g_hi - g0);
    if (g0 != g_lo) {
      lds_barrier();  // previous chunk's readers are done with xs / sums
    }
    // Activation loads first, then the first D weight groups of this wave, so the LDS writes
    // below only wait for the activations while the weights stay in flight across the barrier.
    StageRegs<G, MT, CW> st;
    stage_load<G, MT, CW>(st, p, row0, g0, n_chunk);
    // This wave's groups in the chunk: gl = wave + 4t, t < n_w; buffer d holds t = d mod D.
    // Loads are unconditional (past its last group a wave re-reads that group, an L2 hit it
    // does not compute), so the compiler can count the loads behind any buffer and wait for that
    // buffer alone.
    const int n_w = n_chunk > wave ? (n_chunk - wave + kWaves - 1) / kWaves : 0;
    const int t_last = max(n_w - 1, 0);
    const int gl_base = n_w > 0 ? wave : n_chunk - 1;
    const uint8_t* gp = tile_packets + static_cast<size_t>(g0 + gl_base) * stride;
    const size_t step = static_cast<size_t>(kWaves) * stride;
    GroupLoad<G, CW, F> buf[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      load_group<G, CW, F>(buf[d], gp + static_cast<size_t>(min(d, t_last)) * step, la);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load above the first use of the activations
    stage_store<G, A, MT, CW>(sm, st, n_chunk);
    lds_barrier();
    // Blocks of D groups; every block but the last refills each buffer right after computing it.
    const int n_blocks = (n_w + D - 1) / D;
    int t0 = 0;
    for (int blk = 0; blk + 1 < n_blocks; ++blk, t0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        compute_group<G, A, MT, CW, F>(sm, buf[d], wave + (t0 + d) * kWaves, sub, mask_lo, mask_hi, y);
        load_group<G, CW, F>(buf[d], gp + static_cast<size_t>(min(t0 + D + d, t_last)) * step, la);
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (t0 + d < n_w) {
        compute_group<G, A, MT, CW, F>(sm, buf[d], wave + (t0 + d) * kWaves, sub, mask_lo, mask_hi, y);
      }
    }
    // The loads of skipped tail slots are never consumed; retire them here, or the compiler's
    // wait for their registers lands between the next chunk's first loads and serialises them.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  }
}

// Sum y over the lanes that share columns (different word rows) and over the waves into sm.red.
template <int G, int MT, int CW>
__device__ __forceinline__ void reduce_to_lds(Smem<G, MT, CW>& sm, float (&y)[MT][4], int lane,
                                              int wave) {
  constexpr int LPR = Slice<G, CW>::kLanesPerRow;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) {
        y[m][j] += __shfl_xor(y[m][j], off);
      }
    }
  }
  if (lane < LPR) {
    const int c0 = lane * 4;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      *reinterpret_cast<float4*>(&sm.red[wave][m][c0]) = make_float4(y[m][0], y[m][1], y[m][2], y[m][3]);
    }
  }
  __syncthreads();
}

template <int G, int MT, int CW>
__device__ __forceinline__ float red_sum(const Smem<G, MT, CW>& sm, int m, int c) {
  float v = sm.red[0][m][c];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    v += sm.red[w][m][c];
  }
  return v;
}

// Writes the totals of one run of slice T (value(m, c) for row row0 + m, column col_base + c).
// A run that covers the whole slice writes them directly. Otherwise the slice's contributors hand
// off through the workspace without cache-wide maintenance: partials and the arrival counter are
// accessed only through agent-scope relaxed atomics, which the gfx950 memory model serves
// coherently across XCDs (their L2s are not coherent with each other) without the whole-L2
// write-back / invalidate an agent-scope fence costs; ordering between a contributor's partial
// stores and its counter increment comes from waiting for the stores to complete (vmcnt(0))
// before the workgroup barrier that precedes the increment. The last contributor to arrive adds
// the partials in contributor order (deterministic) and resets the counter. `last` is an LDS
// flag. Ends with a workgroup barrier, so LDS used by value() can be reused afterwards.
// Position of stream-K unit u in (m-tile, tile, slice, group) order, the run from u ending at
// the slice's last group or at u_end. 32-bit arithmetic (the host keeps the unit count below
// 2^31): the 64-bit divisions it replaces put about 180 instructions ahead of the first weight
// load, 0.1-0.2 us of every launch on MI355X.
struct RunPos {
  int T;      // (m-tile, tile, slice) index
  int g_lo;   // first group of the run
  int g_hi;   // one past its last group
  int slice;  // slice within the tile
  int tile;
  int mtile;
};

__device__ __forceinline__ RunPos run_pos(const GemvParams& p, uint32_t u, uint32_t u_end,
                                          int slices_per_tile) {
  const uint32_t ng = static_cast<uint32_t>(p.NG);
  const uint32_t t = u / ng;
  const uint32_t g_lo = u - t * ng;
  const uint32_t q = t / static_cast<uint32_t>(slices_per_tile);
  const uint32_t mt = q / static_cast<uint32_t>(p.tiles);
  RunPos r;
  r.T = static_cast<int>(t);
  r.g_lo = static_cast<int>(g_lo);
  r.g_hi = static_cast<int>(min(ng, g_lo + (u_end - u)));
  r.slice = static_cast<int>(t - q * slices_per_tile);
  r.tile = static_cast<int>(q - mt * static_cast<uint32_t>(p.tiles));
  r.mtile = static_cast<int>(mt);
  return r;
}

template <Act A, int MT, int CW, class Value>
__device__ __forceinline__ void finish_run(const GemvParams& p, int T, int b, int row0, int col_base,
                                           int& last, Value value) {
  constexpr int kOut = MT * CW;
  const int tid = static_cast<int>(threadIdx.x);
  const uint32_t slice_u0 = static_cast<uint32_t>(T) * static_cast<uint32_t>(p.NG);
  const int first_wg = static_cast<int>(slice_u0 / static_cast<uint32_t>(p.per));
  const int last_wg = static_cast<int>((slice_u0 + p.NG - 1) / static_cast<uint32_t>(p.per));
  if (first_wg == last_wg) {
    for (int idx = tid; idx < kOut; idx += kThreads) {
      const int m = idx / CW;
      const int c = idx % CW;
      if (row0 + m < p.M) {
        p.out[static_cast<size_t>(row0 + m) * p.N + col_base + c] = float_to_act_bits<A>(value(m, c));
      }
    }
  } else {
    const int contributors = last_wg - first_wg + 1;
    float* ws = p.partials + static_cast<size_t>(T) * p.max_contrib * kOut;
    for (int idx = tid; idx < kOut; idx += kThreads) {
      __hip_atomic_store(&ws[static_cast<size_t>(b - first_wg) * kOut + idx], value(idx / CW, idx % CW),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = __hip_atomic_fetch_add(&p.counters[T], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      last = (prev == static_cast<uint32_t>(contributors - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (last) {
      constexpr int kPer = (kOut + kThreads - 1) / kThreads;
      float acc[kPer];
      sum_tile_partials<kPer, kThreads>(ws, kOut, contributors, tid, acc);
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int idx = tid + i * kThreads;
        const int m = idx / CW;
        const int c = idx % CW;
        if (idx < kOut && row0 + m < p.M) {
          p.out[static_cast<size_t>(row0 + m) * p.N + col_base + c] = float_to_act_bits<A>(acc[i]);
        }
      }
      if (tid == 0) {
        __hip_atomic_store(&p.counters[T], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __syncthreads();
}

// Work decomposition. A "slice" is CW columns of a 128-column tile for one m-tile of rows; the
// slices laid end to end (slices of a tile, then tiles, then m-tiles) form a line of T*NG group
// units. Workgroup b owns units [b*per, (b+1)*per): "stream-K", every workgroup gets the same
// number of groups whatever the shape, and the grid is sized to fit on the chip at once, so no
// workgroup waits for a second round. A slice whose units all belong to one workgroup is written
// directly. A slice split between workgroups is finished by the last of its contributors to
// arrive (device-scope counter), which adds the fp32 partials in workgroup order, so results do
// not depend on arrival order; it also resets the counter, so no memset is needed between calls
// (graph-capture friendly).
//
// kPartials (the reference split-K protocol, whole tiles) instead writes each workgroup's fp32
// partial to partials[split, m, n] with split = b % splits over a fixed per-tile split.
template <int G, Act A, int MT, GemvMode MODE, int CW, PacketFormat F>
__global__ void __launch_bounds__(kThreads, min_waves_per_eu<MT>())
w4a16_gemv_kernel(GemvParams p) {
  constexpr int kOut = MT * CW;
  constexpr int kSlices = Slice<G, CW>::kSlices;
  __shared__ Smem<G, MT, CW> sm;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int sub = lane / Slice<G, CW>::kLanesPerRow;         // word row within a load
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));

  // Logical workgroup id: keep consecutive ids (the contributors of one slice) on one XCD.
  const int grid = p.grid;
  int b = static_cast<int>(blockIdx.x);
  b = p.xcd_remap != 0 ? (b & 7) * p.xcd_remap + (b >> 3) : b;

  if constexpr (MODE == GemvMode::kPartials) {
    static_assert(CW == kTileCols, "the partials protocol runs on whole tiles");
    const int split = b % p.splits;
    const int T = b / p.splits;
    const int tile = T % p.tiles;
    const int row0 = (T / p.tiles) * MT;
    const int g_lo = split * p.gps;
    const int g_hi = min(p.NG, g_lo + p.gps);
    float y[MT][4] = {};
    const uint8_t* tile_packets = p.packets + static_cast<size_t>(tile) * p.NG * stride;
    stream_groups<G, A, MT, CW, F>(sm, p, tile_packets, lane_addr<G, CW>(lane, 0), row0, g_lo,
                                   g_hi, wave, sub, mask_lo, mask_hi, y);
    reduce_to_lds<G, MT, CW>(sm, y, lane, wave);
    for (int idx = tid; idx < kOut; idx += kThreads) {
      const int m = idx / CW;
      const int c = idx % CW;
      if (row0 + m < p.M) {
        p.partials[(static_cast<size_t>(split) * p.M + row0 + m) * p.N + tile * kTileCols + c] =
            red_sum(sm, m, c);
      }
    }
    return;
  } else {
    const uint32_t total_units = static_cast<uint32_t>(p.tiles) * kSlices * p.mtiles * p.NG;
    const uint32_t u_begin = static_cast<uint32_t>(b) * p.per;
    const uint32_t u_end = min(total_units, u_begin + p.per);
    uint32_t u = u_begin;
    while (u < u_end) {
      const RunPos r = run_pos(p, u, u_end, kSlices);
      const int T = r.T;
      const int g_lo = r.g_lo;
      const int g_hi = r.g_hi;
      const int slice = r.slice;
      const int tile = r.tile;
      const int row0 = r.mtile * MT;
      const int col_base = tile * kTileCols + slice * CW;
      float y[MT][4] = {};
      const uint8_t* tile_packets = p.packets + static_cast<size_t>(tile) * p.NG * stride;
      stream_groups<G, A, MT, CW, F>(sm, p, tile_packets, lane_addr<G, CW>(lane, slice), row0,
                                     g_lo, g_hi, wave, sub, mask_lo, mask_hi, y);
      reduce_to_lds<G, MT, CW>(sm, y, lane, wave);

      finish_run<A, MT, CW>(p, T, b, row0, col_base, sm.last,
                            [&](int m, int c) { return red_sum(sm, m, c); });
      u += g_hi - g_lo;
    }
  }
}

template <int G, Act A, int MT, GemvMode MODE, int CW, PacketFormat F>
hipError_t launch_t(const GemvLaunch& l, hipStream_t stream) {
  GemvParams p;
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
  p.mtiles = (l.M + MT - 1) / MT;
  p.pair = 0;
  p.splits = l.splits;
  p.gps = l.gps;
  p.per = l.units_per_workgroup;
  p.max_contrib = l.max_contributors;
  int grid = 0;
  if (MODE == GemvMode::kPartials) {
    grid = p.tiles * p.mtiles * p.splits;
  } else {
    const long long total = static_cast<long long>(p.tiles) * (kTileCols / CW) * p.mtiles * p.NG;
    grid = static_cast<int>((total + p.per - 1) / p.per);
  }
  p.grid = grid;
  p.xcd_remap = grid % 8 == 0 ? grid / 8 : 0;
  hipLaunchKernelGGL((w4a16_gemv_kernel<G, A, MT, MODE, CW, F>), dim3(grid), dim3(kThreads), 0,
                     stream, p);
  return hipGetLastError();
}

template <int G, Act A, int MT, PacketFormat F>
hipError_t dispatch_cw(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode == GemvMode::kPartials) {
    return launch_t<G, A, MT, GemvMode::kPartials, kTileCols, F>(l, stream);
  }
  // Narrow slices serve the small-N shapes of decode (one or two activation rows); with more rows
  // a tile's registers per lane grow with MT and the narrow-slice buffers would spill.
  if constexpr (MT <= 2) {
    switch (l.slice_cols) {
      case 32: return launch_t<G, A, MT, GemvMode::kStreamK, 32, F>(l, stream);
      case 64: return launch_t<G, A, MT, GemvMode::kStreamK, 64, F>(l, stream);
      default: break;
    }
  }
  if (l.slice_cols != kTileCols) {
    return hipErrorInvalidValue;
  }
  return launch_t<G, A, MT, GemvMode::kStreamK, kTileCols, F>(l, stream);
}

template <int G, Act A, PacketFormat F>
hipError_t dispatch_mt(const GemvLaunch& l, hipStream_t stream) {
  switch (l.m_tile) {
    case 1: return dispatch_cw<G, A, 1, F>(l, stream);
    case 2: return dispatch_cw<G, A, 2, F>(l, stream);
    case 4: return dispatch_cw<G, A, 4, F>(l, stream);
    case 8: return dispatch_cw<G, A, 8, F>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

// Launches one packet format's dot2 GEMV kernels (each format is instantiated in its own
// translation unit).
template <PacketFormat F>
hipError_t launch_format(const GemvLaunch& l, hipStream_t stream) {
  if (l.slice_cols != 32 && l.slice_cols != 64 && l.slice_cols != kTileCols) {
    return hipErrorInvalidValue;
  }
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? dispatch_mt<64, Act::kF16, F>(l, stream)
                              : dispatch_mt<64, Act::kBF16, F>(l, stream);
  }
  return l.act == Act::kF16 ? dispatch_mt<128, Act::kF16, F>(l, stream)
                            : dispatch_mt<128, Act::kBF16, F>(l, stream);
}

}  // namespace
}  // namespace fk
