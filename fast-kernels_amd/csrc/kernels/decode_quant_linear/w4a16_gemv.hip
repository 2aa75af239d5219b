// W4A16 GEMV / small-batch GEMM over the reference's packet layout, hand-written for gfx950.
//
// Computes y[m,n] = round( sum_g sum_{k in g} (alpha[n,g]*q[n,k] + beta[n,g]) * x[m,k] ), fp32
// accumulation, output in the activation dtype (fp16 or bf16). Follows the math of the reference
// hot loop (arc_w4a16.cu:222-297, accumulate_arc_group_range) but not its structure:
//
//  * 128-bit loads. A packet (arc_w4a16.cu:87-122) stores word w of column c at byte
//    (w*128 + c)*4, so one 64-lane dwordx4 load covers two word rows x 128 columns: lane l holds
//    word row 2i + (l>>5) for the four columns 4*(l&31) .. +3. A wave streams one whole group
//    (G/16 loads) and keeps the next group's loads in flight while it computes.
//  * Register dequant with no per-element conversion: nibbles are OR-ed into fp16 / bf16
//    mantissas (see w4a16_device.h) and multiplied by v_dot2 against activations that were
//    re-paired once per workgroup in LDS. The constant bias that trick adds (1024 for fp16, 128
//    for bf16, times 1 or 16 depending on nibble position) is removed once per group and column
//    with per-group activation sums: sum((B + s*q) x) = B*sum(x) + s*sum(q x).
//  * Split-K across workgroups with an in-kernel fix-up: each workgroup reduces its 4 waves
//    through LDS (lanes l and l^32 first, with a cross-lane swap), writes an fp32 partial, and the
//    last workgroup of a tile to arrive (device-scope atomic counter) sums the partials in
//    split order, so the result does not depend on arrival order. The counter is reset by that
//    workgroup, so no memset is needed between calls (graph-capture friendly).
//  * Logical tile order is remapped so that consecutive logical workgroups (the splits of one
//    tile) run on the same XCD: the hardware dispatches workgroup b to XCD b % 8.
#include "w4a16_gemv.h"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "w4a16_device.h"

namespace fk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kChunkGroups = 16;  // groups whose activations are staged in LDS at once
// s_waitcnt immediate for gfx9: vmcnt = 0 (bits 3:0 and 15:14), expcnt and lgkmcnt left at max.
constexpr int kWaitVmcnt0 = 0x0F70;

template <int G, int MT>
struct Smem {
  static constexpr int kWordRows = G / 8;
  uint4 xs[MT][kChunkGroups][kWordRows];  // re-paired activations, 16 B per word row
  float4 sums[MT][kChunkGroups];          // {even p0, odd p0, even p1, odd p1}
  float red[kWaves][MT][kTileCols];       // cross-wave reduction
  int last;                               // this workgroup finishes the tile
};

struct GemvParams {
  const uint16_t* x;      // [M, K] activations (fp16 or bf16 bits)
  const uint8_t* packets; // [(N/128) * NG, S]
  uint16_t* out;          // [M, N] (unused in partials mode)
  float* partials;        // fix-up scratch or reference split-K partials [S_k, M, N]
  uint32_t* counters;     // fix-up arrival counters, one per (tile, m-tile)
  int M, N, K, NG;
  int tiles, mtiles, splits, gps;
  int xcd_remap;
};

template <int G, int MT>
struct StageRegs {
  static constexpr int kUnits = MT * kChunkGroups * (G / 8);
  static constexpr int kPerThread = (kUnits + kThreads - 1) / kThreads;
  uint4 raw[kPerThread];
};

// Issue the global loads of one chunk's activations (16 B = one word row per unit).
template <int G, int MT>
__device__ __forceinline__ void stage_load(StageRegs<G, MT>& st, const GemvParams& p, int row0,
                                           int g0, int n_chunk) {
  constexpr int WR = G / 8;
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < StageRegs<G, MT>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunkGroups;
    const int m = u / (WR * kChunkGroups);
    st.raw[it] = make_uint4(0u, 0u, 0u, 0u);
    if (u < StageRegs<G, MT>::kUnits && gl < n_chunk && row0 + m < p.M) {
      const size_t off = static_cast<size_t>(row0 + m) * p.K +
                         static_cast<size_t>(g0 + gl) * G + static_cast<size_t>(w) * 8;
      st.raw[it] = *reinterpret_cast<const uint4*>(p.x + off);
    }
  }
}

// Re-pair the staged activations into LDS and reduce the per-(row, group, parity) sums.
template <int G, Act A, int MT>
__device__ __forceinline__ void stage_store(Smem<G, MT>& sm, const StageRegs<G, MT>& st,
                                            int n_chunk) {
  constexpr int WR = G / 8;
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < StageRegs<G, MT>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunkGroups;
    const int m = u / (WR * kChunkGroups);
    const uint4 r = st.raw[it];
    // even k: x0 x2 x4 x6 (low halves), odd k: x1 x3 x5 x7 (high halves)
    float se = act_bits_to_float<A>(static_cast<uint16_t>(r.x)) +
               act_bits_to_float<A>(static_cast<uint16_t>(r.y)) +
               act_bits_to_float<A>(static_cast<uint16_t>(r.z)) +
               act_bits_to_float<A>(static_cast<uint16_t>(r.w));
    float so = act_bits_to_float<A>(static_cast<uint16_t>(r.x >> 16)) +
               act_bits_to_float<A>(static_cast<uint16_t>(r.y >> 16)) +
               act_bits_to_float<A>(static_cast<uint16_t>(r.z >> 16)) +
               act_bits_to_float<A>(static_cast<uint16_t>(r.w >> 16));
    // Sum the word rows of one (m, group) that share a parity: they sit in WR consecutive,
    // WR-aligned lanes, so xor-shuffles over 2..WR/2 stay inside the group.
#pragma unroll
    for (int off = 2; off < WR; off <<= 1) {
      se += __shfl_xor(se, off);
      so += __shfl_xor(so, off);
    }
    if (u < StageRegs<G, MT>::kUnits && gl < n_chunk) {
      sm.xs[m][gl][w] = pair_activations(r);
      if (w < 2) {
        float* s = reinterpret_cast<float*>(&sm.sums[m][gl]);
        s[2 * w + 0] = se;
        s[2 * w + 1] = so;
      }
    }
  }
}

// A value the compiler must keep in a VGPR and cannot fold: gfx9 VOP3 encodings take no literal,
// so masks held this way let (w & mask) | bias select a single v_and_or_b32.
__device__ __forceinline__ uint32_t vgpr_constant(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int G>
struct GroupLoad {
  static constexpr int NL = G / 16;
  uint4 w[NL];
  uint2 alpha;
  uint2 beta;
};

template <int G>
__device__ __forceinline__ void load_group(GroupLoad<G>& gl, const uint8_t* packet, int lane) {
  constexpr int QB = kTileCols * G / 2;
  const int c0 = (lane & 31) * 4;
  gl.alpha = *reinterpret_cast<const uint2*>(packet + QB + c0 * 2);
  gl.beta = *reinterpret_cast<const uint2*>(packet + QB + kTileCols * 2 + c0 * 2);
  const uint4* q = reinterpret_cast<const uint4*>(packet) + lane;
#pragma unroll
  for (int i = 0; i < GroupLoad<G>::NL; ++i) {
    gl.w[i] = q[i * 64];
  }
}

template <int G, Act A, int MT>
__device__ __forceinline__ void compute_group(const Smem<G, MT>& sm, const GroupLoad<G>& ld,
                                              int gl, int parity, uint32_t mask_lo,
                                              uint32_t mask_hi, float (&y)[MT][4]) {
  constexpr int NL = G / 16;
  float acc_e[MT][4];
  float acc_o[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc_e[m][j] = 0.0f;
      acc_o[m][j] = 0.0f;
    }
  }

#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int wrow = 2 * i + parity;
    uint4 xp[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      xp[m] = sm.xs[m][gl][wrow];
    }
    const uint32_t words[4] = {ld.w[i].x, ld.w[i].y, ld.w[i].z, ld.w[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t wv = words[j];
      if constexpr (A == Act::kF16) {
        constexpr uint32_t kBias = 0x64006400u;
        const uint32_t e0 = (wv & mask_lo) | kBias;  // 1024+q for k0,k4
        const uint32_t o0 = (wv & mask_hi) | kBias;  // 1024+16q for k1,k5
        const uint32_t w8 = wv >> 8;
        const uint32_t e1 = (w8 & mask_lo) | kBias;  // k2,k6
        const uint32_t o1 = (w8 & mask_hi) | kBias;  // k3,k7
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          acc_e[m][j] = dot2<A>(e0, xp[m].x, acc_e[m][j]);
          acc_o[m][j] = dot2<A>(o0, xp[m].y, acc_o[m][j]);
          acc_e[m][j] = dot2<A>(e1, xp[m].z, acc_e[m][j]);
          acc_o[m][j] = dot2<A>(o1, xp[m].w, acc_o[m][j]);
        }
      } else {
        constexpr uint32_t kBias = 0x43004300u;  // bf16 128.0 pair
        const uint32_t t0 = (wv & mask_lo) | kBias;
        const uint32_t t1 = ((wv >> 4) & mask_lo) | kBias;
        const uint32_t t2 = ((wv >> 8) & mask_lo) | kBias;
        const uint32_t t3 = ((wv >> 12) & mask_lo) | kBias;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          acc_e[m][j] = dot2<A>(t0, xp[m].x, acc_e[m][j]);
          acc_o[m][j] = dot2<A>(t1, xp[m].y, acc_o[m][j]);
          acc_e[m][j] = dot2<A>(t2, xp[m].z, acc_e[m][j]);
          acc_o[m][j] = dot2<A>(t3, xp[m].w, acc_o[m][j]);
        }
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
    const float b = half_bits_to_float(b_bits[j]);
    if constexpr (A == Act::kF16) {
      const float a16 = a * 0.0625f;
      const float ce = fmaf(-1024.0f, a, b);  // beta - 1024 alpha
      const float co = fmaf(-64.0f, a, b);    // beta - 64 alpha
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 s = sm.sums[m][gl];
        const float se = parity ? s.z : s.x;
        const float so = parity ? s.w : s.y;
        float t = fmaf(a, acc_e[m][j], ce * se);
        t = fmaf(a16, acc_o[m][j], t);
        t = fmaf(co, so, t);
        y[m][j] += t;
      }
    } else {
      const float c = fmaf(-128.0f, a, b);  // beta - 128 alpha
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 s = sm.sums[m][gl];
        const float sp = parity ? (s.z + s.w) : (s.x + s.y);
        const float t = fmaf(a, acc_e[m][j] + acc_o[m][j], c * sp);
        y[m][j] += t;
      }
    }
  }
}

template <int G, Act A, int MT, GemvMode MODE>
__global__ void __launch_bounds__(kThreads)
w4a16_gemv_kernel(GemvParams p) {
  __shared__ Smem<G, MT> sm;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int parity = lane >> 5;

  // Logical workgroup id: keep consecutive ids (the splits of one tile) on one XCD.
  const int total = p.tiles * p.mtiles * p.splits;
  int L = static_cast<int>(blockIdx.x);
  if (p.xcd_remap) {
    L = (L & 7) * (total >> 3) + (L >> 3);
  }
  const int split = L % p.splits;
  const int rest = L / p.splits;
  const int tile = rest % p.tiles;
  const int mtile = rest / p.tiles;
  const int row0 = mtile * MT;

  const int g_begin = split * p.gps;
  const int g_end = min(p.NG, g_begin + p.gps);
  const size_t stride = static_cast<size_t>(packet_stride_bytes(G));
  const uint8_t* tile_packets = p.packets + static_cast<size_t>(tile) * p.NG * stride;

  float y[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      y[m][j] = 0.0f;
    }
  }

  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  for (int g0 = g_begin; g0 < g_end; g0 += kChunkGroups) {
    const int n_chunk = min(kChunkGroups, g_end - g0);
    if (g0 != g_begin) {
      lds_barrier();  // previous chunk's readers are done with xs / sums
    }
    // Activation loads first, then this wave's first weight group, so the LDS writes below only
    // wait for the activations while the weights stay in flight across the barrier.
    StageRegs<G, MT> st;
    stage_load<G, MT>(st, p, row0, g0, n_chunk);
    GroupLoad<G> buf_a;
    GroupLoad<G> buf_b;
    int gl = wave;
    if (gl < n_chunk) {
      load_group<G>(buf_a, tile_packets + static_cast<size_t>(g0 + gl) * stride, lane);
    }
    stage_store<G, A, MT>(sm, st, n_chunk);
    lds_barrier();
    // Ping-pong between two register buffers: the next group's loads are issued before the
    // current group is computed.
    while (gl < n_chunk) {
      if (gl + kWaves < n_chunk) {
        load_group<G>(buf_b, tile_packets + static_cast<size_t>(g0 + gl + kWaves) * stride, lane);
      }
      compute_group<G, A, MT>(sm, buf_a, gl, parity, mask_lo, mask_hi, y);
      gl += kWaves;
      if (gl >= n_chunk) {
        break;
      }
      if (gl + kWaves < n_chunk) {
        load_group<G>(buf_a, tile_packets + static_cast<size_t>(g0 + gl + kWaves) * stride, lane);
      }
      compute_group<G, A, MT>(sm, buf_b, gl, parity, mask_lo, mask_hi, y);
      gl += kWaves;
    }
  }

  // Lanes l and l^32 hold the two word-row parities of the same four columns.
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      y[m][j] += __shfl_xor(y[m][j], 32);
    }
  }
  if (parity == 0) {
    const int c0 = lane * 4;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      *reinterpret_cast<float4*>(&sm.red[wave][m][c0]) = make_float4(y[m][0], y[m][1], y[m][2], y[m][3]);
    }
  }
  __syncthreads();

  const int col_base = tile * kTileCols;
  constexpr int kOut = MT * kTileCols;

  if constexpr (MODE == GemvMode::kDirect) {
    for (int idx = tid; idx < kOut; idx += kThreads) {
      const int m = idx / kTileCols;
      const int c = idx % kTileCols;
      if (row0 + m < p.M) {
        const float v = sm.red[0][m][c] + sm.red[1][m][c] + sm.red[2][m][c] + sm.red[3][m][c];
        p.out[static_cast<size_t>(row0 + m) * p.N + col_base + c] = float_to_act_bits<A>(v);
      }
    }
  } else if constexpr (MODE == GemvMode::kPartials) {
    for (int idx = tid; idx < kOut; idx += kThreads) {
      const int m = idx / kTileCols;
      const int c = idx % kTileCols;
      if (row0 + m < p.M) {
        const float v = sm.red[0][m][c] + sm.red[1][m][c] + sm.red[2][m][c] + sm.red[3][m][c];
        p.partials[(static_cast<size_t>(split) * p.M + row0 + m) * p.N + col_base + c] = v;
      }
    }
  } else {
    // Cross-workgroup hand-off without cache-wide maintenance: the partials and the counter are
    // accessed only through agent-scope relaxed atomics, which the gfx950 memory model serves
    // coherently across XCDs (their L2s are not coherent with each other) without the
    // whole-L2 write-back / invalidate an agent-scope fence costs. Ordering between the partial
    // stores and the counter increment comes from waiting for the stores to complete (vmcnt(0))
    // before the workgroup barrier that precedes the increment.
    const int tm = mtile * p.tiles + tile;
    float* ws = p.partials + static_cast<size_t>(tm) * p.splits * kOut;
    for (int idx = tid; idx < kOut; idx += kThreads) {
      const int m = idx / kTileCols;
      const int c = idx % kTileCols;
      const float v = sm.red[0][m][c] + sm.red[1][m][c] + sm.red[2][m][c] + sm.red[3][m][c];
      __hip_atomic_store(&ws[static_cast<size_t>(split) * kOut + idx], v, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev =
          __hip_atomic_fetch_add(&p.counters[tm], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sm.last = (prev == static_cast<uint32_t>(p.splits - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (sm.last) {
      for (int idx = tid; idx < kOut; idx += kThreads) {
        const int m = idx / kTileCols;
        const int c = idx % kTileCols;
        if (row0 + m < p.M) {
          float v = 0.0f;
          for (int s = 0; s < p.splits; ++s) {
            v += __hip_atomic_load(&ws[static_cast<size_t>(s) * kOut + idx], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          }
          p.out[static_cast<size_t>(row0 + m) * p.N + col_base + c] = float_to_act_bits<A>(v);
        }
      }
      if (tid == 0) {
        __hip_atomic_store(&p.counters[tm], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <int G, Act A, int MT, GemvMode MODE>
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
  p.splits = l.splits;
  p.gps = l.gps;
  const int total = p.tiles * p.mtiles * p.splits;
  p.xcd_remap = (total % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((w4a16_gemv_kernel<G, A, MT, MODE>), dim3(total), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

template <int G, Act A, GemvMode MODE>
hipError_t dispatch_mt(const GemvLaunch& l, hipStream_t stream) {
  switch (l.m_tile) {
    case 1: return launch_t<G, A, 1, MODE>(l, stream);
    case 2: return launch_t<G, A, 2, MODE>(l, stream);
    case 4: return launch_t<G, A, 4, MODE>(l, stream);
    default: return launch_t<G, A, 8, MODE>(l, stream);
  }
}

template <int G, Act A>
hipError_t dispatch_mode(const GemvLaunch& l, hipStream_t stream) {
  switch (l.mode) {
    case GemvMode::kDirect: return dispatch_mt<G, A, GemvMode::kDirect>(l, stream);
    case GemvMode::kPartials: return dispatch_mt<G, A, GemvMode::kPartials>(l, stream);
    default: return dispatch_mt<G, A, GemvMode::kFixup>(l, stream);
  }
}

}  // namespace

int gemv_m_tile_for_batch(int batch) {
  if (batch <= 1) return 1;
  if (batch <= 2) return 2;
  if (batch <= 4) return 4;
  return 8;
}

hipError_t launch_w4a16_gemv(const GemvLaunch& l, hipStream_t stream) {
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? dispatch_mode<64, Act::kF16>(l, stream)
                              : dispatch_mode<64, Act::kBF16>(l, stream);
  }
  return l.act == Act::kF16 ? dispatch_mode<128, Act::kF16>(l, stream)
                            : dispatch_mode<128, Act::kBF16>(l, stream);
}

}  // namespace fk
