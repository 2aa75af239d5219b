// Building blocks of the native-slab GEMV kernels (w4a16_gemv_native.hip: the plain forward;
// w4a16_gemv_fused.hip: the forward with an RMSNorm prologue or a SiLU-and-multiply epilogue).
// The W4A16 GEMV / small-batch GEMM (dot2 path) over the native slab formats (PacketFormat in
// w4a16_device.h): kNativeSym and kNativeAsym, 1-8 activation rows. Same math, staging, stream-K
// work split and fix-up as the reference-packet kernel (w4a16_gemv_kernels.h), with a lane mapping
// that follows the slab's quarter order:
//
//  * A workgroup streams runs of one 32-column slice; the slice's groups are one contiguous byte
//    range, and every wave-wide load reads 1 KB (G = 128: two loads per group; G = 64: one).
//  * Lane l = 16t + n owns quarter t (U = G/32 consecutive code words, 8U values of k) of columns
//    n and n + 16. Per group it therefore applies scales to two columns, not four, and reads U
//    16-byte activation vectors per row (broadcast: the 16 lanes of a quarter read the same one).
//  * The unpack bias and the offsets fold into per-(row, group, quarter) constants formed while
//    staging, so the epilogue is short. The even (1024 + q) and odd (64 + q) nibble unpacks
//    add into one accumulator:
//    acc = C + sum (1024 + q) x_e + (64 + q) x_o. kNativeSym: beta = half_rn(-8 alpha) = -8 alpha
//    exactly, C = -1032 S_even - 72 S_odd and y += alpha * acc. kNativeAsym:
//    C = -1024 S_even - 64 S_odd and y += alpha * acc + beta * (S_even + S_odd), beta =
//    half_rn(-alpha * zp) rebuilt from the stored zero point (both columns in one packed fp16
//    multiply).
//  * The four quarters of a column are summed across lanes (xor 16, xor 32) once per run, then
//    across waves in LDS.
#pragma once

#include "w4a16_gemv_kernels.h"

namespace fk {
namespace {

constexpr int kCW = kSliceCols;

template <int G, int MT>
struct NativeSmem {
  static constexpr int kChunk = chunk_groups<G, MT, kCW>();
  static constexpr int kWordRows = G / 8;
  uint4 xs[MT][kChunk][kWordRows];  // re-paired fp16 activations, 16 B per word row
  float2 sums[MT][kChunk][4];       // offset terms per quarter of the group (native_stage_store)
  float scale[MT][kChunk];          // power of two undoing the bf16 staging scale
  float red[kWaves][MT][kCW];       // cross-wave reduction
  float aux[MT][kCW];               // SiLU-and-multiply epilogue: the gate half's totals
  float inv_rms[MT];                // RMSNorm prologue: 1 / rms of each row
  int last;                         // this workgroup finishes the slice

  // The staged activations as native_stage_unit writes and native_compute_group reads them.
  __device__ uint4 x_at(int m, int gl, int i) const { return xs[m][gl][i]; }
  __device__ float2 sums_at(int m, int gl, int t) const { return sums[m][gl][t]; }
  __device__ float scale_at(int m, int gl) const { return scale[m][gl]; }
  __device__ void set_x(int m, int gl, int i, uint4 v) { xs[m][gl][i] = v; }
  __device__ void set_sums(int m, int gl, int t, float2 v) { sums[m][gl][t] = v; }
  __device__ void set_scale(int m, int gl, float v) { scale[m][gl] = v; }
};

// RMSNorm prologue: gamma for the staged units (the same k as the activation units).
template <int G, int MT>
struct NormRegs {
  uint4 raw[StageRegs<G, MT, kSliceCols>::kPerThread];
};

template <int G, int MT>
__device__ __forceinline__ void norm_stage_load(NormRegs<G, MT>& nr, const GemvParams& p, int g0,
                                                int n_chunk) {
  constexpr int WR = G / 8;
  constexpr int kChunk = chunk_groups<G, MT, kSliceCols>();
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < StageRegs<G, MT, kSliceCols>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunk;
    // clamped and unconditional like stage_load; the staged x of a unit outside the chunk is
    // zero, and so is its normalised value
    nr.raw[it] = *reinterpret_cast<const uint4*>(
        p.norm_weight + static_cast<size_t>(g0 + min(gl, n_chunk - 1)) * G +
        static_cast<size_t>(w) * 8);
  }
}

// Two activation values of a word normalised as the unfused pipeline does:
// round(gamma * round(x * inv_rms)) in the activation dtype.
template <Act A>
__device__ __forceinline__ uint32_t norm_pair(uint32_t xw, uint32_t gw, float inv_rms) {
  uint32_t r = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float x = act_bits_to_float<A>(static_cast<uint16_t>(xw >> (16 * h)));
    const float g = act_bits_to_float<A>(static_cast<uint16_t>(gw >> (16 * h)));
    const float xn = act_bits_to_float<A>(float_to_act_bits<A>(x * inv_rms));
    r |= static_cast<uint32_t>(float_to_act_bits<A>(g * xn)) << (16 * h);
  }
  return r;
}

// Sum of squares of two activations of a word.
template <Act A>
__device__ __forceinline__ float sum_sq_word(uint32_t w, float acc) {
  const float a = act_bits_to_float<A>(static_cast<uint16_t>(w));
  const float b = act_bits_to_float<A>(static_cast<uint16_t>(w >> 16));
  return fmaf(b, b, fmaf(a, a, acc));
}

// Reduces the per-thread sums of squares of rows row0 .. row0 + MT - 1 and writes
// 1 / sqrt(mean(x^2) + eps) to sm.inv_rms. Uses sm.red; ends with a workgroup barrier.
template <int G, int MT>
__device__ __forceinline__ void native_rms_finish(NativeSmem<G, MT>& sm, const GemvParams& p,
                                                  float (&ss)[MT], int lane, int wave) {
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      ss[m] += __shfl_xor(ss[m], off);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      sm.red[wave][m][0] = ss[m];
    }
  }
  __syncthreads();
  if (tid < MT) {
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      total += sm.red[w][tid][0];
    }
    sm.inv_rms[tid] = 1.0f / sqrtf(total / static_cast<float>(p.K) + p.eps);
  }
  __syncthreads();
}

// 1 / sqrt(mean(x^2) + eps) of rows row0 .. row0 + MT - 1 into sm.inv_rms (fp32 sums; every
// workgroup forms it for its own rows), loading and reducing in one go.
template <int G, Act A, int MT>
__device__ __forceinline__ void native_row_inv_rms(NativeSmem<G, MT>& sm, const GemvParams& p,
                                                   int row0, int lane, int wave) {
  const int tid = static_cast<int>(threadIdx.x);
  float ss[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    ss[m] = 0.0f;
    if (row0 + m < p.M) {
      const uint16_t* row = p.x + static_cast<size_t>(row0 + m) * p.K;
      for (int k8 = tid; k8 < p.K / 8; k8 += kThreads) {
        const uint4 v = *reinterpret_cast<const uint4*>(row + static_cast<size_t>(k8) * 8);
        ss[m] = sum_sq_word<A>(v.x, ss[m]);
        ss[m] = sum_sq_word<A>(v.y, ss[m]);
        ss[m] = sum_sq_word<A>(v.z, ss[m]);
        ss[m] = sum_sq_word<A>(v.w, ss[m]);
      }
    }
  }
  native_rms_finish<G, MT>(sm, p, ss, lane, wave);
}

// One activation row of up to kRmsRegs * kThreads * 8 values held in registers, so that its
// loads can be issued ahead of the weight loads and its reduction done behind them.
constexpr int kRmsRegs = 4;
struct RmsRegs {
  uint4 v[kRmsRegs];
};

__device__ __forceinline__ bool rms_fits_registers(const GemvParams& p) {
  return p.K <= kRmsRegs * kThreads * 8;
}

__device__ __forceinline__ void rms_preload(RmsRegs& rr, const GemvParams& p, int row) {
  const int tid = static_cast<int>(threadIdx.x);
  const uint16_t* x = p.x + static_cast<size_t>(row) * p.K;
  const int words = p.K / 8;
#pragma unroll
  for (int it = 0; it < kRmsRegs; ++it) {
    const int k8 = min(it * kThreads + tid, words - 1);  // clamped; the excess is masked in use
    rr.v[it] = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(k8) * 8);
  }
}

template <Act A>
__device__ __forceinline__ float rms_sum(const RmsRegs& rr, const GemvParams& p) {
  const int tid = static_cast<int>(threadIdx.x);
  float ss = 0.0f;
#pragma unroll
  for (int it = 0; it < kRmsRegs; ++it) {
    if (it * kThreads + tid < p.K / 8) {
      ss = sum_sq_word<A>(rr.v[it].x, ss);
      ss = sum_sq_word<A>(rr.v[it].y, ss);
      ss = sum_sq_word<A>(rr.v[it].z, ss);
      ss = sum_sq_word<A>(rr.v[it].w, ss);
    }
  }
  return ss;
}

template <int G>
struct NativeLoad {
  static constexpr int kVecs = G == 128 ? 2 : 1;
  uint4 w[kVecs];
  uint32_t alpha;  // alpha of columns n (bits 0-15) and n + 16
  uint32_t zp;     // kNativeAsym: -zp of columns n (bits 0-15) and n + 16 as fp16
};

template <int G, PacketFormat F>
__device__ __forceinline__ void native_load(NativeLoad<G>& ld, const uint8_t* slab, int lane) {
#pragma unroll
  for (int v = 0; v < NativeLoad<G>::kVecs; ++v) {
    ld.w[v] = stream_load16(slab + v * 1024 + lane * 16);
  }
  const uint8_t* record = slab + native_record_offset(G) + native_record_bytes(F) * (lane % 16);
  if constexpr (F == PacketFormat::kNativeAsym) {
    const uint2 r = stream_load8(record);
    ld.alpha = r.x;
    ld.zp = r.y;
  } else {
    ld.alpha = stream_load4(record);
  }
}

// Half a G = 128 slab: the 1 KB of code words of columns 16 * half .. 16 * half + 15 (into
// ld.w[0]) and the lane's record (both columns' scales; the kernel picks its half).
template <int G, PacketFormat F>
__device__ __forceinline__ void native_load_half(NativeLoad<G>& ld, const uint8_t* slab, int lane,
                                                 int half) {
  static_assert(G == 128, "half slabs need G = 128");
  ld.w[0] = stream_load16(slab + half * 1024 + lane * 16);
  const uint8_t* record = slab + native_record_offset(G) + native_record_bytes(F) * (lane % 16);
  if constexpr (F == PacketFormat::kNativeAsym) {
    const uint2 r = stream_load8(record);
    ld.alpha = r.x;
    ld.zp = r.y;
  } else {
    ld.alpha = stream_load4(record);
  }
}

// Word j of the lane's unit of column n + 16 i.
template <int G>
__device__ __forceinline__ uint32_t unit_word(const NativeLoad<G>& ld, int i, int j) {
  if constexpr (G == 128) {
    const uint4 v = ld.w[i];
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
  } else {
    const uint4 v = ld.w[0];
    return i == 0 ? (j == 0 ? v.x : v.y) : (j == 0 ? v.z : v.w);
  }
}

// One staged unit (word row w of group gl of row m: 8 activations) into LDS: converted (bf16) and
// re-paired, with the {even, odd} sums over its quarter (U consecutive word rows, U consecutive
// lanes: every lane of a quarter must call this together). S is the LDS view (NativeSmem or
// StreamLds).
template <int G, Act A, PacketFormat F, class S>
__device__ __forceinline__ void native_stage_unit(S& sm, uint4 r, int m, int gl, int w) {
  constexpr int WR = G / 8;
  constexpr int U = native_unit_words(G);
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
  // Both nibble positions accumulate into one sum, (1024 + q) x_e + (64 + q) x_o (the high
  // nibbles unpack as 64 + q), so the activations are staged as they are, re-paired
  // (x0,x4) (x1,x5) (x2,x6) (x3,x7).
  const uint4 xp = pair_activations(r);
  // even k: x0 x2 x4 x6 (xp.x, xp.z), odd k: x1 x3 x5 x7 (xp.y, xp.w); v_dot2 by (1, 1) adds
  // two fp16 values into an fp32 sum
  constexpr uint32_t kOnes = 0x3c003c00u;
  float se = dot2<Act::kF16>(xp.z, kOnes, dot2<Act::kF16>(xp.x, kOnes, 0.0f));
  float so = dot2<Act::kF16>(xp.w, kOnes, dot2<Act::kF16>(xp.y, kOnes, 0.0f));
  se = group_sum<U>(se);
  so = group_sum<U>(so);
  sm.set_x(m, gl, w, xp);
  // The offset terms of the epilogue divided by alpha, per (row, group, quarter):
  // kNativeSym (beta = -8 alpha): -1032 S_e - 72 S_o; kNativeAsym: -1024 S_e - 64 S_o, plus
  // S_e + S_o for the beta * S term. Every lane of the quarter (and, for the scale, of the group)
  // holds the same value and writes it, so the staging has no branch.
  sm.set_sums(m, gl, w / U,
              F == PacketFormat::kNativeSym
                  ? make_float2(fmaf(-1032.0f, se, -72.0f * so), 0.0f)
                  : make_float2(fmaf(-1024.0f, se, -64.0f * so), se + so));
  sm.set_scale(m, gl, undo);
}

// Activations of one chunk into LDS: the staged, re-paired values as in the reference-packet
// kernel, and the {even, odd} sums over each quarter (U consecutive word rows, U consecutive
// lanes here).
template <int G, Act A, int MT, PacketFormat F, bool kNorm>
__device__ __forceinline__ void native_stage_store(NativeSmem<G, MT>& sm, StageRegs<G, MT, kCW>& st,
                                                   const NormRegs<G, MT>& nr, int n_chunk) {
  constexpr int WR = G / 8;
  constexpr int kChunk = NativeSmem<G, MT>::kChunk;
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int it = 0; it < StageRegs<G, MT, kCW>::kPerThread; ++it) {
    const int u = it * kThreads + tid;
    const int w = u % WR;
    const int gl = (u / WR) % kChunk;
    const int m = u / (WR * kChunk);
    // Units past the chunk (a short last chunk, or K shorter than a chunk) stage nothing; a
    // group's WR lanes share gl, so the cross-lane sums below stay within live lanes.
    if (u >= StageRegs<G, MT, kCW>::kUnits || gl >= n_chunk) {
      continue;
    }
    uint4 r = st.unit(it);
    if constexpr (kNorm) {
      const float inv = sm.inv_rms[m < MT ? m : 0];
      const uint4 gw = nr.raw[it];
      r.x = norm_pair<A>(r.x, gw.x, inv);
      r.y = norm_pair<A>(r.y, gw.y, inv);
      r.z = norm_pair<A>(r.z, gw.z, inv);
      r.w = norm_pair<A>(r.w, gw.w, inv);
    }
    native_stage_unit<G, A, F>(sm, r, m, gl, w);
  }
}

// kCols = 2: the lane's two columns n and n + 16 (ld holds both halves of the slab). kCols = 1
// (G = 128, native_load_half): column n + 16 * half only, its words in ld.w[0]; y[m][0] gets it.
template <int G, Act A, int MT, PacketFormat F, class S, int kCols = 2>
__device__ __forceinline__ void native_compute_group(const S& sm,
                                                     const NativeLoad<G>& ld, int gl, int t,
                                                     uint32_t mask_lo, uint32_t mask_hi,
                                                     float (&y)[MT][2], int half = 0) {
  static_assert(kCols == 2 || G == 128, "half slabs need G = 128");
  constexpr int U = native_unit_words(G);
  // One accumulator per (row, column): with the odd nibbles unpacked as 64 + q both nibble
  // positions add into it. A single row keeps a second one so that the dependent dot2 chains are
  // interleaved in pairs.
  constexpr int kAcc = MT == 1 ? 2 : 1;
  float acc[MT][2][kAcc];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    // The offset term divided by alpha seeds the accumulator (see native_stage_store).
    const float seed = sm.sums_at(m, gl, t).x;
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
      acc[m][i][0] = seed;
      if constexpr (kAcc == 2) {
        acc[m][i][kAcc - 1] = 0.0f;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    uint32_t e0[2], o0[2], e1[2], o1[2];
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
      const uint32_t wv = unit_word<G>(ld, i, j);
      const uint32_t w8 = wv >> 8;
      e0[i] = (wv & mask_lo) | kBiasLow;   // 1024+q for k0,k4
      o0[i] = (wv & mask_hi) | kBiasHigh;  // 64+q for k1,k5
      e1[i] = (w8 & mask_lo) | kBiasLow;   // k2,k6
      o1[i] = (w8 & mask_hi) | kBiasHigh;  // k3,k7
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint4 xp = sm.x_at(m, gl, U * t + j);
#pragma unroll
      for (int i = 0; i < kCols; ++i) {
        float& a0 = acc[m][i][0];
        float& a1 = acc[m][i][kAcc - 1];
        a0 = dot2<Act::kF16>(e0[i], xp.x, a0);
        a1 = dot2<Act::kF16>(o0[i], xp.y, a1);
        a0 = dot2<Act::kF16>(e1[i], xp.z, a0);
        a1 = dot2<Act::kF16>(o1[i], xp.w, a1);
      }
    }
  }
  // kNativeAsym: beta = half_rn(-alpha * zp) for both columns with one packed fp16 multiply of
  // the alphas by the stored (-zp) pair.
  uint32_t beta_pair = 0;
  if constexpr (F == PacketFormat::kNativeAsym) {
    beta_pair = __builtin_bit_cast(
        uint32_t, __builtin_bit_cast(half2_t, ld.alpha) * __builtin_bit_cast(half2_t, ld.zp));
  }
#pragma unroll
  for (int i = 0; i < kCols; ++i) {
    const int sh = 16 * (kCols == 2 ? i : half);
    const float a = half_bits_to_float(static_cast<uint16_t>(ld.alpha >> sh));
    const float b = half_bits_to_float(static_cast<uint16_t>(beta_pair >> sh));
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float sum = acc[m][i][0];
      if constexpr (kAcc == 2) {
        sum += acc[m][i][1];
      }
      if constexpr (A == Act::kBF16) {
        // the staged activations carry a power-of-two scale per (row, group)
        float t_sum = a * sum;
        if constexpr (F == PacketFormat::kNativeAsym) {
          t_sum = fmaf(b, sm.sums_at(m, gl, t).y, t_sum);
        }
        y[m][i] = fmaf(t_sum, sm.scale_at(m, gl), y[m][i]);
      } else {
        y[m][i] = fmaf(a, sum, y[m][i]);
        if constexpr (F == PacketFormat::kNativeAsym) {
          y[m][i] = fmaf(b, sm.sums_at(m, gl, t).y, y[m][i]);
        }
      }
    }
  }
}

// One row's staged operands of one group for a lane (quarter t): its U activation words, the
// {offset, sum} pair and (bf16) the staging scale, read from LDS ahead of the slab they serve.
template <int G>
struct RowOps {
  uint4 x[native_unit_words(G)];
  float2 sums;
  float scale;
};

template <int G, Act A, class S>
__device__ __forceinline__ void native_load_ops(const S& sm, int gl, int t, RowOps<G>& o) {
  constexpr int U = native_unit_words(G);
#pragma unroll
  for (int j = 0; j < U; ++j) {
    o.x[j] = sm.x_at(0, gl, U * t + j);
  }
  o.sums = sm.sums_at(0, gl, t);
  o.scale = A == Act::kBF16 ? sm.scale_at(0, gl) : 1.0f;
}

// native_compute_group for one row from operands already in registers (RowOps): the same
// arithmetic in the same order.
template <int G, Act A, PacketFormat F, int kCols = 2>
__device__ __forceinline__ void native_compute_ops(const RowOps<G>& o, const NativeLoad<G>& ld,
                                                   uint32_t mask_lo, uint32_t mask_hi,
                                                   float (&y)[1][2], int half = 0) {
  static_assert(kCols == 2 || G == 128, "half slabs need G = 128");
  constexpr int U = native_unit_words(G);
  float acc[2][2];
#pragma unroll
  for (int i = 0; i < kCols; ++i) {
    acc[i][0] = o.sums.x;
    acc[i][1] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint4 xp = o.x[j];
#pragma unroll
    for (int i = 0; i < kCols; ++i) {
      const uint32_t wv = unit_word<G>(ld, i, j);
      const uint32_t w8 = wv >> 8;
      const uint32_t e0 = (wv & mask_lo) | kBiasLow;
      const uint32_t o0 = (wv & mask_hi) | kBiasHigh;
      const uint32_t e1 = (w8 & mask_lo) | kBiasLow;
      const uint32_t o1 = (w8 & mask_hi) | kBiasHigh;
      acc[i][0] = dot2<Act::kF16>(e0, xp.x, acc[i][0]);
      acc[i][1] = dot2<Act::kF16>(o0, xp.y, acc[i][1]);
      acc[i][0] = dot2<Act::kF16>(e1, xp.z, acc[i][0]);
      acc[i][1] = dot2<Act::kF16>(o1, xp.w, acc[i][1]);
    }
  }
  uint32_t beta_pair = 0;
  if constexpr (F == PacketFormat::kNativeAsym) {
    beta_pair = __builtin_bit_cast(
        uint32_t, __builtin_bit_cast(half2_t, ld.alpha) * __builtin_bit_cast(half2_t, ld.zp));
  }
#pragma unroll
  for (int i = 0; i < kCols; ++i) {
    const int sh = 16 * (kCols == 2 ? i : half);
    const float a = half_bits_to_float(static_cast<uint16_t>(ld.alpha >> sh));
    const float b = half_bits_to_float(static_cast<uint16_t>(beta_pair >> sh));
    const float sum = acc[i][0] + acc[i][1];
    if constexpr (A == Act::kBF16) {
      float t_sum = a * sum;
      if constexpr (F == PacketFormat::kNativeAsym) {
        t_sum = fmaf(b, o.sums.y, t_sum);
      }
      y[0][i] = fmaf(t_sum, o.scale, y[0][i]);
    } else {
      y[0][i] = fmaf(a, sum, y[0][i]);
      if constexpr (F == PacketFormat::kNativeAsym) {
        y[0][i] = fmaf(b, o.sums.y, y[0][i]);
      }
    }
  }
}

// Groups [g_lo, g_hi) of one slice: stage the activations of up to kChunk groups in LDS, then
// each wave streams groups g_lo + wave, g_lo + wave + 4, ... through D register buffers (as the
// reference-packet kernel's stream_groups).
//
// rms_first (kNorm): form the rows' 1 / rms at the start of the first chunk. One row whose K fits
// RmsRegs issues the row's loads first and reduces them after the chunk's weight loads are in
// flight (the in-order load counter then waits for the row alone); otherwise the row is loaded
// and reduced before any other load.
// staged: [g_lo, g_hi) is one chunk whose activations a previous call left in LDS; they are
// reused as they are (no loads, no staging, no barrier).
template <int G, Act A, int MT, PacketFormat F, bool kNorm>
__device__ __forceinline__ void native_stream_groups(NativeSmem<G, MT>& sm, const GemvParams& p,
                                                     const uint8_t* slabs, int row0, int g_lo,
                                                     int g_hi, int lane, int wave,
                                                     uint32_t mask_lo, uint32_t mask_hi,
                                                     float (&y)[MT][2], bool rms_first = false,
                                                     bool staged = false, bool pair = false) {
  constexpr int kChunk = NativeSmem<G, MT>::kChunk;
  // 8 KB of weights in flight per wave (4 groups at G = 128, 8 at G = 64): measured on MI355X,
  // deeper pipelines (8 or 16 KB per wave) lower the achieved HBM bandwidth of every decode shape.
  constexpr int D = 8 / NativeLoad<G>::kVecs / (MT >= 8 ? 2 : 1);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  const int t = lane / 16;
  for (int g0 = g_lo; g0 < g_hi; g0 += kChunk) {
    const int n_chunk = min(kChunk, g_hi - g0);
    if (g0 != g_lo) {
      lds_barrier();  // previous chunk's readers are done with xs / sums
    }
    bool rms_late = false;
    RmsRegs rr;
    if constexpr (kNorm) {
      if (rms_first && g0 == g_lo) {
        if (MT == 1 && rms_fits_registers(p)) {
          rms_preload(rr, p, row0);
          rms_late = true;
        } else {
          native_row_inv_rms<G, A, MT>(sm, p, row0, lane, wave);
        }
      }
    }
    StageRegs<G, MT, kCW> st;
    NormRegs<G, MT> nr;
    if (!staged) {
      stage_load<G, MT, kCW>(st, p, row0, g0, n_chunk);
      if constexpr (kNorm) {
        norm_stage_load<G, MT>(nr, p, g0, n_chunk);
      }
    }
    // Slice pairs: waves 0 and 2 stream the first slice, waves 1 and 3 the second, each over
    // every other group of the chunk; a single slice is shared by all four waves.
    const int ws = pair ? (wave >> 1) : wave;
    const int lw = pair ? 1 : 2;  // log2 of the waves per slice
    const int W = 1 << lw;
    const int n_w = n_chunk > ws ? (n_chunk - ws + W - 1) >> lw : 0;
    const int t_last = max(n_w - 1, 0);
    const int gl_base = n_w > 0 ? ws : n_chunk - 1;
    const uint8_t* gp = slabs + (pair ? static_cast<size_t>(wave & 1) * p.NG * stride : 0) +
                        static_cast<size_t>(g0 + gl_base) * stride;
    const size_t step = static_cast<size_t>(W) * stride;
    NativeLoad<G> buf[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      native_load<G, F>(buf[d], gp + static_cast<size_t>(min(d, t_last)) * step, lane);
    }
    if constexpr (kNorm) {
      if (rms_late) {
        float ss[MT] = {};
        ss[0] = rms_sum<A>(rr, p);
        native_rms_finish<G, MT>(sm, p, ss, lane, wave);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load above the first use of the activations
    if (!staged) {
      native_stage_store<G, A, MT, F, kNorm>(sm, st, nr, n_chunk);
      lds_barrier();
    }
    const int n_blocks = (n_w + D - 1) / D;
    int t0 = 0;
    for (int blk = 0; blk + 1 < n_blocks; ++blk, t0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        native_compute_group<G, A, MT, F>(sm, buf[d], ws + ((t0 + d) << lw), t, mask_lo,
                                          mask_hi, y);
        native_load<G, F>(buf[d], gp + static_cast<size_t>(min(t0 + D + d, t_last)) * step, lane);
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (t0 + d < n_w) {
        native_compute_group<G, A, MT, F>(sm, buf[d], ws + ((t0 + d) << lw), t, mask_lo,
                                          mask_hi, y);
      }
    }
    // The loads of skipped tail slots are never consumed; retire them here, or the compiler's
    // wait for their registers lands between the next chunk's first loads and serialises them.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  }
}

// Sums a run's per-lane totals over the quarters of each column (lanes n, n+16, n+32, n+48) and
// writes each wave's 32 column totals to sm.red; ends with a workgroup barrier.
template <int G, int MT>
__device__ __forceinline__ void native_reduce_run(NativeSmem<G, MT>& sm, float (&y)[MT][2],
                                                  int lane, int wave) {
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      y[m][i] += __shfl_xor(y[m][i], 16);
      y[m][i] += __shfl_xor(y[m][i], 32);
    }
  }
  if (lane < 16) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      sm.red[wave][m][lane] = y[m][0];
      sm.red[wave][m][lane + 16] = y[m][1];
    }
  }
  __syncthreads();
}

// Column c of a slice pair (0-31 first slice, 32-63 second): waves 0 and 2 hold the first
// slice's totals, waves 1 and 3 the second's.
template <int G, int MT>
__device__ __forceinline__ float native_pair_red_sum(const NativeSmem<G, MT>& sm, int m, int c) {
  const int s = c >> 5;
  return sm.red[s][m][c & 31] + sm.red[s + 2][m][c & 31];
}

template <int G, int MT>
__device__ __forceinline__ float native_red_sum(const NativeSmem<G, MT>& sm, int m, int c) {
  float v = sm.red[0][m][c];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    v += sm.red[w][m][c];
  }
  return v;
}

// Stream-K over (m-tile, tile, slice, group) units, as the reference-packet kernel with 32-column
// slices: workgroup b owns units [b*per, (b+1)*per); slices split between workgroups are finished
// by finish_run.
//
// kNorm: the RMSNorm prologue (GemvFuse::kRmsNorm); every run first forms 1 / rms of its rows.
template <int G, Act A, int MT, PacketFormat F, bool kNorm>
__global__ void __launch_bounds__(kThreads, min_waves_per_eu<MT>())
w4a16_gemv_native_kernel(GemvParams p) {
  __shared__ NativeSmem<G, MT> sm;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  const int grid = p.grid;
  if constexpr (kNorm) {
    }
  int b = static_cast<int>(blockIdx.x);
  b = p.xcd_remap != 0 ? (b & 7) * p.xcd_remap + (b >> 3) : b;
  const uint32_t total_units =
      static_cast<uint32_t>(p.tiles) * kSlicesPerTile * p.mtiles * p.NG;
  const uint32_t u_begin = static_cast<uint32_t>(b) * p.per;
  const uint32_t u_end = min(total_units, u_begin + p.per);
  uint32_t u = u_begin;
  const bool pair = p.pair != 0;
  while (u < u_end) {
    const RunPos r = run_pos(p, u, u_end, kSlicesPerTile);
    const int T = r.T;
    const int g_lo = r.g_lo;
    const int g_hi = r.g_hi;
    const int slice = r.slice;
    const int tile = r.tile;
    const int row0 = r.mtile * MT;
    const uint8_t* slabs =
        p.packets + (static_cast<size_t>(tile) * kSlicesPerTile + slice) * p.NG * stride;
    float y[MT][2] = {};
    native_stream_groups<G, A, MT, F, kNorm>(sm, p, slabs, row0, g_lo, g_hi, lane, wave, mask_lo,
                                             mask_hi, y, /*rms_first=*/true, /*staged=*/false,
                                             pair);
    native_reduce_run<G, MT>(sm, y, lane, wave);
    if (pair) {
      // Runs are whole slice pairs (the host checks per % (2 NG) == 0): written directly.
      finish_run<A, MT, 2 * kCW>(p, T, b, row0, tile * kTileCols + slice * kCW, sm.last,
                                 [&](int m, int c) { return native_pair_red_sum(sm, m, c); });
      u += 2 * (g_hi - g_lo);
    } else {
      finish_run<A, MT, kCW>(p, T, b, row0, tile * kTileCols + slice * kCW, sm.last,
                             [&](int m, int c) { return native_red_sum(sm, m, c); });
      u += g_hi - g_lo;
    }
  }
}

// Kernel parameters of a stream-K launch over native slabs, and its grid.
template <int G, int MT>
GemvParams native_params(const GemvLaunch& l, int* grid) {
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
  p.splits = 0;
  p.gps = 0;
  p.per = l.units_per_workgroup;
  p.max_contrib = l.max_contributors;
  p.norm_weight = static_cast<const uint16_t*>(l.norm_weight);
  p.eps = l.eps;
  p.pair = l.slice_pair ? 1 : 0;
  const long long total = static_cast<long long>(p.tiles) * kSlicesPerTile * p.mtiles * p.NG;
  *grid = p.per > 0 ? static_cast<int>((total + p.per - 1) / p.per) : 0;
  p.grid = *grid;
  p.xcd_remap = *grid % 8 == 0 ? *grid / 8 : 0;
  return p;
}

}  // namespace
}  // namespace fk
