// Device-side helpers shared by the W4A16 kernels (gfx950 / CDNA4 only).
//
// Packing convention (the reference's, arc_w4a16.cu:176-177 and decode_linear_w4a16.py:186-188):
// byte b of a row of q_u8 holds code k=2b in bits 0-3 and k=2b+1 in bits 4-7, so one
// little-endian uint32 word holds codes k=8w..8w+7 with code j in bits 4j..4j+3.
//
// Nibble -> 16-bit float without a conversion instruction: OR-ing a nibble into the low mantissa
// bits of a constant gives an exactly representable "bias + scale*q":
//   fp16 0x6400 | q        = 1024 + q        (nibble in bits 0-3: exponent 2^10, ulp 1)
//   fp16 0x5400 | (q << 4) = 64 + q          (nibble in bits 4-7: exponent 2^6, ulp 1/16)
//   bf16 0x4300 | q        = 128 + q         (bf16 keeps only 7 mantissa bits, so bits 0-3 only)
// One v_and_or_b32 turns a masked word into two such values (bits 0-15 and 16-31). A 32-bit word
// of codes therefore unpacks into the four half2 pairs (k0,k4) (k1,k5) (k2,k6) (k3,k7); the GEMV
// stores the activations in the same pair order so a v_dot2 multiplies matching k.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fk {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));

enum class Act : int { kF16 = 0, kBF16 = 1 };

constexpr int kTileCols = 128;  // output columns per packet tile (arc_w4a16.cu:16)

__host__ __device__ constexpr int packet_stride_bytes(int group_size) {
  return kTileCols * (group_size / 2) + 2 * kTileCols * 2;
}

// Packet formats.
//  kArc: the reference's packet (arc_w4a16.cu:87-122), one per (128-column tile, group): G/8 word
//    rows of 512 bytes (word w of column c at byte (w*128 + c)*4), alpha[128], beta[128] fp16.
//  kNativeSym / kNativeAsym: slabs, one per (tile, 32-column slice, group), laid out
//    [tile][slice][group] so that the groups of a slice are one contiguous byte range. A slab
//    holds the slice's code words in "quarter" order, then its alphas, then (kNativeAsym) its
//    zero points. Quarter order: slice column c = 16*i + n (i = 0, 1; n < 16) has W = G/8 words,
//    cut into four quarters of U = W/4 consecutive words; lane l = 16*t + n of a wave owns
//    quarter t of columns n and n + 16. G = 128 (U = 4): the words of column 16*i + n, quarter t
//    are the 16 bytes at i*1024 + l*16, so each 64-lane dwordx4 load reads 1 KB contiguous.
//    G = 64 (U = 2): both of the lane's units share the 16 bytes at l*16 (column n first). Then
//    16 records, one per column pair (n, n + 16): the two alphas, and for kNativeAsym the two
//    negated zero points as fp16 (-zp[n], -zp[n + 16]). The fp16 offsets are not stored: the
//    kernels rebuild beta = half_rn(-alpha * zp) exactly, one packed fp16 multiply for both
//    columns (zp = 8 for kNativeSym), the reference recipe's definition of beta. A lane thus applies each group's scale to two columns, and the same
//    layout feeds the matrix cores (w4a16_gemm_mfma.hip).
enum class PacketFormat : int { kArc = 0, kNativeSym = 1, kNativeAsym = 2 };

constexpr int kSliceCols = 32;  // native formats: columns per slab
constexpr int kSlicesPerTile = kTileCols / kSliceCols;

// Native slab offsets (see above). Unit = the U words of one (column, quarter).
__host__ __device__ constexpr int native_unit_words(int group_size) { return group_size / 32; }

// Byte offset, in a slab, of word j of the unit of column 16*i + n, quarter t.
__host__ __device__ constexpr int native_word_offset(int group_size, int i, int t, int n, int j) {
  return group_size == 128 ? i * 1024 + (16 * t + n) * 16 + 4 * j
                           : (16 * t + n) * 16 + i * 8 + 4 * j;
}

// The scales (and zero points) of a slab follow its code words as 16 records, record n for
// columns n and n + 16: kNativeSym 4 bytes (alpha[n], alpha[n + 16]); kNativeAsym 8 bytes (the
// two alphas, then -zp[n] and -zp[n + 16] as fp16), so a lane reads everything its two columns
// need with one load and forms both betas with one packed fp16 multiply.
__host__ __device__ constexpr int native_record_offset(int group_size) {
  return kSliceCols * group_size / 2;
}

__host__ __device__ constexpr int native_record_bytes(PacketFormat format) {
  return format == PacketFormat::kNativeAsym ? 8 : 4;
}

__host__ __device__ constexpr bool is_native(PacketFormat format) {
  return format != PacketFormat::kArc;
}

// Bytes per packet (kArc) or per slab (native formats).
__host__ __device__ constexpr int format_packet_stride(int group_size, PacketFormat format) {
  return format == PacketFormat::kArc
             ? packet_stride_bytes(group_size)
             : kSliceCols * (group_size / 2) + 16 * native_record_bytes(format);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t bits) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
}

// fp32 -> bf16, round to nearest even; NaN stays a NaN (gfx950's v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// fp32 -> fp16, round to nearest even (v_cvt_f16_f32 under the default round mode).
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// fp16 bits of -zp (zp in 0..15, exact; zp = 0 gives -0), as stored in asymmetric native slabs.
__device__ __forceinline__ uint16_t neg_zp_half_bits(uint32_t zp) {
  return static_cast<uint16_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(zp)) ^ 0x8000u);
}

// Bits of half_rn(-alpha * zp) for an fp16 alpha and an integer zp in 0..15, signed zeros
// included. alpha * zp is exact in 15 bits, so one fp16 multiply rounds it exactly as the
// reference's fp32 product then fp16 conversion does; the negation is a sign flip. (Written as
// "(half)(-(float)alpha * zp)" the compiler may fold the conversion into an fma with a +0
// addend, which turns the -0 of zp = 0 into +0.)
__device__ __forceinline__ uint16_t neg_alpha_zp_bits(uint16_t alpha_bits, uint32_t zp) {
  const _Float16 p = __builtin_bit_cast(_Float16, alpha_bits) * static_cast<_Float16>(zp);
  return static_cast<uint16_t>(__builtin_bit_cast(uint16_t, p) ^ 0x8000u);
}

template <Act A>
__device__ __forceinline__ float act_bits_to_float(uint16_t bits) {
  if constexpr (A == Act::kF16) {
    return half_bits_to_float(bits);
  } else {
    return bf16_bits_to_float(bits);
  }
}

template <Act A>
__device__ __forceinline__ uint16_t float_to_act_bits(float f) {
  if constexpr (A == Act::kF16) {
    return float_to_half_bits(f);
  } else {
    return float_to_bf16_bits(f);
  }
}

// acc + a.lo*b.lo + a.hi*b.hi with fp32 accumulation (v_dot2_f32_f16 / v_dot2_f32_bf16).
template <Act A>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (A == Act::kF16) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b),
                                  acc, false);
  } else {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a),
                                           __builtin_bit_cast(bf162_t, b), acc, false);
  }
}

// fp16 value of a group's offset for one column: read (kArc) or rebuilt from alpha and the zero
// point (native formats) with the same rounding the quantizer used.
template <PacketFormat F>
__device__ __forceinline__ float group_offset(float alpha, uint16_t beta_bits, uint32_t zero_point) {
  if constexpr (F == PacketFormat::kArc) {
    return half_bits_to_float(beta_bits);
  } else {
    const float zp = F == PacketFormat::kNativeSym ? 8.0f : static_cast<float>(zero_point);
    return half_bits_to_float(float_to_half_bits(-alpha * zp));  // -alpha*zp is exact in fp32
  }
}

// Re-pair 8 consecutive 16-bit activations x0..x7 (four words, two per word) into the order the
// nibble unpack produces: (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ uint4 pair_activations(uint4 x) {
  uint4 p;
  p.x = __builtin_amdgcn_perm(x.z, x.x, 0x05040100u);
  p.y = __builtin_amdgcn_perm(x.z, x.x, 0x07060302u);
  p.z = __builtin_amdgcn_perm(x.w, x.y, 0x05040100u);
  p.w = __builtin_amdgcn_perm(x.w, x.y, 0x07060302u);
  return p;
}


// Weight loads. Every weight byte is read once per call, so the GEMV kernels load them
// non-temporally (global_load ... nt): measured on MI355X with a pure streaming kernel
// (benchmarks/hbm_read_floor.hip), nt loads read 242 MB in 36.1 us against 39.3 us for plain
// loads of the same pattern, and 121 MB in 18.7 against 20.1 us. Activations, which every
// workgroup re-reads from L2, keep plain loads.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 stream_load16(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 stream_load8(const uint8_t* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return make_uint2(v.x, v.y);
}

__device__ __forceinline__ uint32_t stream_load4(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// s_waitcnt immediate for gfx9 waiting until at most n vector-memory operations are outstanding:
// vmcnt in bits 3:0 and 15:14, expcnt (6:4) and lgkmcnt (11:8) left at their maximum (no wait).
constexpr int wait_vmcnt(int n) {
  return (n & 0xF) | (((n >> 4) & 0x3) << 14) | 0x0F70;
}
constexpr int kWaitVmcnt0 = wait_vmcnt(0);
// Largest bf16 biased exponent whose values all fit in fp16 (2^15 * (2 - 2^-7) < 65504).
constexpr int kMaxFp16SafeBf16Exp = 142;

// Unpack biases of a masked code word: the low nibbles of each half (bits 0-3) become
// 1024 + q, the high nibbles (bits 4-7) 64 + q, both exact fp16 values.
constexpr uint32_t kBiasLow = 0x64006400u;
constexpr uint32_t kBiasHigh = 0x54005400u;

// Power-of-two staging shift for a (row, group) of bf16 activations whose largest biased
// exponent is e: the group is multiplied by 2^-shift so that its largest magnitude lands in
// [2^15, 2^16), the top binade of fp16. Large groups scale down (no fp16 overflow), small ones
// scale up, so every bf16 value within 2^-29 of the group maximum converts exactly (an fp16
// normal). Clamped so that 2^-shift and 2^shift stay normal fp32 values.
__device__ __forceinline__ int bf16_stage_shift(uint32_t e) {
  return max(-126, static_cast<int>(e) - kMaxFp16SafeBf16Exp);
}

typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

// Largest magnitude (bits without the sign, so its biased exponent is bits >> 7) of the eight
// bf16 values in four words: packed 16-bit maxima (v_pk_max_u16), one per pair of words. The
// magnitude bits of bf16 order as the values do (NaN above Inf above finite values).
__device__ __forceinline__ uint32_t bf16_max_mag(uint4 r) {
  const uint32_t k = 0x7fff7fffu;
  const u16x2_t a = __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, r.x & k),
                                              __builtin_bit_cast(u16x2_t, r.y & k));
  const u16x2_t b = __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, r.z & k),
                                              __builtin_bit_cast(u16x2_t, r.w & k));
  const u16x2_t m = __builtin_elementwise_max(a, b);
  return max(static_cast<uint32_t>(m.x), static_cast<uint32_t>(m.y));
}

// Two bf16 values, each multiplied by s (a power of two), as an fp16 pair: exact whenever the
// scaled value is an fp16 normal (bf16 has 8 significant bits, fp16 11), which the staging shift
// guarantees for every value within 2^-29 of its group's largest; smaller ones are truncated
// (the conversion rounds toward zero: one v_cvt_pkrtz_f16_f32 for both). Inf and NaN stay so.
__device__ __forceinline__ uint32_t bf16_pair_to_half_pair(uint32_t w, float s) {
  const float lo = __builtin_bit_cast(float, w << 16) * s;
  const float hi = __builtin_bit_cast(float, w & 0xffff0000u) * s;
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
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


// Cross-lane reductions over aligned groups of N in {8, 16} lanes (inside one 16-lane DPP row)
// with DPP moves, so each step is one VALU instruction instead of an LDS round trip: xor 1 and
// xor 2 (quad permutes), then the half-row mirror (lane i <-> 7 - i) and, for 16, the row mirror
// (i <-> 15 - i). Every lane of the group ends with the group's total.
namespace dpp {
constexpr int kQuadXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

template <int kCtrl>
__device__ __forceinline__ float move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl,
                                                                0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ uint32_t move(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
}  // namespace dpp

template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "group of 2, 4, 8 or 16 lanes");
  v += dpp::move<dpp::kQuadXor1>(v);
  if constexpr (N >= 4) {
    v += dpp::move<dpp::kQuadXor2>(v);
  }
  if constexpr (N >= 8) {
    v += dpp::move<dpp::kRowHalfMirror>(v);
  }
  if constexpr (N == 16) {
    v += dpp::move<dpp::kRowMirror>(v);
  }
  return v;
}

// Sums over the lanes of a 16-lane row that share lane index mod R (R in {1, 2, 4, 8}): rotating
// the row by R, 2R, ... keeps every lane inside its residue class.
template <int R>
__device__ __forceinline__ float row_strided_sum(float v) {
  static_assert(R == 1 || R == 2 || R == 4 || R == 8, "stride 1, 2, 4 or 8");
  if constexpr (R <= 1) {
    v += dpp::move<0x121>(v);  // row_ror:1
  }
  if constexpr (R <= 2) {
    v += dpp::move<0x122>(v);  // row_ror:2
  }
  if constexpr (R <= 4) {
    v += dpp::move<0x124>(v);  // row_ror:4
  }
  v += dpp::move<0x128>(v);    // row_ror:8
  return v;
}

template <int N>
__device__ __forceinline__ uint32_t group_max(uint32_t v) {
  static_assert(N == 2 || N == 4 || N == 8 || N == 16, "group of 2, 4, 8 or 16 lanes");
  v = max(v, dpp::move<dpp::kQuadXor1>(v));
  if constexpr (N >= 4) {
    v = max(v, dpp::move<dpp::kQuadXor2>(v));
  }
  if constexpr (N >= 8) {
    v = max(v, dpp::move<dpp::kRowHalfMirror>(v));
  }
  if constexpr (N == 16) {
    v = max(v, dpp::move<dpp::kRowMirror>(v));
  }
  return v;
}

// Last-contributor sum of a split tile's fp32 partials: acc[i] = sum over s = 0 .. n-1, in that
// order, of ws[s * count + e] for this thread's elements e = tid + i * threads (e < count). The
// loads are relaxed agent-scope atomics (coherent across XCDs); the loads of 4 contributors for all
// of the thread's elements are issued before the first add, so the hand-off costs one memory
// round trip per 4 contributors rather than one per element and contributor.
template <int kPer, int kThreadCount>
__device__ __forceinline__ void sum_tile_partials(const float* ws, int count, int n, int tid,
                                                  float (&acc)[kPer]) {
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    acc[i] = 0.0f;
  }
  for (int s0 = 0; s0 < n; s0 += 4) {
    float v[kPer][4];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = tid + i * kThreadCount;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[i][j] = 0.0f;
        if (s0 + j < n && e < count) {
          v[i][j] = __hip_atomic_load(ws + static_cast<size_t>(s0 + j) * count + e, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (s0 + j < n) {
          acc[i] += v[i][j];
        }
      }
    }
  }
}

}  // namespace fk
