// Device-side helpers shared by the W4A16 kernels (gfx950 / CDNA4 only).
//
// Packing convention (the reference's, arc_w4a16.cu:176-177 and decode_linear_w4a16.py:186-188):
// byte b of a row of q_u8 holds code k=2b in bits 0-3 and k=2b+1 in bits 4-7, so one
// little-endian uint32 word holds codes k=8w..8w+7 with code j in bits 4j..4j+3.
//
// Nibble -> 16-bit float without a conversion instruction: OR-ing a nibble into the low mantissa
// bits of a constant gives an exactly representable "bias + scale*q":
//   fp16 0x6400 | q        = 1024 + q        (nibble in bits 0-3)
//   fp16 0x6400 | (q << 4) = 1024 + 16*q     (nibble in bits 4-7)
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

__device__ __forceinline__ float half_bits_to_float(uint16_t bits) {
  return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t bits) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
}

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    return static_cast<uint16_t>((u >> 16) | 0x0040u);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// fp32 -> fp16, round to nearest even (v_cvt_f16_f32 under the default round mode).
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
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

}  // namespace fk
