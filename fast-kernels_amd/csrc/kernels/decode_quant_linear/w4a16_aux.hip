// W4A16 support kernels: packet builder, dequantisers, activation group sums, split-K reduction.
//
// Each follows the math of its reference counterpart in arc_w4a16.cu (cited per kernel) with a
// gfx950-shaped decomposition: 16-byte global accesses, one thread per 8 codes (one uint32 of
// nibbles), and no per-element 1-byte loads.
#include "w4a16_aux.h"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "w4a16_device.h"

namespace fk {
namespace {

constexpr int kAuxThreads = 256;

// pack_arc_packets_kernel (arc_w4a16.cu:87-122): packet (tile, g) holds word w of column c at
// byte (w*128 + c)*4, then alpha[128], then beta[128] (fp16). One thread per (tile, g, column):
// it reads its G/2 code bytes as 16-byte vectors and writes G/8 words; lanes of a wave write
// consecutive columns, so every store instruction covers 256 contiguous bytes.
template <int G>
__global__ void __launch_bounds__(kTileCols)
pack_packets_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ alpha,
                    const uint16_t* __restrict__ beta, uint8_t* __restrict__ packets, int k,
                    int num_groups) {
  constexpr int kGroupBytes = G / 2;
  constexpr int kVecs = kGroupBytes / 16;
  constexpr int QB = kTileCols * kGroupBytes;
  const int tile = static_cast<int>(blockIdx.x);
  const int g = static_cast<int>(blockIdx.y);
  const int c = static_cast<int>(threadIdx.x);
  const size_t row = static_cast<size_t>(tile) * kTileCols + c;
  const size_t stride = static_cast<size_t>(packet_stride_bytes(G));
  uint8_t* packet = packets + (static_cast<size_t>(tile) * num_groups + g) * stride;
  const uint4* src = reinterpret_cast<const uint4*>(q + row * (k / 2) + static_cast<size_t>(g) * kGroupBytes);
  uint32_t* words = reinterpret_cast<uint32_t*>(packet);
#pragma unroll
  for (int v = 0; v < kVecs; ++v) {
    const uint4 d = src[v];
    words[(4 * v + 0) * kTileCols + c] = d.x;
    words[(4 * v + 1) * kTileCols + c] = d.y;
    words[(4 * v + 2) * kTileCols + c] = d.z;
    words[(4 * v + 3) * kTileCols + c] = d.w;
  }
  uint16_t* a_dst = reinterpret_cast<uint16_t*>(packet + QB);
  uint16_t* b_dst = a_dst + kTileCols;
  a_dst[c] = alpha[row * num_groups + g];
  b_dst[c] = beta[row * num_groups + g];
}

// half_rn(fma(alpha, q, beta)) for the 8 codes of one uint32 word (k = 8w .. 8w+7). For the
// quantisation recipes used here alpha*q + beta is exact in fp32, so the single fp16 rounding
// makes the result bit-exact whatever the evaluation order (dequant_w4a16_kernel,
// arc_w4a16.cu:160-181, computes the same value).
__device__ __forceinline__ uint4 dequant_word(uint32_t word, float a, float b) {
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float q = static_cast<float>((word >> (4 * j)) & 0xfu);
    h[j] = float_to_half_bits(fmaf(a, q, b));
  }
  return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

// dequant_w4a16_kernel (arc_w4a16.cu:160-181): q_u8[N, K/2] + alpha/beta[N, NG] -> W[N, K] fp16.
template <int G>
__global__ void __launch_bounds__(kAuxThreads)
dequant_kernel(const uint32_t* __restrict__ q, const uint16_t* __restrict__ alpha,
               const uint16_t* __restrict__ beta, uint4* __restrict__ out, size_t total_words,
               int words_per_row, int num_groups) {
  const size_t idx = static_cast<size_t>(blockIdx.x) * kAuxThreads + threadIdx.x;
  if (idx >= total_words) {
    return;
  }
  const size_t row = idx / words_per_row;
  const int w = static_cast<int>(idx % words_per_row);
  const int g = (w * 8) / G;
  const float a = half_bits_to_float(alpha[row * num_groups + g]);
  const float b = half_bits_to_float(beta[row * num_groups + g]);
  out[idx] = dequant_word(q[idx], a, b);
}

// dequant_arc_packets_kernel (arc_w4a16.cu:183-220): packets -> W[N, K] fp16. One thread per
// (row, word); consecutive threads take consecutive words of a row so the 16-byte stores are
// contiguous.
template <int G>
__global__ void __launch_bounds__(kAuxThreads)
dequant_packets_kernel(const uint8_t* __restrict__ packets, uint4* __restrict__ out,
                       size_t total_words, int words_per_row, int num_groups) {
  constexpr int QB = kTileCols * G / 2;
  const size_t idx = static_cast<size_t>(blockIdx.x) * kAuxThreads + threadIdx.x;
  if (idx >= total_words) {
    return;
  }
  const size_t row = idx / words_per_row;
  const int w = static_cast<int>(idx % words_per_row);
  const int g = (w * 8) / G;
  const int wg = w % (G / 8);
  const size_t tile = row / kTileCols;
  const int c = static_cast<int>(row % kTileCols);
  const uint8_t* packet =
      packets + (tile * num_groups + g) * static_cast<size_t>(packet_stride_bytes(G));
  const uint32_t word = reinterpret_cast<const uint32_t*>(packet)[wg * kTileCols + c];
  const uint16_t* ab = reinterpret_cast<const uint16_t*>(packet + QB);
  out[idx] = dequant_word(word, half_bits_to_float(ab[c]), half_bits_to_float(ab[kTileCols + c]));
}

// compute_arc_group_sums_kernel (arc_w4a16.cu:124-158): sums[b, g] = sum of x[b, g*G .. +G) in
// fp32. One wave per (row, group): each lane adds two values, then a shuffle tree.
template <int G>
__global__ void __launch_bounds__(64)
group_sums_kernel(const uint32_t* __restrict__ x, float* __restrict__ sums, int k,
                  int num_groups) {
  const int b = static_cast<int>(blockIdx.x);
  const int g = static_cast<int>(blockIdx.y);
  const int lane = static_cast<int>(threadIdx.x);
  float v = 0.0f;
  if (lane < G / 2) {
    const uint32_t pair = x[(static_cast<size_t>(b) * k + static_cast<size_t>(g) * G) / 2 + lane];
    v = half_bits_to_float(static_cast<uint16_t>(pair)) + half_bits_to_float(static_cast<uint16_t>(pair >> 16));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v += __shfl_xor(v, off);
  }
  if (lane == 0) {
    sums[static_cast<size_t>(b) * num_groups + g] = v;
  }
}

// reduce_arc_w4a16_split_k_partials_kernel (arc_w4a16.cu:388-402): out[i] = half_rn(sum over
// slices of partials[s, i]), slices added in order 0..S-1.
__global__ void __launch_bounds__(kAuxThreads)
reduce_partials_kernel(const float* __restrict__ partials, uint16_t* __restrict__ out,
                       size_t total, int split_k_slices) {
  const size_t idx = static_cast<size_t>(blockIdx.x) * kAuxThreads + threadIdx.x;
  if (idx >= total) {
    return;
  }
  float v = 0.0f;
  for (int s = 0; s < split_k_slices; ++s) {
    v += partials[static_cast<size_t>(s) * total + idx];
  }
  out[idx] = float_to_half_bits(v);
}

unsigned int blocks_for(size_t n, int threads) {
  return static_cast<unsigned int>((n + threads - 1) / threads);
}


// Where column c (0..127) of tile `tile`, group g lives in the native slabs (PacketFormat in
// w4a16_device.h): its slab and its column 16*i + n inside the slab.
struct NativeSlot {
  uint8_t* slab;
  int i;
  int n;
};

template <int G, PacketFormat F>
__device__ __forceinline__ NativeSlot native_slot(uint8_t* packets, int tile, int g, int c,
                                                  int num_groups) {
  const size_t slab = (static_cast<size_t>(tile) * kSlicesPerTile + c / kSliceCols) * num_groups + g;
  const int cs = c % kSliceCols;
  return {packets + slab * static_cast<size_t>(format_packet_stride(G, F)), cs / 16, cs % 16};
}

// Code word w (codes k = 8w .. 8w+7 of the group) of the slot's column.
template <int G>
__device__ __forceinline__ uint32_t* slab_word(NativeSlot s, int w) {
  constexpr int U = native_unit_words(G);
  return reinterpret_cast<uint32_t*>(s.slab + native_word_offset(G, s.i, w / U, s.n, w % U));
}

template <int G, PacketFormat F>
__device__ __forceinline__ uint16_t* slab_alpha(NativeSlot s) {
  return reinterpret_cast<uint16_t*>(s.slab + native_record_offset(G) + native_record_bytes(F) * s.n) +
         s.i;
}

// kNativeAsym: the word after the column pair's alphas (-zp[n] and -zp[n + 16] as fp16).
template <int G>
__device__ __forceinline__ uint32_t* slab_zp_word(NativeSlot s) {
  return reinterpret_cast<uint32_t*>(s.slab + native_record_offset(G) +
                                     native_record_bytes(PacketFormat::kNativeAsym) * s.n + 4);
}

// Writes -zp of this thread's column (half s.i of the column pair's word).
template <int G>
__device__ __forceinline__ void store_neg_zp(NativeSlot s, uint32_t zp) {
  reinterpret_cast<uint16_t*>(slab_zp_word<G>(s))[s.i] = neg_zp_half_bits(zp & 0xFu);
}

// Native slabs from q_u8 / alpha / zero points (uint8 [N, NG], values 0..15, unused for
// kNativeSym). One thread per column of a (tile, group).
template <int G, PacketFormat F>
__global__ void __launch_bounds__(kTileCols)
pack_native_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ alpha,
                   const uint8_t* __restrict__ zero_points, uint8_t* __restrict__ packets, int k,
                   int num_groups) {
  constexpr int kGroupBytes = G / 2;
  constexpr int kVecs = kGroupBytes / 16;
  const int tile = static_cast<int>(blockIdx.x);
  const int g = static_cast<int>(blockIdx.y);
  const int c = static_cast<int>(threadIdx.x);
  const size_t row = static_cast<size_t>(tile) * kTileCols + c;
  const NativeSlot s = native_slot<G, F>(packets, tile, g, c, num_groups);
  const uint4* src = reinterpret_cast<const uint4*>(q + row * (k / 2) + static_cast<size_t>(g) * kGroupBytes);
#pragma unroll
  for (int v = 0; v < kVecs; ++v) {
    const uint4 d = src[v];
    *slab_word<G>(s, 4 * v + 0) = d.x;
    *slab_word<G>(s, 4 * v + 1) = d.y;
    *slab_word<G>(s, 4 * v + 2) = d.z;
    *slab_word<G>(s, 4 * v + 3) = d.w;
  }
  *slab_alpha<G, F>(s) = alpha[row * num_groups + g];
  if constexpr (F == PacketFormat::kNativeAsym) {
    store_neg_zp<G>(s, zero_points[row * num_groups + g]);
  }
}

// Reference packets -> native slabs. The zero point of a (column, group) is the integer zp in
// 0..15 with half_rn(-alpha * zp) == beta (bit for bit); kNativeSym requires zp = 8.
// (column, group)s with no such zp raise *bad, and the caller rejects the conversion.
template <int G, PacketFormat F>
__global__ void __launch_bounds__(kTileCols)
arc_to_native_kernel(const uint8_t* __restrict__ arc, uint8_t* __restrict__ native, int num_groups,
                     uint32_t* __restrict__ bad) {
  constexpr int QB = kTileCols * G / 2;
  const int tile = static_cast<int>(blockIdx.x);
  const int g = static_cast<int>(blockIdx.y);
  const int c = static_cast<int>(threadIdx.x);
  const size_t unit = static_cast<size_t>(tile) * num_groups + g;
  const uint8_t* src = arc + unit * static_cast<size_t>(packet_stride_bytes(G));
  const NativeSlot s = native_slot<G, F>(native, tile, g, c, num_groups);
  const uint32_t* sw = reinterpret_cast<const uint32_t*>(src);
#pragma unroll
  for (int w = 0; w < G / 8; ++w) {
    *slab_word<G>(s, w) = sw[w * kTileCols + c];
  }
  const uint16_t a_bits = reinterpret_cast<const uint16_t*>(src + QB)[c];
  const uint16_t b_bits = reinterpret_cast<const uint16_t*>(src + QB)[kTileCols + c];
  *slab_alpha<G, F>(s) = a_bits;
  int zp = -1;
  if constexpr (F == PacketFormat::kNativeSym) {
    zp = neg_alpha_zp_bits(a_bits, 8) == b_bits ? 8 : -1;
  } else {
    for (int z = 0; z < 16; ++z) {
      if (zp < 0 && neg_alpha_zp_bits(a_bits, static_cast<uint32_t>(z)) == b_bits) {
        zp = z;
      }
    }
  }
  if (zp < 0) {
    __hip_atomic_fetch_or(bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    zp = 0;
  }
  if constexpr (F == PacketFormat::kNativeAsym) {
    store_neg_zp<G>(s, static_cast<uint32_t>(zp));
  }
}

// Native slabs -> reference packets: the same codes and alpha, beta = half_rn(-alpha * zp).
template <int G, PacketFormat F>
__global__ void __launch_bounds__(kTileCols)
native_to_arc_kernel(const uint8_t* __restrict__ native, uint8_t* __restrict__ arc, int num_groups) {
  constexpr int QB = kTileCols * G / 2;
  const int tile = static_cast<int>(blockIdx.x);
  const int g = static_cast<int>(blockIdx.y);
  const int c = static_cast<int>(threadIdx.x);
  const size_t unit = static_cast<size_t>(tile) * num_groups + g;
  // The slab is only read here; native_slot takes a non-const pointer for the writers.
  const NativeSlot s = native_slot<G, F>(const_cast<uint8_t*>(native), tile, g, c, num_groups);
  uint8_t* dst = arc + unit * static_cast<size_t>(packet_stride_bytes(G));
  uint32_t* dw = reinterpret_cast<uint32_t*>(dst);
#pragma unroll
  for (int w = 0; w < G / 8; ++w) {
    dw[w * kTileCols + c] = *slab_word<G>(s, w);
  }
  const uint16_t a_bits = *slab_alpha<G, F>(s);
  uint32_t zp = 8;
  if constexpr (F == PacketFormat::kNativeAsym) {
    const uint16_t neg = reinterpret_cast<const uint16_t*>(slab_zp_word<G>(s))[s.i];
    zp = static_cast<uint32_t>(static_cast<float>(__builtin_bit_cast(_Float16, neg)) * -1.0f);
  }
  reinterpret_cast<uint16_t*>(dst + QB)[c] = a_bits;
  reinterpret_cast<uint16_t*>(dst + QB)[kTileCols + c] = neg_alpha_zp_bits(a_bits, zp);
}

}  // namespace

hipError_t launch_pack_packets(const void* q, const void* alpha, const void* beta, void* packets,
                               int n, int k, int group_size, hipStream_t stream) {
  const int num_groups = k / group_size;
  const dim3 grid(static_cast<unsigned int>(n / kTileCols), static_cast<unsigned int>(num_groups));
  auto* qp = static_cast<const uint8_t*>(q);
  auto* ap = static_cast<const uint16_t*>(alpha);
  auto* bp = static_cast<const uint16_t*>(beta);
  auto* pp = static_cast<uint8_t*>(packets);
  if (group_size == 64) {
    hipLaunchKernelGGL(pack_packets_kernel<64>, grid, dim3(kTileCols), 0, stream, qp, ap, bp, pp, k, num_groups);
  } else {
    hipLaunchKernelGGL(pack_packets_kernel<128>, grid, dim3(kTileCols), 0, stream, qp, ap, bp, pp, k, num_groups);
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const void* q, const void* alpha, const void* beta, void* out, int n,
                          int k, int group_size, hipStream_t stream) {
  const int words_per_row = k / 8;
  const size_t total = static_cast<size_t>(n) * words_per_row;
  const int num_groups = k / group_size;
  auto* qp = static_cast<const uint32_t*>(q);
  auto* ap = static_cast<const uint16_t*>(alpha);
  auto* bp = static_cast<const uint16_t*>(beta);
  auto* op = static_cast<uint4*>(out);
  if (group_size == 64) {
    hipLaunchKernelGGL(dequant_kernel<64>, dim3(blocks_for(total, kAuxThreads)), dim3(kAuxThreads), 0, stream,
                       qp, ap, bp, op, total, words_per_row, num_groups);
  } else {
    hipLaunchKernelGGL(dequant_kernel<128>, dim3(blocks_for(total, kAuxThreads)), dim3(kAuxThreads), 0, stream,
                       qp, ap, bp, op, total, words_per_row, num_groups);
  }
  return hipGetLastError();
}

hipError_t launch_dequant_packets(const void* packets, void* out, int n, int k, int group_size,
                                  hipStream_t stream) {
  const int words_per_row = k / 8;
  const size_t total = static_cast<size_t>(n) * words_per_row;
  const int num_groups = k / group_size;
  auto* pp = static_cast<const uint8_t*>(packets);
  auto* op = static_cast<uint4*>(out);
  if (group_size == 64) {
    hipLaunchKernelGGL(dequant_packets_kernel<64>, dim3(blocks_for(total, kAuxThreads)), dim3(kAuxThreads), 0,
                       stream, pp, op, total, words_per_row, num_groups);
  } else {
    hipLaunchKernelGGL(dequant_packets_kernel<128>, dim3(blocks_for(total, kAuxThreads)), dim3(kAuxThreads), 0,
                       stream, pp, op, total, words_per_row, num_groups);
  }
  return hipGetLastError();
}

hipError_t launch_group_sums(const void* x, void* sums, int batch, int k, int group_size,
                             hipStream_t stream) {
  const int num_groups = k / group_size;
  const dim3 grid(static_cast<unsigned int>(batch), static_cast<unsigned int>(num_groups));
  auto* xp = static_cast<const uint32_t*>(x);
  auto* sp = static_cast<float*>(sums);
  if (group_size == 64) {
    hipLaunchKernelGGL(group_sums_kernel<64>, grid, dim3(64), 0, stream, xp, sp, k, num_groups);
  } else {
    hipLaunchKernelGGL(group_sums_kernel<128>, grid, dim3(64), 0, stream, xp, sp, k, num_groups);
  }
  return hipGetLastError();
}

hipError_t launch_reduce_partials(const void* partials, void* out, int batch, int n,
                                  int split_k_slices, hipStream_t stream) {
  const size_t total = static_cast<size_t>(batch) * n;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(blocks_for(total, kAuxThreads)), dim3(kAuxThreads), 0, stream,
                     static_cast<const float*>(partials), static_cast<uint16_t*>(out), total, split_k_slices);
  return hipGetLastError();
}


hipError_t launch_pack_native(const void* q, const void* alpha, const void* zero_points,
                              void* packets, int n, int k, int group_size, PacketFormat format,
                              hipStream_t stream) {
  const int ng = k / group_size;
  const dim3 grid(static_cast<unsigned int>(n / kTileCols), static_cast<unsigned int>(ng));
  auto* qp = static_cast<const uint8_t*>(q);
  auto* ap = static_cast<const uint16_t*>(alpha);
  auto* zp = static_cast<const uint8_t*>(zero_points);
  auto* pp = static_cast<uint8_t*>(packets);
  const bool g64 = group_size == 64;
  if (format == PacketFormat::kNativeSym) {
    if (g64) hipLaunchKernelGGL((pack_native_kernel<64, PacketFormat::kNativeSym>), grid, dim3(kTileCols), 0, stream, qp, ap, zp, pp, k, ng);
    else hipLaunchKernelGGL((pack_native_kernel<128, PacketFormat::kNativeSym>), grid, dim3(kTileCols), 0, stream, qp, ap, zp, pp, k, ng);
  } else if (format == PacketFormat::kNativeAsym) {
    if (g64) hipLaunchKernelGGL((pack_native_kernel<64, PacketFormat::kNativeAsym>), grid, dim3(kTileCols), 0, stream, qp, ap, zp, pp, k, ng);
    else hipLaunchKernelGGL((pack_native_kernel<128, PacketFormat::kNativeAsym>), grid, dim3(kTileCols), 0, stream, qp, ap, zp, pp, k, ng);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_arc_to_native(const void* arc, void* native, int n, int k, int group_size,
                                PacketFormat format, void* bad_flag, hipStream_t stream) {
  const int ng = k / group_size;
  const dim3 grid(static_cast<unsigned int>(n / kTileCols), static_cast<unsigned int>(ng));
  auto* src = static_cast<const uint8_t*>(arc);
  auto* dst = static_cast<uint8_t*>(native);
  auto* bad = static_cast<uint32_t*>(bad_flag);
  const bool g64 = group_size == 64;
  if (format == PacketFormat::kNativeSym) {
    if (g64) hipLaunchKernelGGL((arc_to_native_kernel<64, PacketFormat::kNativeSym>), grid, dim3(kTileCols), 0, stream, src, dst, ng, bad);
    else hipLaunchKernelGGL((arc_to_native_kernel<128, PacketFormat::kNativeSym>), grid, dim3(kTileCols), 0, stream, src, dst, ng, bad);
  } else if (format == PacketFormat::kNativeAsym) {
    if (g64) hipLaunchKernelGGL((arc_to_native_kernel<64, PacketFormat::kNativeAsym>), grid, dim3(kTileCols), 0, stream, src, dst, ng, bad);
    else hipLaunchKernelGGL((arc_to_native_kernel<128, PacketFormat::kNativeAsym>), grid, dim3(kTileCols), 0, stream, src, dst, ng, bad);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_native_to_arc(const void* native, void* arc, int n, int k, int group_size,
                                PacketFormat format, hipStream_t stream) {
  const int ng = k / group_size;
  const dim3 grid(static_cast<unsigned int>(n / kTileCols), static_cast<unsigned int>(ng));
  auto* src = static_cast<const uint8_t*>(native);
  auto* dst = static_cast<uint8_t*>(arc);
  const bool g64 = group_size == 64;
  if (format == PacketFormat::kNativeSym) {
    if (g64) hipLaunchKernelGGL((native_to_arc_kernel<64, PacketFormat::kNativeSym>), grid, dim3(kTileCols), 0, stream, src, dst, ng);
    else hipLaunchKernelGGL((native_to_arc_kernel<128, PacketFormat::kNativeSym>), grid, dim3(kTileCols), 0, stream, src, dst, ng);
  } else if (format == PacketFormat::kNativeAsym) {
    if (g64) hipLaunchKernelGGL((native_to_arc_kernel<64, PacketFormat::kNativeAsym>), grid, dim3(kTileCols), 0, stream, src, dst, ng);
    else hipLaunchKernelGGL((native_to_arc_kernel<128, PacketFormat::kNativeAsym>), grid, dim3(kTileCols), 0, stream, src, dst, ng);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace fk
