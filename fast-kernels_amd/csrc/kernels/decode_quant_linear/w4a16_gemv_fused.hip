// W4A16 GEMV over native slabs with a decode-step neighbour fused in (GemvFuse in w4a16_gemv.h):
//
//  * kRmsNorm: the input RMSNorm of a Llama block's qkv / gate_up projection. Every run first
//    forms 1 / sqrt(mean(x^2) + eps) of its rows (fp32, read from L2), then stages
//    round(gamma * round(x * inv_rms)) instead of x: the activations the unfused pipeline would
//    have written between its norm kernel and the GEMV. Launch plan and fix-up as the plain
//    forward.
//  * kSiluMul: the gate_up projection with its activation. The weight is [W_gate; W_up] stacked
//    along N; workgroup b computes one 32-column slice of the gate half and the same slice of
//    the up half over all of K (each exactly as the plain forward computes it, run for run), and
//    writes round(round(silu(round(g))) * round(u)) to out[M, N/2]: the unfused pipeline's
//    GEMV, SiLU and product, each rounded to the activation dtype, in one launch and without the
//    [M, N] intermediate. kRmsNormSiluMul adds the RMSNorm prologue to it (a Llama block's
//    gate_up projection with its input norm and its activation in one launch).
#include "w4a16_gemv_native.h"

namespace fk {
namespace {

// kNorm: with the RMSNorm prologue (GemvFuse::kRmsNormSiluMul).
template <int G, Act A, int MT, PacketFormat F, bool kNorm>
__global__ void __launch_bounds__(kThreads, min_waves_per_eu<MT>())
w4a16_gemv_silu_mul_kernel(GemvParams p) {
  __shared__ NativeSmem<G, MT> sm;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t mask_lo = vgpr_constant(0x000f000fu);
  const uint32_t mask_hi = vgpr_constant(0x00f000f0u);
  const size_t stride = static_cast<size_t>(format_packet_stride(G, F));
  const int half_tiles = p.tiles / 2;
  const int pairs = half_tiles * kSlicesPerTile;
  const int b = static_cast<int>(blockIdx.x);
  const int pair = b % pairs;
  const int row0 = (b / pairs) * MT;
  const int tile = pair / kSlicesPerTile;
  const int slice = pair % kSlicesPerTile;
  auto slabs_of = [&](int t) {
    return p.packets + (static_cast<size_t>(t) * kSlicesPerTile + slice) * p.NG * stride;
  };

  float y[MT][2] = {};
  native_stream_groups<G, A, MT, F, kNorm>(sm, p, slabs_of(tile), row0, 0, p.NG, lane, wave,
                                           mask_lo, mask_hi, y, /*rms_first=*/true);
  native_reduce_run<G, MT>(sm, y, lane, wave);
  for (int idx = tid; idx < MT * kSliceCols; idx += kThreads) {
    sm.aux[idx / kSliceCols][idx % kSliceCols] =
        native_red_sum(sm, idx / kSliceCols, idx % kSliceCols);
  }
  __syncthreads();

  // When all of K fits one staging chunk, the up half reuses the activations the gate half
  // staged (normalised, for kNorm) instead of loading and converting them again.
  const bool one_chunk = p.NG <= NativeSmem<G, MT>::kChunk;
  float z[MT][2] = {};
  native_stream_groups<G, A, MT, F, kNorm>(sm, p, slabs_of(tile + half_tiles), row0, 0, p.NG,
                                           lane, wave, mask_lo, mask_hi, z, /*rms_first=*/false,
                                           /*staged=*/one_chunk);
  native_reduce_run<G, MT>(sm, z, lane, wave);
  const int out_cols = p.N / 2;
  for (int idx = tid; idx < MT * kSliceCols; idx += kThreads) {
    const int m = idx / kSliceCols;
    const int c = idx % kSliceCols;
    if (row0 + m < p.M) {
      const float g = act_bits_to_float<A>(float_to_act_bits<A>(sm.aux[m][c]));
      const float u = act_bits_to_float<A>(float_to_act_bits<A>(native_red_sum(sm, m, c)));
      const float s = act_bits_to_float<A>(float_to_act_bits<A>(g / (1.0f + expf(-g))));
      p.out[static_cast<size_t>(row0 + m) * out_cols + tile * kTileCols + slice * kSliceCols + c] =
          float_to_act_bits<A>(s * u);
    }
  }
}

template <int G, Act A, int MT, PacketFormat F>
hipError_t launch_fused_t(const GemvLaunch& l, hipStream_t stream) {
  int grid = 0;
  GemvParams p = native_params<G, MT>(l, &grid);
  if (l.fuse == GemvFuse::kRmsNorm) {
    hipLaunchKernelGGL((w4a16_gemv_native_kernel<G, A, MT, F, true>), dim3(grid), dim3(kThreads),
                       0, stream, p);
  } else {
    const int pairs = (l.N / kTileCols / 2) * kSlicesPerTile;
    if (l.fuse == GemvFuse::kRmsNormSiluMul) {
      hipLaunchKernelGGL((w4a16_gemv_silu_mul_kernel<G, A, MT, F, true>), dim3(pairs * p.mtiles),
                         dim3(kThreads), 0, stream, p);
    } else {
      hipLaunchKernelGGL((w4a16_gemv_silu_mul_kernel<G, A, MT, F, false>), dim3(pairs * p.mtiles),
                         dim3(kThreads), 0, stream, p);
    }
  }
  return hipGetLastError();
}

template <int G, Act A, PacketFormat F>
hipError_t fused_dispatch_mt(const GemvLaunch& l, hipStream_t stream) {
  switch (l.m_tile) {
    case 1: return launch_fused_t<G, A, 1, F>(l, stream);
    case 2: return launch_fused_t<G, A, 2, F>(l, stream);
    case 4: return launch_fused_t<G, A, 4, F>(l, stream);
    case 8: return launch_fused_t<G, A, 8, F>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

template <PacketFormat F>
hipError_t fused_dispatch(const GemvLaunch& l, hipStream_t stream) {
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? fused_dispatch_mt<64, Act::kF16, F>(l, stream)
                              : fused_dispatch_mt<64, Act::kBF16, F>(l, stream);
  }
  return l.act == Act::kF16 ? fused_dispatch_mt<128, Act::kF16, F>(l, stream)
                            : fused_dispatch_mt<128, Act::kBF16, F>(l, stream);
}

}  // namespace

hipError_t launch_w4a16_gemv_fused(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode != GemvMode::kStreamK || l.slice_cols != kSliceCols || l.fuse == GemvFuse::kNone ||
      l.slice_pair) {
    return hipErrorInvalidValue;
  }
  switch (l.format) {
    case PacketFormat::kNativeSym: return fused_dispatch<PacketFormat::kNativeSym>(l, stream);
    case PacketFormat::kNativeAsym: return fused_dispatch<PacketFormat::kNativeAsym>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fk
