// W4A16 GEMV over the native slab formats: the plain forward (kernel, launch and dispatch). The
// layout, lane mapping and device building blocks are described in w4a16_gemv_native.h.
#include "w4a16_gemv_native.h"

namespace fk {
namespace {

template <int G, Act A, int MT, PacketFormat F>
hipError_t launch_native_t(const GemvLaunch& l, hipStream_t stream) {
  int grid = 0;
  const GemvParams p = native_params<G, MT>(l, &grid);
  hipLaunchKernelGGL((w4a16_gemv_native_kernel<G, A, MT, F, false>), dim3(grid), dim3(kThreads), 0,
                     stream, p);
  return hipGetLastError();
}

template <int G, Act A, PacketFormat F>
hipError_t native_dispatch_mt(const GemvLaunch& l, hipStream_t stream) {
  switch (l.m_tile) {
    case 1: return launch_native_t<G, A, 1, F>(l, stream);
    case 2: return launch_native_t<G, A, 2, F>(l, stream);
    case 4: return launch_native_t<G, A, 4, F>(l, stream);
    case 8: return launch_native_t<G, A, 8, F>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

template <PacketFormat F>
hipError_t native_dispatch(const GemvLaunch& l, hipStream_t stream) {
  if (l.group_size == 64) {
    return l.act == Act::kF16 ? native_dispatch_mt<64, Act::kF16, F>(l, stream)
                              : native_dispatch_mt<64, Act::kBF16, F>(l, stream);
  }
  return l.act == Act::kF16 ? native_dispatch_mt<128, Act::kF16, F>(l, stream)
                            : native_dispatch_mt<128, Act::kBF16, F>(l, stream);
}

}  // namespace

hipError_t launch_w4a16_gemv_native(const GemvLaunch& l, hipStream_t stream) {
  if (l.mode != GemvMode::kStreamK || l.slice_cols != kSliceCols) {
    return hipErrorInvalidValue;
  }
  if (l.slice_pair) {
    // Whole slice pairs per run: no fused neighbour, runs of a multiple of two slices' groups.
    const int ng = l.group_size > 0 ? l.K / l.group_size : 0;
    if (l.fuse != GemvFuse::kNone || ng <= 0 || l.units_per_workgroup <= 0 ||
        l.units_per_workgroup % (2 * ng) != 0) {
      return hipErrorInvalidValue;
    }
  }
  switch (l.format) {
    case PacketFormat::kNativeSym: return native_dispatch<PacketFormat::kNativeSym>(l, stream);
    case PacketFormat::kNativeAsym: return native_dispatch<PacketFormat::kNativeAsym>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fk
