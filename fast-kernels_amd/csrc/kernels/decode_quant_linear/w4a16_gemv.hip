// W4A16 GEMV launch entry points. The kernels are in w4a16_gemv_kernels.h; this file instantiates
// the reference packet format (kArc, stream-K and the reference split-K protocol) and routes every
// launch: 16-row m-tiles to the matrix-core kernels (w4a16_gemm_mfma.hip, or on the stream schedule
// w4a16_gemm_mfma_stream.hip), native packet formats to w4a16_gemv_native.hip or, on the stream
// schedule, w4a16_gemv_stream.hip; the fused decode-step neighbours to w4a16_gemv_fused.hip or, on
// the stream schedule (one row), w4a16_gemv_stream.hip; one row over reference packets on the
// stream schedule to w4a16_gemv_arc_stream.hip.
#include "w4a16_gemv_kernels.h"

namespace fk {

int gemv_m_tile_for_batch(int batch) {
  if (batch >= kMfmaMinBatch) return kMfmaRows;
  return gemv_partials_m_tile_for_batch(batch);
}

int gemv_partials_m_tile_for_batch(int batch) {
  if (batch <= 1) return 1;
  if (batch <= 2) return 2;
  if (batch <= 4) return 4;
  return 8;
}

hipError_t launch_w4a16_gemv(const GemvLaunch& l, hipStream_t stream) {
  if (l.stream && l.m_tile == kMfmaRows) {
    return launch_w4a16_gemm_mfma_stream(l, stream);
  }
  if (l.stream && l.format == PacketFormat::kArc) {
    return l.slice_cols == kSliceCols || l.slice_cols == kSliceCols / 2
               ? launch_w4a16_gemv_arc_quarter(l, stream)
               : launch_w4a16_gemv_arc_stream(l, stream);
  }
  if (l.fuse != GemvFuse::kNone) {
    return l.stream ? launch_w4a16_gemv_stream(l, stream) : launch_w4a16_gemv_fused(l, stream);
  }
  if (l.m_tile == kMfmaRows) {
    return l.stream ? launch_w4a16_gemm_mfma_stream(l, stream) : launch_w4a16_gemm_mfma(l, stream);
  }
  if (l.stream) {
    return launch_w4a16_gemv_stream(l, stream);
  }
  if (l.format != PacketFormat::kArc) {
    return launch_w4a16_gemv_native(l, stream);
  }
  return launch_format<PacketFormat::kArc>(l, stream);
}

}  // namespace fk
