// Dot2 GEMV kernels over the native packet formats (no stored fp16 offsets; see PacketFormat in
// w4a16_device.h), instantiated apart from the reference-format ones so both compile in parallel.
#include "w4a16_gemv_kernels.h"

namespace fk {

hipError_t launch_w4a16_gemv_native(const GemvLaunch& l, hipStream_t stream) {
  switch (l.format) {
    case PacketFormat::kNativeSym: return launch_format<PacketFormat::kNativeSym>(l, stream);
    case PacketFormat::kNativeAsym: return launch_format<PacketFormat::kNativeAsym>(l, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fk
