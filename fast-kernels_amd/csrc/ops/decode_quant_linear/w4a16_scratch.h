// Fixed per-device scratch of the no-allocation entry point (w4a16_scratch.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace fast_kernels::decode_quant_linear {

// Bytes of the file-scope scratch array each GPU holds: the 64 KB counter region of the stream-K
// fix-up and 8 MB of fp32 partials. The automatic plans of up to 16 activation rows and N up to
// 131072 need at most 6.1 MB of scratch on 256 CUs (8 rows, N = 32768, G = 64, reference packets).
constexpr std::size_t kNoAllocScratchBytes = (8u << 20) + (64u << 10);

// Device address of the scratch array on the current device, looked up once per device. On that
// first lookup the first clear_bytes of it are zeroed by a kernel on `stream`.
void* noalloc_scratch(std::size_t clear_bytes, hipStream_t stream);

// Records `stream` as the one using the current device's scratch. Throws std::runtime_error when
// another stream recorded earlier still has work queued (or is being captured), since the two
// would race on the scratch. Not checked while `stream` itself is being captured.
void noalloc_claim_stream(hipStream_t stream);

}  // namespace fast_kernels::decode_quant_linear
