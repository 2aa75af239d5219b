// Fixed scratch memory for the entry point that allocates nothing (fk_w4a16_forward_noalloc).
//
// The stream-K fix-up of a split slice needs device scratch (arrival counters, then fp32
// partials). The other entry points take it from the caller or allocate it; this one uses a
// file-scope device array of kNoAllocScratchBytes instead, which every GPU the library runs on
// holds until the process ends. In host code `scratch` names a host-side stand-in, not device
// memory: its device address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that address is ever handed to kernels.
//
// Every call on one GPU shares that GPU's array. The GEMV returns the counter region to zero at
// the end of every call, and the region is cleared once, by a fill kernel on the first calling
// stream, when the device's address is first looked up; calls that overlap on one GPU (other
// streams, concurrent graphs) race on it. As a guard against the common misuse, the last stream
// that called on a device is recorded, and a call from another stream while that one still has
// work queued is refused (noalloc_claim_stream).
#include "ops/decode_quant_linear/w4a16_scratch.h"

#include "fk_w4a16.h"

#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>
#include <mutex>
#include <sstream>
#include <stdexcept>

namespace fast_kernels::decode_quant_linear {
namespace {

static_assert(kNoAllocScratchBytes == FK_NOALLOC_SCRATCH_BYTES, "the C header states the size");

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;

__global__ void clear_words(uint32_t* words, int count) {
  const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < count) {
    words[i] = 0u;
  }
}

void check(hipError_t status, const char* what) {
  if (status != hipSuccess) {
    std::ostringstream oss;
    oss << what << " failed: " << hipGetErrorString(status);
    throw std::runtime_error(oss.str());
  }
}

}  // namespace

void* noalloc_scratch(std::size_t clear_bytes, hipStream_t stream) {
  static std::array<void*, kMaxScratchDevices> addresses{};
  static std::mutex mutex;
  int device = 0;
  check(hipGetDevice(&device), "hipGetDevice");
  if (device < 0 || device >= kMaxScratchDevices) {
    throw std::runtime_error("device index out of range");
  }
  std::lock_guard<std::mutex> lock(mutex);
  if (addresses[device] == nullptr) {
    void* ptr = nullptr;
    check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    // Clear the region the kernels expect to find zero (a fill kernel, not a memset node, so
    // that a first call under graph capture records an ordinary kernel).
    const int words = static_cast<int>(clear_bytes / sizeof(uint32_t));
    if (words > 0) {
      hipLaunchKernelGGL(clear_words, dim3((words + 255) / 256), dim3(256), 0, stream,
                         static_cast<uint32_t*>(ptr), words);
      check(hipGetLastError(), "clear_words launch");
    }
    addresses[device] = ptr;
  }
  return addresses[device];
}

void noalloc_claim_stream(hipStream_t stream) {
  static std::array<hipStream_t, kMaxScratchDevices> owners{};
  static std::array<bool, kMaxScratchDevices> owned{};
  static std::mutex mutex;
  int device = 0;
  check(hipGetDevice(&device), "hipGetDevice");
  if (device < 0 || device >= kMaxScratchDevices) {
    throw std::runtime_error("device index out of range");
  }
  std::lock_guard<std::mutex> lock(mutex);
  if (!owned[device] || owners[device] == stream) {
    owners[device] = stream;
    owned[device] = true;
    return;
  }
  // A call being captured records kernels that run only when the graph is replayed, so there is
  // nothing to compare against now (and stream queries are not allowed during a capture).
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &status) == hipSuccess &&
      status != hipStreamCaptureStatusNone) {
    return;
  }
  bool busy = false;
  if (hipStreamIsCapturing(owners[device], &status) == hipSuccess &&
      status != hipStreamCaptureStatusNone) {
    busy = true;
  } else {
    busy = hipStreamQuery(owners[device]) == hipErrorNotReady;
  }
  // a query that is not hipSuccess leaves its code as the thread's last error; the launch checks
  // that follow must not see it
  (void)hipGetLastError();
  if (busy) {
    std::ostringstream oss;
    oss << "fk_w4a16_forward_noalloc: stream " << static_cast<const void*>(stream)
        << " would share device " << device << "'s scratch with stream "
        << static_cast<const void*>(owners[device])
        << ", which still has work queued; synchronise it first (calls that overlap on one GPU "
           "race on the scratch)";
    throw std::runtime_error(oss.str());
  }
  owners[device] = stream;
}

}  // namespace fast_kernels::decode_quant_linear
