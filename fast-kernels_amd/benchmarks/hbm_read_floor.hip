// HBM read floor on one GPU: how fast a kernel that only streams bytes (no arithmetic) reads a
// buffer of a given size, timed the way bench.py times the GEMV (a HIP graph of launches over
// rotated copies, so that every launch reads HBM, not the 256 MiB Infinity Cache).
//
// Each workgroup (256 threads) streams one contiguous chunk with 16 dwordx4 loads in flight per
// lane; sizes are the Llama-7B/70B decode weight sizes, grids 128-2048 workgroups. The minimum
// over grids is the floor a weight-streaming GEMV of that size can approach.
//
// Build and run (from this directory):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       -o /tmp/hbm_read_floor hbm_read_floor.hip && /tmp/hbm_read_floor
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t err_ = (x);                                                        \
    if (err_ != hipSuccess) {                                                     \
      std::printf("error %s at line %d\n", hipGetErrorString(err_), __LINE__);    \
      std::exit(1);                                                               \
    }                                                                             \
  } while (0)

__global__ void __launch_bounds__(256) read_chunks(const uint4* __restrict__ p, size_t chunk16,
                                                   unsigned* out) {
  const uint4* base = p + static_cast<size_t>(blockIdx.x) * chunk16;
  const int t = static_cast<int>(threadIdx.x);
  unsigned acc = 0;
  for (size_t i = 0; i < chunk16; i += 256 * 16) {
    uint4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const size_t idx = i + u * 256 + t;
      v[u] = idx < chunk16 ? base[idx] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      acc ^= v[u].x + v[u].y + v[u].z + v[u].w;
    }
  }
  if (acc == 0x12345678u) {  // keeps the loads; never true for the constant fill below
    out[0] = acc;
  }
}

int main() {
  unsigned* out;
  CHECK(hipMalloc(&out, 4));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  hipStream_t stream;
  CHECK(hipStreamCreate(&stream));
  const size_t total = 2048ull << 20;
  char* buf;
  CHECK(hipMalloc(&buf, total));
  CHECK(hipMemset(buf, 1, total));
  std::printf("%10s %6s %5s %9s %9s\n", "MB", "wgs", "rot", "us", "GB/s");
  for (double mb : {8.7, 26.0, 34.6, 43.3, 121.2, 242.4}) {
    for (int wgs : {128, 256, 512, 1024, 2048}) {
      const size_t c16 = static_cast<size_t>(mb * 1e6 / 16) / wgs;
      const double bytes = static_cast<double>(c16) * 16 * wgs;
      const size_t slot = (static_cast<size_t>(bytes) + 65535) & ~static_cast<size_t>(65535);
      int rot = std::max(2, static_cast<int>(2 * 268435456.0 / bytes) + 1);
      rot = std::min<int>(rot, static_cast<int>(total / slot));
      hipGraph_t graph;
      hipGraphExec_t exec;
      CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
      for (int r = 0; r < rot; ++r) {
        hipLaunchKernelGGL(read_chunks, dim3(wgs), dim3(256), 0, stream,
                           reinterpret_cast<const uint4*>(buf + r * slot), c16, out);
      }
      CHECK(hipStreamEndCapture(stream, &graph));
      CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
      for (int i = 0; i < 3; ++i) {
        CHECK(hipGraphLaunch(exec, stream));
      }
      CHECK(hipStreamSynchronize(stream));
      const int reps = std::max(1, 300 / rot);
      CHECK(hipEventRecord(e0, stream));
      for (int i = 0; i < reps; ++i) {
        CHECK(hipGraphLaunch(exec, stream));
      }
      CHECK(hipEventRecord(e1, stream));
      CHECK(hipEventSynchronize(e1));
      float ms = 0.0f;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      const double us = ms * 1e3 / (reps * rot);
      std::printf("%10.1f %6d %5d %9.2f %9.1f\n", bytes / 1e6, wgs, rot, us, bytes / us / 1e3);
      CHECK(hipGraphExecDestroy(exec));
      CHECK(hipGraphDestroy(graph));
    }
  }
  return 0;
}
