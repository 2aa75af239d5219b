// HBM read floor on one GPU: how fast a kernel that only streams bytes (no arithmetic) reads a
// buffer of a given size, timed the way bench.py times the GEMV (a HIP graph of launches over
// rotated copies, so that every launch reads HBM, not the 256 MiB Infinity Cache).
//
// The access pattern is swept, so the minimum is a floor for any weight-streaming kernel rather
// than for one way of reading:
//   threads per workgroup  256, 512, 1024
//   loads in flight        UNROLL dwordx4 loads per lane (4 KB .. 32 KB per wave)
//   mapping                "chunk": workgroup b reads one contiguous 1/grid of the buffer
//                          (grids 256 .. 8192); "stride": a grid of CUs x {1, 2, 4, 8}
//                          workgroups walks tiles of threads x UNROLL x 16 bytes, workgroup b
//                          taking tiles b, b + grid, ... (interleaved)
//   load kind              plain global_load_dwordx4, or non-temporal (__builtin_nontemporal_load)
// Sizes are the Llama-70B decode weight sizes; a 2 GB single-buffer read (one launch, no
// rotation) gives the asymptotic rate. Output: one line per variant, then the best per size.
//
// Build and run (from the repository root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       -o /tmp/hbm_read_floor fast-kernels_amd/benchmarks/hbm_read_floor.hip && /tmp/hbm_read_floor
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t err_ = (x);                                                        \
    if (err_ != hipSuccess) {                                                     \
      std::printf("error %s at line %d\n", hipGetErrorString(err_), __LINE__);    \
      std::exit(1);                                                               \
    }                                                                             \
  } while (0)

template <bool NT>
__device__ __forceinline__ uint4 load16(const uint4* p) {
  if constexpr (NT) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *p;
  }
}

// tiles: number of THREADS*UNROLL*16-byte tiles in the buffer. kStride = false: workgroup b reads
// tiles [b*per, (b+1)*per); true: tiles b, b + grid, b + 2*grid, ...
template <int THREADS, int UNROLL, bool NT, bool kStride>
__global__ void __launch_bounds__(THREADS) read_tiles(const uint4* __restrict__ p, int tiles,
                                                      int per, unsigned* out) {
  const int t = static_cast<int>(threadIdx.x);
  const int b = static_cast<int>(blockIdx.x);
  const int grid = static_cast<int>(gridDim.x);
  int begin, end, step;
  if constexpr (kStride) {
    begin = b;
    end = tiles;
    step = grid;
  } else {
    begin = b * per;
    end = min(tiles, begin + per);
    step = 1;
  }
  unsigned acc = 0;
  for (int tile = begin; tile < end; tile += step) {
    const uint4* base = p + static_cast<size_t>(tile) * (THREADS * UNROLL) + t;
    uint4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      v[u] = load16<NT>(base + u * THREADS);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      acc ^= v[u].x + v[u].y + v[u].z + v[u].w;
    }
  }
  if (acc == 0x12345678u) {  // keeps the loads; never true for the constant fill below
    out[0] = acc;
  }
}

struct Variant {
  int threads, unroll;
  bool nt, stride;
};

using KernelFn = void (*)(const uint4*, int, int, unsigned*);

template <int T, int U>
KernelFn pick(bool nt, bool stride) {
  if (nt) {
    return stride ? read_tiles<T, U, true, true> : read_tiles<T, U, true, false>;
  }
  return stride ? read_tiles<T, U, false, true> : read_tiles<T, U, false, false>;
}

KernelFn kernel_for(const Variant& v) {
  switch (v.threads * 100 + v.unroll) {
    case 25604: return pick<256, 4>(v.nt, v.stride);
    case 25608: return pick<256, 8>(v.nt, v.stride);
    case 25616: return pick<256, 16>(v.nt, v.stride);
    case 25632: return pick<256, 32>(v.nt, v.stride);
    case 51204: return pick<512, 4>(v.nt, v.stride);
    case 51208: return pick<512, 8>(v.nt, v.stride);
    case 51216: return pick<512, 16>(v.nt, v.stride);
    case 102404: return pick<1024, 4>(v.nt, v.stride);
    case 102408: return pick<1024, 8>(v.nt, v.stride);
    case 102416: return pick<1024, 16>(v.nt, v.stride);
    default: return nullptr;
  }
}

int main() {
  int dev = 0;
  CHECK(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, dev));
  const int cus = prop.multiProcessorCount;
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
  CHECK(hipDeviceSynchronize());

  std::vector<Variant> variants;
  for (int th : {256, 512, 1024}) {
    for (int un : {4, 8, 16, 32}) {
      if (th * un > 8192) continue;  // at most 128 KB per workgroup in flight
      for (bool nt : {false, true}) {
        for (bool st : {false, true}) variants.push_back({th, un, nt, st});
      }
    }
  }
  std::printf("CUs %d\n", cus);
  std::printf("%8s %5s %3s %3s %6s %6s %5s %9s %8s\n", "MB", "thr", "unr", "nt", "map", "grid",
              "rot", "us", "GB/s");
  struct Best {
    double us = 1e30, gbs = 0;
    std::string what;
  };
  const std::vector<double> sizes_mb = {34.6, 43.3, 121.2, 242.4, 2048.0};
  std::vector<Best> best(sizes_mb.size());
  for (size_t si = 0; si < sizes_mb.size(); ++si) {
    const double mb = sizes_mb[si];
    const bool single = mb > 1000.0;  // one launch over the whole buffer, no rotation
    for (const Variant& v : variants) {
      const KernelFn fn = kernel_for(v);
      const size_t tile_bytes = static_cast<size_t>(v.threads) * v.unroll * 16;
      const int tiles = static_cast<int>(static_cast<size_t>(mb * 1e6) / tile_bytes);
      const double bytes = static_cast<double>(tiles) * tile_bytes;
      const size_t slot = (static_cast<size_t>(bytes) + 65535) & ~static_cast<size_t>(65535);
      int rot = single ? 1 : std::max(2, static_cast<int>(2 * 268435456.0 / bytes) + 1);
      rot = std::min<int>(rot, static_cast<int>(total / slot));
      std::vector<int> grids;
      if (v.stride) {
        for (int k : {1, 2, 4, 8}) grids.push_back(cus * k);
      } else {
        for (int g : {256, 512, 1024, 2048, 4096, 8192}) grids.push_back(g);
      }
      for (int grid : grids) {
        const int per = (tiles + grid - 1) / grid;
        if (!v.stride && per < 1) continue;
        const int launch_grid = v.stride ? grid : (tiles + per - 1) / per;
        hipGraph_t graph;
        hipGraphExec_t exec;
        CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeGlobal));
        for (int r = 0; r < rot; ++r) {
          hipLaunchKernelGGL(fn, dim3(launch_grid), dim3(v.threads), 0, stream,
                             reinterpret_cast<const uint4*>(buf + r * slot), tiles, per, out);
        }
        CHECK(hipStreamEndCapture(stream, &graph));
        CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
        const int reps = single ? 20 : std::max(1, 300 / rot);
        for (int i = 0; i < std::max(2, reps / 4); ++i) CHECK(hipGraphLaunch(exec, stream));
        CHECK(hipStreamSynchronize(stream));
        CHECK(hipEventRecord(e0, stream));
        for (int i = 0; i < reps; ++i) CHECK(hipGraphLaunch(exec, stream));
        CHECK(hipEventRecord(e1, stream));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        const double us = ms * 1e3 / (reps * rot);
        const double gbs = bytes / us / 1e3;
        std::printf("%8.1f %5d %3d %3d %6s %6d %5d %9.2f %8.1f\n", bytes / 1e6, v.threads,
                    v.unroll, v.nt ? 1 : 0, v.stride ? "stride" : "chunk", launch_grid, rot, us,
                    gbs);
        std::fflush(stdout);
        if (us < best[si].us) {
          char what[128];
          std::snprintf(what, sizeof(what), "%d thr, unroll %d, %s, %s, grid %d", v.threads,
                        v.unroll, v.nt ? "nt" : "plain", v.stride ? "stride" : "chunk",
                        launch_grid);
          best[si] = {us, gbs, what};
        }
        CHECK(hipGraphExecDestroy(exec));
        CHECK(hipGraphDestroy(graph));
      }
    }
  }
  std::printf("\nbest per size\n");
  for (size_t si = 0; si < sizes_mb.size(); ++si) {
    std::printf("%8.1f MB  %8.2f us  %7.1f GB/s  %5.1f %%  %s\n", sizes_mb[si], best[si].us,
                best[si].gbs, best[si].gbs / 80.0, best[si].what.c_str());
  }
  return 0;
}
