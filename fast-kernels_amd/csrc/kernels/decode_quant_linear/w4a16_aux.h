// Host launchers for the W4A16 support kernels (w4a16_aux.hip). No validation here: the op layer
// (ops/decode_quant_linear) checks every argument before calling these.
#pragma once

#include <hip/hip_runtime.h>

namespace fk {

hipError_t launch_pack_packets(const void* q, const void* alpha, const void* beta, void* packets,
                               int n, int k, int group_size, hipStream_t stream);
hipError_t launch_dequant(const void* q, const void* alpha, const void* beta, void* out, int n,
                          int k, int group_size, hipStream_t stream);
hipError_t launch_dequant_packets(const void* packets, void* out, int n, int k, int group_size,
                                  hipStream_t stream);
hipError_t launch_group_sums(const void* x, void* sums, int batch, int k, int group_size,
                             hipStream_t stream);
hipError_t launch_reduce_partials(const void* partials, void* out, int batch, int n,
                                  int split_k_slices, hipStream_t stream);

}  // namespace fk
