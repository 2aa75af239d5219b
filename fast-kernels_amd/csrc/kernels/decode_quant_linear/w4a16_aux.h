// Host launchers for the W4A16 support kernels (w4a16_aux.hip). No validation here: the op layer
// (ops/decode_quant_linear) checks every argument before calling these.
#pragma once

#include <hip/hip_runtime.h>

#include "w4a16_device.h"

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

// Native packet formats (PacketFormat): build from q_u8 / alpha / zero points (uint8 [N, NG],
// ignored for kNativeSym), and convert to and from reference packets. arc -> native sets
// *bad_flag (device uint32, zeroed by the caller) when some beta is not half_rn(-alpha * zp)
// for an integer zp in 0..15 (zp = 8 for kNativeSym).
hipError_t launch_pack_native(const void* q, const void* alpha, const void* zero_points,
                              void* packets, int n, int k, int group_size, PacketFormat format,
                              hipStream_t stream);
hipError_t launch_arc_to_native(const void* arc, void* native, int n, int k, int group_size,
                                PacketFormat format, void* bad_flag, hipStream_t stream);
hipError_t launch_native_to_arc(const void* native, void* arc, int n, int k, int group_size,
                                PacketFormat format, hipStream_t stream);

}  // namespace fk
