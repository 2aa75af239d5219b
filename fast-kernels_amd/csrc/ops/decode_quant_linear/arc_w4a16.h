// C++ op API of the W4A16 decode linear ("ARC") family.
//
// The first eleven declarations keep the names, argument order and meaning of the reference op
// header (csrc/ops/decode_quant_linear/arc_w4a16.h:8-52): device buffers as std::uintptr_t,
// dimensions as int, the HIP stream last. Errors are thrown as std::invalid_argument (bad
// arguments, checked before any device call) or std::runtime_error (HIP / hipBLASLt failures),
// as in the reference (arc_w4a16.cu:23-85). The three vendor-baseline functions keep the
// reference's cublaslt_* names for drop-in callers and are served by hipBLASLt.
//
// The declarations after them are additions for MI355X callers: bf16 activations, an explicit
// caller-owned workspace and split-K choice, and a workspace-size query.
#pragma once

#include <cstddef>
#include <cstdint>

namespace fast_kernels::decode_quant_linear {

void pack_arc_w4a16_packets(std::uintptr_t q_ptr, std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
                            std::uintptr_t packets_ptr, int n, int k, int group_size,
                            int packet_stride_bytes, std::uintptr_t stream_ptr);

void compute_arc_w4a16_group_sums(std::uintptr_t activations_ptr, std::uintptr_t sums_ptr,
                                  int batch, int k, int group_size, std::uintptr_t stream_ptr);

void arc_w4a16_forward(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                       std::uintptr_t group_sums_ptr, std::uintptr_t output_ptr, int batch, int n,
                       int k, int group_size, int packet_stride_bytes, std::uintptr_t stream_ptr);

void arc_w4a16_forward_split_k(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                               std::uintptr_t group_sums_ptr, std::uintptr_t partials_ptr,
                               int batch, int n, int k, int group_size, int packet_stride_bytes,
                               int split_k_slices, std::uintptr_t stream_ptr);

void reduce_arc_w4a16_split_k_partials(std::uintptr_t partials_ptr, std::uintptr_t output_ptr,
                                       int batch, int n, int split_k_slices,
                                       std::uintptr_t stream_ptr);

void dequant_w4a16_to_fp16(std::uintptr_t q_ptr, std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
                           std::uintptr_t output_ptr, int n, int k, int group_size,
                           std::uintptr_t stream_ptr);

void dequant_arc_w4a16_packets_to_fp16(std::uintptr_t packets_ptr, std::uintptr_t output_ptr, int n,
                                       int k, int group_size, int packet_stride_bytes,
                                       std::uintptr_t stream_ptr);

void cublaslt_fp16_with_weight(std::uintptr_t activations_ptr, std::uintptr_t weight_ptr,
                               std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                               std::size_t workspace_bytes, int batch, int n, int k,
                               std::uintptr_t stream_ptr);

void cublaslt_fp16_after_packet_dequant(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                                        std::uintptr_t output_ptr, std::uintptr_t weight_ptr,
                                        std::uintptr_t workspace_ptr, std::size_t workspace_bytes,
                                        int batch, int n, int k, int group_size,
                                        int packet_stride_bytes, std::uintptr_t stream_ptr);

void cublaslt_fp16_after_dequant(std::uintptr_t activations_ptr, std::uintptr_t q_ptr,
                                 std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
                                 std::uintptr_t output_ptr, std::uintptr_t weight_ptr,
                                 std::uintptr_t workspace_ptr, std::size_t workspace_bytes,
                                 int batch, int n, int k, int group_size,
                                 std::uintptr_t stream_ptr);

// ---- additions (no reference counterpart) -------------------------------------------------

enum ActivationDtype : int { kActivationF16 = 0, kActivationBF16 = 1 };

// Packet formats: the reference's packets (codes, alpha, beta per 128-column tile and group,
// 64*G + 512 bytes) and the native gfx950 slabs, one per (tile, 32-column slice, group) in
// [tile][slice][group] order, holding the slice's code words and then 16 column-pair records:
// the two alphas (symmetric, zero point 8: 16*G + 64 bytes) or the two alphas and the two int4
// zero points padded to 8 bytes (asymmetric: 16*G + 128 bytes). A native buffer is
// [(N/32) * K/G, slab bytes].
enum PacketFormatCode : int { kPacketArc = 0, kPacketNativeSym = 1, kPacketNativeAsym = 2 };

struct ArcW4A16Plan {
  int m_tile;                   // activation rows per tile
  int workgroups;               // grid size
  int groups_per_workgroup;     // stream-K run length in (tile, group) units
  int max_tile_contributors;    // workgroups that can share one slice
  std::size_t workspace_bytes;  // caller workspace needed by arc_w4a16_forward_ex
  int slice_cols;               // columns per workgroup slice of a tile (128, 64, 32 or 16)
  int schedule;                 // kSchedule*: how the workgroups walk their units
  int stream_depth;             // kScheduleStream: slabs in flight per wave
  int stream_whole;             // kScheduleStream: whole slices per workgroup
  int stream_pieces;            // kScheduleStream: left-over slices dealt as pieces
  int stream_half;              // kScheduleStream: one half-slice (16 columns) per workgroup
};

// Launch schedules of a plan. kScheduleRuns: workgroups stream runs of one slice (or tile) at a
// time; kSchedulePairs: one-row native plans whose workgroups stream two adjacent whole 32-column
// slices at once (slice_cols 64); kScheduleStream: one-row native plans on a persistent grid,
// each workgroup streaming one contiguous range of slabs across slices with the whole activation
// row staged in LDS (w4a16_gemv_stream.hip).
enum Schedule : int { kScheduleRuns = 0, kSchedulePairs = 1, kScheduleStream = 2 };

// The launch the GEMV will use for this shape on the current device. split_k_slices = 0 picks
// the built-in policy; S > 0 gives every workgroup ceil(K / G / S) groups of whole 128-column
// tiles (each tile is then shared by about S workgroups).
ArcW4A16Plan plan_arc_w4a16(int batch, int n, int k, int group_size, int activation_dtype,
                            int split_k_slices);
// The same policy for a given CU count, with no device query (host-only, testable without a GPU).
ArcW4A16Plan plan_arc_w4a16_for_cu_count(int batch, int n, int k, int group_size,
                                         int activation_dtype, int split_k_slices, int cu_count);

// Packet GEMV with fp16 or bf16 activations (output in the same dtype), one launch, no group-sum
// prepass. workspace must be at least plan.workspace_bytes and zero-filled before its first use;
// every call leaves it zero-filled again. Calls that share a workspace must be stream-ordered.
void arc_w4a16_forward_ex(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                          std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                          std::size_t workspace_bytes, int batch, int n, int k, int group_size,
                          int packet_stride_bytes, int activation_dtype, int split_k_slices,
                          std::uintptr_t stream_ptr);

// Launch plan of arc_w4a16_forward_native for packets of the given format (kPacket*): the
// reference-format plan for kPacketArc and for the matrix-core batches, 32-column slices
// otherwise. cu_count = 0 queries the current device.
ArcW4A16Plan plan_w4a16_for_format(int batch, int n, int k, int group_size, int activation_dtype,
                                   int split_k_slices, int cu_count, int packet_format);

// Fused decode-step neighbours over native slabs (packet_format kPacketNativeSym or
// kPacketNativeAsym). y = W . rmsnorm(x), rmsnorm(x) = round(gamma * round(x * rsqrt(mean(x^2) +
// eps))) in the activation dtype, gamma = norm_weight [K]; plan, workspace contract and results
// otherwise as arc_w4a16_forward_native (the plan keeps 8+ rows on the dot2 kernel).
void arc_w4a16_forward_rmsnorm(std::uintptr_t activations_ptr, std::uintptr_t norm_weight_ptr,
                               float eps, std::uintptr_t packets_ptr, std::uintptr_t output_ptr,
                               std::uintptr_t workspace_ptr, std::size_t workspace_bytes, int batch,
                               int n, int k, int group_size, int packet_format,
                               int activation_dtype, int split_k_slices, std::uintptr_t stream_ptr);
ArcW4A16Plan plan_w4a16_rmsnorm(int batch, int n, int k, int group_size, int activation_dtype,
                                int split_k_slices, int cu_count, int packet_format);

// The gate_up projection with its SiLU: the slabs hold [W_gate; W_up] stacked along n (n % 256
// == 0); output [batch, n / 2] = round(round(silu(round(x.W_gate^T))) * round(x.W_up^T)) in the
// activation dtype. A non-null norm_weight_ptr adds the RMSNorm prologue of
// arc_w4a16_forward_rmsnorm to x. No workspace.
void arc_w4a16_forward_silu_mul(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                                std::uintptr_t output_ptr, int batch, int n, int k, int group_size,
                                int packet_format, int activation_dtype,
                                std::uintptr_t stream_ptr, std::uintptr_t norm_weight_ptr = 0,
                                float eps = 0.0f);

// Bytes per packet of a format.
int packet_format_stride_bytes(int group_size, int packet_format);

// Native packets from q_u8 [N, K/2], alpha [N, K/G] fp16 and (asymmetric only) zero_points uint8
// [N, K/G] with values 0..15 (zero_points_ptr is ignored for the symmetric format).
void pack_native_w4a16_packets(std::uintptr_t q_ptr, std::uintptr_t alpha_ptr,
                               std::uintptr_t zero_points_ptr, std::uintptr_t packets_ptr, int n,
                               int k, int group_size, int packet_format, std::uintptr_t stream_ptr);

// Reference packets -> native packets. Every beta must be half_rn(-alpha * zp) for an integer
// zp in 0..15 (zp = 8 for the symmetric format), otherwise std::invalid_argument. Synchronises
// the stream (the check reads a device flag back).
void convert_arc_w4a16_packets_to_native(std::uintptr_t arc_packets_ptr,
                                         std::uintptr_t native_packets_ptr, int n, int k,
                                         int group_size, int packet_format,
                                         std::uintptr_t stream_ptr);

// Native packets -> reference packets (beta = half_rn(-alpha * zp)); the inverse of the above,
// bit for bit.
void convert_native_w4a16_packets_to_arc(std::uintptr_t native_packets_ptr,
                                         std::uintptr_t arc_packets_ptr, int n, int k,
                                         int group_size, int packet_format,
                                         std::uintptr_t stream_ptr);

// arc_w4a16_forward_ex over packets of any format (kPacketArc, kPacketNativeSym,
// kPacketNativeAsym); same plan, workspace contract and results.
void arc_w4a16_forward_native(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                              std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                              std::size_t workspace_bytes, int batch, int n, int k, int group_size,
                              int packet_format, int activation_dtype, int split_k_slices,
                              std::uintptr_t stream_ptr);

// Kernel choice: the automatic dispatch (dot2 loop below 8 rows, matrix cores from 8), the dot2
// loop for every batch (m-tiles of at most 8 rows), or the matrix-core kernel for every batch
// (16-row m-tiles over whole 128-column tiles). The suites time each against the others.
enum KernelChoice : int { kKernelAuto = 0, kKernelDot2 = 1, kKernelMfma = 2 };

// plan_w4a16_for_format / arc_w4a16_forward_native with a kernel choice.
ArcW4A16Plan plan_w4a16_for_kernel(int batch, int n, int k, int group_size, int activation_dtype,
                                   int split_k_slices, int cu_count, int packet_format,
                                   int kernel);
void w4a16_forward_kernel(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                          std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                          std::size_t workspace_bytes, int batch, int n, int k, int group_size,
                          int packet_format, int activation_dtype, int split_k_slices, int kernel,
                          std::uintptr_t stream_ptr);

// arc_w4a16_forward_native (automatic plan) with no workspace argument and no allocation: the
// fix-up scratch is a fixed per-device array (w4a16_scratch.hip), so launches whose plan needs
// more than kNoAllocScratchBytes are rejected (std::invalid_argument), and calls that overlap on
// one device race on it.
void w4a16_forward_noalloc(std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                           std::uintptr_t output_ptr, int batch, int n, int k, int group_size,
                           int packet_format, int activation_dtype, std::uintptr_t stream_ptr);

}  // namespace fast_kernels::decode_quant_linear
