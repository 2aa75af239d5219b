// libfk_w4a16 without HIP (FK_ENABLE_HIP=OFF in CMakeLists.txt): every entry point of
// include/fk_w4a16.h, each failing with FK_ERR_RUNTIME and a message saying so, so that the Python
// package (suites, reports, the fk CLI) imports and runs on machines without a GPU toolchain.
#include "fk_w4a16.h"

namespace {

const char kMessage[] = "libfk_w4a16 was built without HIP (FK_ENABLE_HIP=OFF): no GPU entry points";

}  // namespace

extern "C" {

const char* fk_last_error(void) { return kMessage; }

const char* fk_build_info(void) { return "fast-kernels-amd 0.1.0 cpu-only"; }

int fk_pack_arc_w4a16_packets(const void* q, const void* alpha, const void* beta, void* packets, int n, int k, int group_size, int packet_stride_bytes, void* stream) {
  (void)q;
  (void)alpha;
  (void)beta;
  (void)packets;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_stride_bytes;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_compute_arc_w4a16_group_sums(const void* activations, void* sums, int batch, int k, int group_size, void* stream) {
  (void)activations;
  (void)sums;
  (void)batch;
  (void)k;
  (void)group_size;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_arc_w4a16_forward(const void* activations, const void* packets, const void* group_sums, void* output, int batch, int n, int k, int group_size, int packet_stride_bytes, void* stream) {
  (void)activations;
  (void)packets;
  (void)group_sums;
  (void)output;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_stride_bytes;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_arc_w4a16_forward_split_k(const void* activations, const void* packets, const void* group_sums, void* partials, int batch, int n, int k, int group_size, int packet_stride_bytes, int split_k_slices, void* stream) {
  (void)activations;
  (void)packets;
  (void)group_sums;
  (void)partials;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_stride_bytes;
  (void)split_k_slices;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_reduce_arc_w4a16_split_k_partials(const void* partials, void* output, int batch, int n, int split_k_slices, void* stream) {
  (void)partials;
  (void)output;
  (void)batch;
  (void)n;
  (void)split_k_slices;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_dequant_w4a16_to_fp16(const void* q, const void* alpha, const void* beta, void* output, int n, int k, int group_size, void* stream) {
  (void)q;
  (void)alpha;
  (void)beta;
  (void)output;
  (void)n;
  (void)k;
  (void)group_size;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_dequant_arc_w4a16_packets_to_fp16(const void* packets, void* output, int n, int k, int group_size, int packet_stride_bytes, void* stream) {
  (void)packets;
  (void)output;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_stride_bytes;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_hipblaslt_fp16_with_weight(const void* activations, const void* weight, void* output, void* workspace, size_t workspace_bytes, int batch, int n, int k, void* stream) {
  (void)activations;
  (void)weight;
  (void)output;
  (void)workspace;
  (void)workspace_bytes;
  (void)batch;
  (void)n;
  (void)k;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_hipblaslt_fp16_after_packet_dequant(const void* activations, const void* packets, void* output, void* weight, void* workspace, size_t workspace_bytes, int batch, int n, int k, int group_size, int packet_stride_bytes, void* stream) {
  (void)activations;
  (void)packets;
  (void)output;
  (void)weight;
  (void)workspace;
  (void)workspace_bytes;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_stride_bytes;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_hipblaslt_fp16_after_dequant(const void* activations, const void* q, const void* alpha, const void* beta, void* output, void* weight, void* workspace, size_t workspace_bytes, int batch, int n, int k, int group_size, void* stream) {
  (void)activations;
  (void)q;
  (void)alpha;
  (void)beta;
  (void)output;
  (void)weight;
  (void)workspace;
  (void)workspace_bytes;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_arc_w4a16_plan_for(int batch, int n, int k, int group_size, int activation_dtype, int split_k_slices, int cu_count, fk_arc_w4a16_plan* plan) {
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)cu_count;
  (void)plan;
  return FK_ERR_RUNTIME;
}

int fk_arc_w4a16_forward_ex(const void* activations, const void* packets, void* output, void* workspace, size_t workspace_bytes, int batch, int n, int k, int group_size, int packet_stride_bytes, int activation_dtype, int split_k_slices, void* stream) {
  (void)activations;
  (void)packets;
  (void)output;
  (void)workspace;
  (void)workspace_bytes;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_stride_bytes;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_packet_stride_bytes(int group_size, int packet_format) {
  (void)group_size;
  (void)packet_format;
  return -1;
}

int fk_pack_native_w4a16_packets(const void* q, const void* alpha, const void* zero_points, void* packets, int n, int k, int group_size, int packet_format, void* stream) {
  (void)q;
  (void)alpha;
  (void)zero_points;
  (void)packets;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_convert_arc_to_native_packets(const void* arc_packets, void* native_packets, int n, int k, int group_size, int packet_format, void* stream) {
  (void)arc_packets;
  (void)native_packets;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_convert_native_to_arc_packets(const void* native_packets, void* arc_packets, int n, int k, int group_size, int packet_format, void* stream) {
  (void)native_packets;
  (void)arc_packets;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_w4a16_plan_for_format(int batch, int n, int k, int group_size, int activation_dtype, int split_k_slices, int cu_count, int packet_format, fk_arc_w4a16_plan* plan) {
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)cu_count;
  (void)packet_format;
  (void)plan;
  return FK_ERR_RUNTIME;
}

int fk_arc_w4a16_forward_native(const void* activations, const void* packets, void* output, void* workspace, size_t workspace_bytes, int batch, int n, int k, int group_size, int packet_format, int activation_dtype, int split_k_slices, void* stream) {
  (void)activations;
  (void)packets;
  (void)output;
  (void)workspace;
  (void)workspace_bytes;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_w4a16_forward_noalloc(const void* activations, const void* packets, void* output, int batch, int n, int k, int group_size, int packet_format, int activation_dtype, void* stream) {
  (void)activations;
  (void)packets;
  (void)output;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)activation_dtype;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_w4a16_plan_for_kernel(int batch, int n, int k, int group_size, int activation_dtype, int split_k_slices, int cu_count, int packet_format, int kernel, fk_arc_w4a16_plan* plan) {
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)cu_count;
  (void)packet_format;
  (void)kernel;
  (void)plan;
  return FK_ERR_RUNTIME;
}

int fk_w4a16_forward_kernel(const void* activations, const void* packets, void* output, void* workspace, size_t workspace_bytes, int batch, int n, int k, int group_size, int packet_format, int activation_dtype, int split_k_slices, int kernel, void* stream) {
  (void)activations;
  (void)packets;
  (void)output;
  (void)workspace;
  (void)workspace_bytes;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)kernel;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_w4a16_plan_rmsnorm(int batch, int n, int k, int group_size, int activation_dtype, int split_k_slices, int cu_count, int packet_format, fk_arc_w4a16_plan* plan) {
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)cu_count;
  (void)packet_format;
  (void)plan;
  return FK_ERR_RUNTIME;
}

int fk_w4a16_forward_rmsnorm(const void* activations, const void* norm_weight, float eps, const void* packets, void* output, void* workspace, size_t workspace_bytes, int batch, int n, int k, int group_size, int packet_format, int activation_dtype, int split_k_slices, void* stream) {
  (void)activations;
  (void)norm_weight;
  (void)eps;
  (void)packets;
  (void)output;
  (void)workspace;
  (void)workspace_bytes;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)activation_dtype;
  (void)split_k_slices;
  (void)stream;
  return FK_ERR_RUNTIME;
}

int fk_w4a16_forward_silu_mul(const void* activations, const void* packets, void* output, int batch, int n, int k, int group_size, int packet_format, int activation_dtype, const void* norm_weight, float eps, void* stream) {
  (void)activations;
  (void)packets;
  (void)output;
  (void)batch;
  (void)n;
  (void)k;
  (void)group_size;
  (void)packet_format;
  (void)activation_dtype;
  (void)norm_weight;
  (void)eps;
  (void)stream;
  return FK_ERR_RUNTIME;
}

}  // extern "C"
