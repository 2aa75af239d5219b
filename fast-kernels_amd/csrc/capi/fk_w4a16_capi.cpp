// extern "C" boundary of libfk_w4a16.so (declared in include/fk_w4a16.h).
//
// Each entry point forwards to the C++ op of the same name and turns its exceptions into status
// codes: std::invalid_argument -> FK_ERR_INVALID_ARGUMENT, anything else -> FK_ERR_RUNTIME. The
// message is kept per thread for fk_last_error().
#include "fk_w4a16.h"

#include <cstdint>
#include <exception>
#include <stdexcept>
#include <string>

#include "ops/decode_quant_linear/arc_w4a16.h"

namespace ops = fast_kernels::decode_quant_linear;

namespace {

thread_local std::string g_last_error;

template <typename Fn>
int guarded(Fn&& fn) {
  g_last_error.clear();
  try {
    fn();
    return FK_OK;
  } catch (const std::invalid_argument& e) {
    g_last_error = e.what();
    return FK_ERR_INVALID_ARGUMENT;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return FK_ERR_RUNTIME;
  } catch (...) {
    g_last_error = "unknown error";
    return FK_ERR_RUNTIME;
  }
}

inline std::uintptr_t P(const void* p) { return reinterpret_cast<std::uintptr_t>(p); }

}  // namespace

extern "C" {

const char* fk_last_error(void) { return g_last_error.c_str(); }

const char* fk_build_info(void) { return "fast-kernels-amd 0.1.0 gfx950 hip"; }

int fk_pack_arc_w4a16_packets(const void* q, const void* alpha, const void* beta, void* packets,
                              int n, int k, int group_size, int packet_stride_bytes, void* stream) {
  return guarded([&] {
    ops::pack_arc_w4a16_packets(P(q), P(alpha), P(beta), P(packets), n, k, group_size,
                                packet_stride_bytes, P(stream));
  });
}

int fk_compute_arc_w4a16_group_sums(const void* activations, void* sums, int batch, int k,
                                    int group_size, void* stream) {
  return guarded([&] {
    ops::compute_arc_w4a16_group_sums(P(activations), P(sums), batch, k, group_size, P(stream));
  });
}

int fk_arc_w4a16_forward(const void* activations, const void* packets, const void* group_sums,
                         void* output, int batch, int n, int k, int group_size,
                         int packet_stride_bytes, void* stream) {
  return guarded([&] {
    ops::arc_w4a16_forward(P(activations), P(packets), P(group_sums), P(output), batch, n, k,
                           group_size, packet_stride_bytes, P(stream));
  });
}

int fk_arc_w4a16_forward_split_k(const void* activations, const void* packets,
                                 const void* group_sums, void* partials, int batch, int n, int k,
                                 int group_size, int packet_stride_bytes, int split_k_slices,
                                 void* stream) {
  return guarded([&] {
    ops::arc_w4a16_forward_split_k(P(activations), P(packets), P(group_sums), P(partials), batch,
                                   n, k, group_size, packet_stride_bytes, split_k_slices,
                                   P(stream));
  });
}

int fk_reduce_arc_w4a16_split_k_partials(const void* partials, void* output, int batch, int n,
                                         int split_k_slices, void* stream) {
  return guarded([&] {
    ops::reduce_arc_w4a16_split_k_partials(P(partials), P(output), batch, n, split_k_slices,
                                           P(stream));
  });
}

int fk_dequant_w4a16_to_fp16(const void* q, const void* alpha, const void* beta, void* output,
                             int n, int k, int group_size, void* stream) {
  return guarded([&] {
    ops::dequant_w4a16_to_fp16(P(q), P(alpha), P(beta), P(output), n, k, group_size, P(stream));
  });
}

int fk_dequant_arc_w4a16_packets_to_fp16(const void* packets, void* output, int n, int k,
                                         int group_size, int packet_stride_bytes, void* stream) {
  return guarded([&] {
    ops::dequant_arc_w4a16_packets_to_fp16(P(packets), P(output), n, k, group_size,
                                           packet_stride_bytes, P(stream));
  });
}

int fk_hipblaslt_fp16_with_weight(const void* activations, const void* weight, void* output,
                                  void* workspace, size_t workspace_bytes, int batch, int n, int k,
                                  void* stream) {
  return guarded([&] {
    ops::cublaslt_fp16_with_weight(P(activations), P(weight), P(output), P(workspace),
                                   workspace_bytes, batch, n, k, P(stream));
  });
}

int fk_hipblaslt_fp16_after_packet_dequant(const void* activations, const void* packets,
                                           void* output, void* weight, void* workspace,
                                           size_t workspace_bytes, int batch, int n, int k,
                                           int group_size, int packet_stride_bytes, void* stream) {
  return guarded([&] {
    ops::cublaslt_fp16_after_packet_dequant(P(activations), P(packets), P(output), P(weight),
                                            P(workspace), workspace_bytes, batch, n, k,
                                            group_size, packet_stride_bytes, P(stream));
  });
}

int fk_hipblaslt_fp16_after_dequant(const void* activations, const void* q, const void* alpha,
                                    const void* beta, void* output, void* weight, void* workspace,
                                    size_t workspace_bytes, int batch, int n, int k,
                                    int group_size, void* stream) {
  return guarded([&] {
    ops::cublaslt_fp16_after_dequant(P(activations), P(q), P(alpha), P(beta), P(output), P(weight),
                                     P(workspace), workspace_bytes, batch, n, k, group_size,
                                     P(stream));
  });
}

namespace {

void copy_plan(const ops::ArcW4A16Plan& p, fk_arc_w4a16_plan* plan) {
  plan->m_tile = p.m_tile;
  plan->workgroups = p.workgroups;
  plan->groups_per_workgroup = p.groups_per_workgroup;
  plan->max_tile_contributors = p.max_tile_contributors;
  plan->workspace_bytes = p.workspace_bytes;
  plan->slice_cols = p.slice_cols;
  plan->schedule = p.schedule;
}

}  // namespace

int fk_arc_w4a16_plan_for(int batch, int n, int k, int group_size, int activation_dtype,
                          int split_k_slices, int cu_count, fk_arc_w4a16_plan* plan) {
  return guarded([&] {
    if (plan == nullptr) {
      throw std::invalid_argument("plan must not be null");
    }
    copy_plan(cu_count > 0 ? ops::plan_arc_w4a16_for_cu_count(batch, n, k, group_size,
                                                              activation_dtype, split_k_slices,
                                                              cu_count)
                           : ops::plan_arc_w4a16(batch, n, k, group_size, activation_dtype,
                                                 split_k_slices),
              plan);
  });
}

int fk_w4a16_plan_for_format(int batch, int n, int k, int group_size, int activation_dtype,
                             int split_k_slices, int cu_count, int packet_format,
                             fk_arc_w4a16_plan* plan) {
  return guarded([&] {
    if (plan == nullptr) {
      throw std::invalid_argument("plan must not be null");
    }
    copy_plan(ops::plan_w4a16_for_format(batch, n, k, group_size, activation_dtype,
                                         split_k_slices, cu_count, packet_format),
              plan);
  });
}

int fk_arc_w4a16_forward_ex(const void* activations, const void* packets, void* output,
                            void* workspace, size_t workspace_bytes, int batch, int n, int k,
                            int group_size, int packet_stride_bytes, int activation_dtype,
                            int split_k_slices, void* stream) {
  return guarded([&] {
    ops::arc_w4a16_forward_ex(P(activations), P(packets), P(output), P(workspace), workspace_bytes,
                              batch, n, k, group_size, packet_stride_bytes, activation_dtype,
                              split_k_slices, P(stream));
  });
}

int fk_packet_stride_bytes(int group_size, int packet_format) {
  int stride = -1;
  const int status =
      guarded([&] { stride = ops::packet_format_stride_bytes(group_size, packet_format); });
  return status == FK_OK ? stride : -1;
}

int fk_pack_native_w4a16_packets(const void* q, const void* alpha, const void* zero_points,
                                 void* packets, int n, int k, int group_size, int packet_format,
                                 void* stream) {
  return guarded([&] {
    ops::pack_native_w4a16_packets(P(q), P(alpha), P(zero_points), P(packets), n, k, group_size,
                                   packet_format, P(stream));
  });
}

int fk_convert_arc_to_native_packets(const void* arc_packets, void* native_packets, int n, int k,
                                     int group_size, int packet_format, void* stream) {
  return guarded([&] {
    ops::convert_arc_w4a16_packets_to_native(P(arc_packets), P(native_packets), n, k, group_size,
                                             packet_format, P(stream));
  });
}

int fk_convert_native_to_arc_packets(const void* native_packets, void* arc_packets, int n, int k,
                                     int group_size, int packet_format, void* stream) {
  return guarded([&] {
    ops::convert_native_w4a16_packets_to_arc(P(native_packets), P(arc_packets), n, k, group_size,
                                             packet_format, P(stream));
  });
}

int fk_w4a16_plan_for_kernel(int batch, int n, int k, int group_size, int activation_dtype,
                             int split_k_slices, int cu_count, int packet_format, int kernel,
                             fk_arc_w4a16_plan* plan) {
  return guarded([&] {
    if (plan == nullptr) {
      throw std::invalid_argument("plan must not be null");
    }
    copy_plan(ops::plan_w4a16_for_kernel(batch, n, k, group_size, activation_dtype,
                                         split_k_slices, cu_count, packet_format, kernel),
              plan);
  });
}

int fk_w4a16_forward_kernel(const void* activations, const void* packets, void* output,
                            void* workspace, size_t workspace_bytes, int batch, int n, int k,
                            int group_size, int packet_format, int activation_dtype,
                            int split_k_slices, int kernel, void* stream) {
  return guarded([&] {
    ops::w4a16_forward_kernel(P(activations), P(packets), P(output), P(workspace), workspace_bytes,
                              batch, n, k, group_size, packet_format, activation_dtype,
                              split_k_slices, kernel, P(stream));
  });
}

int fk_arc_w4a16_forward_native(const void* activations, const void* packets, void* output,
                                void* workspace, size_t workspace_bytes, int batch, int n, int k,
                                int group_size, int packet_format, int activation_dtype,
                                int split_k_slices, void* stream) {
  return guarded([&] {
    ops::arc_w4a16_forward_native(P(activations), P(packets), P(output), P(workspace),
                                  workspace_bytes, batch, n, k, group_size, packet_format,
                                  activation_dtype, split_k_slices, P(stream));
  });
}

int fk_w4a16_forward_noalloc(const void* activations, const void* packets, void* output, int batch,
                             int n, int k, int group_size, int packet_format,
                             int activation_dtype, void* stream) {
  return guarded([&] {
    ops::w4a16_forward_noalloc(P(activations), P(packets), P(output), batch, n, k, group_size,
                               packet_format, activation_dtype, P(stream));
  });
}

int fk_w4a16_plan_rmsnorm(int batch, int n, int k, int group_size, int activation_dtype,
                          int split_k_slices, int cu_count, int packet_format,
                          fk_arc_w4a16_plan* plan) {
  return guarded([&] {
    if (plan == nullptr) {
      throw std::invalid_argument("plan must not be null");
    }
    copy_plan(ops::plan_w4a16_rmsnorm(batch, n, k, group_size, activation_dtype, split_k_slices,
                                      cu_count, packet_format),
              plan);
  });
}

int fk_w4a16_forward_rmsnorm(const void* activations, const void* norm_weight, float eps,
                             const void* packets, void* output, void* workspace,
                             size_t workspace_bytes, int batch, int n, int k, int group_size,
                             int packet_format, int activation_dtype, int split_k_slices,
                             void* stream) {
  return guarded([&] {
    ops::arc_w4a16_forward_rmsnorm(P(activations), P(norm_weight), eps, P(packets), P(output),
                                   P(workspace), workspace_bytes, batch, n, k, group_size,
                                   packet_format, activation_dtype, split_k_slices, P(stream));
  });
}

int fk_w4a16_forward_silu_mul(const void* activations, const void* packets, void* output,
                              int batch, int n, int k, int group_size, int packet_format,
                              int activation_dtype, const void* norm_weight, float eps,
                              void* stream) {
  return guarded([&] {
    ops::arc_w4a16_forward_silu_mul(P(activations), P(packets), P(output), batch, n, k,
                                    group_size, packet_format, activation_dtype, P(stream),
                                    P(norm_weight), eps);
  });
}

}  // extern "C"
