// pybind11 module fast_kernels._native over the C ABI of libfk_w4a16.so (include/fk_w4a16.h).
//
// Mirrors the reference module (csrc/bindings/python_module.cpp:17-26 build_info, :119-240 the
// W4A16 defs): same function names and keyword arguments (*_ptr as integers, batch, n, k,
// group_size, packet_stride_bytes, split_k_slices, stream_ptr), the GIL released around every
// device call, FK_ERR_INVALID_ARGUMENT raised as ValueError and FK_ERR_RUNTIME as RuntimeError
// (pybind's mapping of the reference's std::invalid_argument / std::runtime_error). The vendor
// baseline is bound under both the reference's cublaslt_* names and hipblaslt_* names.
#include <pybind11/pybind11.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "fk_w4a16.h"

namespace py = pybind11;

// 1 when libfk_w4a16.so holds the HIP kernels, 0 for the host-only stub (FK_ENABLE_HIP=OFF).
#ifndef FK_COMPILED_WITH_HIP
#define FK_COMPILED_WITH_HIP 1
#endif

namespace {

void check(int status) {
  if (status == FK_OK) {
    return;
  }
  const std::string message = fk_last_error();
  if (status == FK_ERR_INVALID_ARGUMENT) {
    throw py::value_error(message);
  }
  throw std::runtime_error(message);
}

inline const void* cp(std::uintptr_t p) { return reinterpret_cast<const void*>(p); }
inline void* mp(std::uintptr_t p) { return reinterpret_cast<void*>(p); }

template <typename Fn>
void call(Fn&& fn) {
  int status = FK_OK;
  {
    py::gil_scoped_release release;
    status = fn();
  }
  check(status);
}

}  // namespace

PYBIND11_MODULE(_native, m) {
  m.doc() = "MI355X (gfx950) W4A16 decode-linear kernels for fast-kernels.";
  m.def("build_info", []() {
    py::dict info;
    info["project_version"] = std::string("0.1.0");
    info["library"] = std::string(fk_build_info());
    info["compiled_with_hip"] = FK_COMPILED_WITH_HIP != 0;
    info["compiled_with_cuda"] = false;
    info["compiled_with_gpu"] = FK_COMPILED_WITH_HIP != 0;
    info["hip_architectures"] = std::string(FK_COMPILED_WITH_HIP ? "gfx950" : "");
    info["cxx_compiler_id"] = std::string("GNU");
    info["cxx_compiler_version"] = std::string(__VERSION__);
    return info;
  });

  m.def(
      "compute_arc_w4a16_group_sums",
      [](std::uintptr_t activations_ptr, std::uintptr_t sums_ptr, int batch, int k, int group_size,
         std::uintptr_t stream_ptr) {
        call([&] {
          return fk_compute_arc_w4a16_group_sums(cp(activations_ptr), mp(sums_ptr), batch, k,
                                                 group_size, mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("sums_ptr"), py::arg("batch"), py::arg("k"),
      py::arg("group_size"), py::arg("stream_ptr"));
  m.def(
      "pack_arc_w4a16_packets",
      [](std::uintptr_t q_ptr, std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
         std::uintptr_t packets_ptr, int n, int k, int group_size, int packet_stride_bytes,
         std::uintptr_t stream_ptr) {
        call([&] {
          return fk_pack_arc_w4a16_packets(cp(q_ptr), cp(alpha_ptr), cp(beta_ptr), mp(packets_ptr),
                                           n, k, group_size, packet_stride_bytes, mp(stream_ptr));
        });
      },
      py::arg("q_ptr"), py::arg("alpha_ptr"), py::arg("beta_ptr"), py::arg("packets_ptr"),
      py::arg("n"), py::arg("k"), py::arg("group_size"), py::arg("packet_stride_bytes"),
      py::arg("stream_ptr"));
  m.def(
      "arc_w4a16_forward",
      [](std::uintptr_t activations_ptr, std::uintptr_t packets_ptr, std::uintptr_t group_sums_ptr,
         std::uintptr_t output_ptr, int batch, int n, int k, int group_size,
         int packet_stride_bytes, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_arc_w4a16_forward(cp(activations_ptr), cp(packets_ptr), cp(group_sums_ptr),
                                      mp(output_ptr), batch, n, k, group_size,
                                      packet_stride_bytes, mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("packets_ptr"), py::arg("group_sums_ptr"),
      py::arg("output_ptr"), py::arg("batch"), py::arg("n"), py::arg("k"), py::arg("group_size"),
      py::arg("packet_stride_bytes"), py::arg("stream_ptr"));
  m.def(
      "arc_w4a16_forward_split_k",
      [](std::uintptr_t activations_ptr, std::uintptr_t packets_ptr, std::uintptr_t group_sums_ptr,
         std::uintptr_t partials_ptr, int batch, int n, int k, int group_size,
         int packet_stride_bytes, int split_k_slices, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_arc_w4a16_forward_split_k(cp(activations_ptr), cp(packets_ptr),
                                              cp(group_sums_ptr), mp(partials_ptr), batch, n, k,
                                              group_size, packet_stride_bytes, split_k_slices,
                                              mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("packets_ptr"), py::arg("group_sums_ptr"),
      py::arg("partials_ptr"), py::arg("batch"), py::arg("n"), py::arg("k"), py::arg("group_size"),
      py::arg("packet_stride_bytes"), py::arg("split_k_slices"), py::arg("stream_ptr"));
  m.def(
      "reduce_arc_w4a16_split_k_partials",
      [](std::uintptr_t partials_ptr, std::uintptr_t output_ptr, int batch, int n,
         int split_k_slices, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_reduce_arc_w4a16_split_k_partials(cp(partials_ptr), mp(output_ptr), batch, n,
                                                      split_k_slices, mp(stream_ptr));
        });
      },
      py::arg("partials_ptr"), py::arg("output_ptr"), py::arg("batch"), py::arg("n"),
      py::arg("split_k_slices"), py::arg("stream_ptr"));
  m.def(
      "dequant_w4a16_to_fp16",
      [](std::uintptr_t q_ptr, std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
         std::uintptr_t output_ptr, int n, int k, int group_size, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_dequant_w4a16_to_fp16(cp(q_ptr), cp(alpha_ptr), cp(beta_ptr), mp(output_ptr), n,
                                          k, group_size, mp(stream_ptr));
        });
      },
      py::arg("q_ptr"), py::arg("alpha_ptr"), py::arg("beta_ptr"), py::arg("output_ptr"),
      py::arg("n"), py::arg("k"), py::arg("group_size"), py::arg("stream_ptr"));
  m.def(
      "dequant_arc_w4a16_packets_to_fp16",
      [](std::uintptr_t packets_ptr, std::uintptr_t output_ptr, int n, int k, int group_size,
         int packet_stride_bytes, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_dequant_arc_w4a16_packets_to_fp16(cp(packets_ptr), mp(output_ptr), n, k,
                                                      group_size, packet_stride_bytes,
                                                      mp(stream_ptr));
        });
      },
      py::arg("packets_ptr"), py::arg("output_ptr"), py::arg("n"), py::arg("k"),
      py::arg("group_size"), py::arg("packet_stride_bytes"), py::arg("stream_ptr"));

  auto with_weight = [](std::uintptr_t activations_ptr, std::uintptr_t weight_ptr,
                        std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
                        std::size_t workspace_bytes, int batch, int n, int k,
                        std::uintptr_t stream_ptr) {
    call([&] {
      return fk_hipblaslt_fp16_with_weight(cp(activations_ptr), cp(weight_ptr), mp(output_ptr),
                                           mp(workspace_ptr), workspace_bytes, batch, n, k,
                                           mp(stream_ptr));
    });
  };
  auto after_packet = [](std::uintptr_t activations_ptr, std::uintptr_t packets_ptr,
                         std::uintptr_t output_ptr, std::uintptr_t weight_ptr,
                         std::uintptr_t workspace_ptr, std::size_t workspace_bytes, int batch,
                         int n, int k, int group_size, int packet_stride_bytes,
                         std::uintptr_t stream_ptr) {
    call([&] {
      return fk_hipblaslt_fp16_after_packet_dequant(
          cp(activations_ptr), cp(packets_ptr), mp(output_ptr), mp(weight_ptr), mp(workspace_ptr),
          workspace_bytes, batch, n, k, group_size, packet_stride_bytes, mp(stream_ptr));
    });
  };
  auto after_dequant = [](std::uintptr_t activations_ptr, std::uintptr_t q_ptr,
                          std::uintptr_t alpha_ptr, std::uintptr_t beta_ptr,
                          std::uintptr_t output_ptr, std::uintptr_t weight_ptr,
                          std::uintptr_t workspace_ptr, std::size_t workspace_bytes, int batch,
                          int n, int k, int group_size, std::uintptr_t stream_ptr) {
    call([&] {
      return fk_hipblaslt_fp16_after_dequant(cp(activations_ptr), cp(q_ptr), cp(alpha_ptr),
                                             cp(beta_ptr), mp(output_ptr), mp(weight_ptr),
                                             mp(workspace_ptr), workspace_bytes, batch, n, k,
                                             group_size, mp(stream_ptr));
    });
  };
  for (const char* prefix : {"cublaslt", "hipblaslt"}) {
    const std::string p(prefix);
    m.def((p + "_fp16_with_weight").c_str(), with_weight, py::arg("activations_ptr"),
          py::arg("weight_ptr"), py::arg("output_ptr"), py::arg("workspace_ptr"),
          py::arg("workspace_bytes"), py::arg("batch"), py::arg("n"), py::arg("k"),
          py::arg("stream_ptr"));
    m.def((p + "_fp16_after_packet_dequant").c_str(), after_packet, py::arg("activations_ptr"),
          py::arg("packets_ptr"), py::arg("output_ptr"), py::arg("weight_ptr"),
          py::arg("workspace_ptr"), py::arg("workspace_bytes"), py::arg("batch"), py::arg("n"),
          py::arg("k"), py::arg("group_size"), py::arg("packet_stride_bytes"),
          py::arg("stream_ptr"));
    m.def((p + "_fp16_after_dequant").c_str(), after_dequant, py::arg("activations_ptr"),
          py::arg("q_ptr"), py::arg("alpha_ptr"), py::arg("beta_ptr"), py::arg("output_ptr"),
          py::arg("weight_ptr"), py::arg("workspace_ptr"), py::arg("workspace_bytes"),
          py::arg("batch"), py::arg("n"), py::arg("k"), py::arg("group_size"),
          py::arg("stream_ptr"));
  }

  // Additions with no reference counterpart.
  m.def(
      "arc_w4a16_plan",
      [](int batch, int n, int k, int group_size, int activation_dtype, int split_k_slices,
         int cu_count, int packet_format, int kernel) {
        fk_arc_w4a16_plan plan{};
        check(fk_w4a16_plan_for_kernel(batch, n, k, group_size, activation_dtype, split_k_slices,
                                       cu_count, packet_format, kernel, &plan));
        py::dict d;
        d["m_tile"] = plan.m_tile;
        d["workgroups"] = plan.workgroups;
        d["groups_per_workgroup"] = plan.groups_per_workgroup;
        d["max_tile_contributors"] = plan.max_tile_contributors;
        d["workspace_bytes"] = plan.workspace_bytes;
        d["slice_cols"] = plan.slice_cols;
        d["schedule"] = plan.schedule;
        return d;
      },
      py::arg("batch"), py::arg("n"), py::arg("k"), py::arg("group_size"),
      py::arg("activation_dtype") = FK_ACT_F16, py::arg("split_k_slices") = 0,
      py::arg("cu_count") = 0, py::arg("packet_format") = FK_PACKET_ARC,
      py::arg("kernel") = FK_KERNEL_AUTO);
  m.def(
      "arc_w4a16_forward_ex",
      [](std::uintptr_t activations_ptr, std::uintptr_t packets_ptr, std::uintptr_t output_ptr,
         std::uintptr_t workspace_ptr, std::size_t workspace_bytes, int batch, int n, int k,
         int group_size, int packet_stride_bytes, int activation_dtype, int split_k_slices,
         std::uintptr_t stream_ptr) {
        call([&] {
          return fk_arc_w4a16_forward_ex(cp(activations_ptr), cp(packets_ptr), mp(output_ptr),
                                         mp(workspace_ptr), workspace_bytes, batch, n, k,
                                         group_size, packet_stride_bytes, activation_dtype,
                                         split_k_slices, mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("packets_ptr"), py::arg("output_ptr"),
      py::arg("workspace_ptr"), py::arg("workspace_bytes"), py::arg("batch"), py::arg("n"),
      py::arg("k"), py::arg("group_size"), py::arg("packet_stride_bytes"),
      py::arg("activation_dtype"), py::arg("split_k_slices"), py::arg("stream_ptr"));
  m.attr("PACKET_ARC") = FK_PACKET_ARC;
  m.attr("PACKET_NATIVE_SYM") = FK_PACKET_NATIVE_SYM;
  m.attr("PACKET_NATIVE_ASYM") = FK_PACKET_NATIVE_ASYM;
  m.def(
      "packet_stride_bytes",
      [](int group_size, int packet_format) {
        const int stride = fk_packet_stride_bytes(group_size, packet_format);
        if (stride < 0) {
          throw std::invalid_argument(fk_last_error());
        }
        return stride;
      },
      py::arg("group_size"), py::arg("packet_format"));
  m.def(
      "pack_native_w4a16_packets",
      [](std::uintptr_t q_ptr, std::uintptr_t alpha_ptr, std::uintptr_t zero_points_ptr,
         std::uintptr_t packets_ptr, int n, int k, int group_size, int packet_format,
         std::uintptr_t stream_ptr) {
        call([&] {
          return fk_pack_native_w4a16_packets(cp(q_ptr), cp(alpha_ptr), cp(zero_points_ptr),
                                              mp(packets_ptr), n, k, group_size, packet_format,
                                              mp(stream_ptr));
        });
      },
      py::arg("q_ptr"), py::arg("alpha_ptr"), py::arg("zero_points_ptr"), py::arg("packets_ptr"),
      py::arg("n"), py::arg("k"), py::arg("group_size"), py::arg("packet_format"),
      py::arg("stream_ptr"));
  m.def(
      "convert_arc_to_native_packets",
      [](std::uintptr_t arc_packets_ptr, std::uintptr_t native_packets_ptr, int n, int k,
         int group_size, int packet_format, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_convert_arc_to_native_packets(cp(arc_packets_ptr), mp(native_packets_ptr), n,
                                                  k, group_size, packet_format, mp(stream_ptr));
        });
      },
      py::arg("arc_packets_ptr"), py::arg("native_packets_ptr"), py::arg("n"), py::arg("k"),
      py::arg("group_size"), py::arg("packet_format"), py::arg("stream_ptr"));
  m.def(
      "convert_native_to_arc_packets",
      [](std::uintptr_t native_packets_ptr, std::uintptr_t arc_packets_ptr, int n, int k,
         int group_size, int packet_format, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_convert_native_to_arc_packets(cp(native_packets_ptr), mp(arc_packets_ptr), n,
                                                  k, group_size, packet_format, mp(stream_ptr));
        });
      },
      py::arg("native_packets_ptr"), py::arg("arc_packets_ptr"), py::arg("n"), py::arg("k"),
      py::arg("group_size"), py::arg("packet_format"), py::arg("stream_ptr"));
  m.def(
      "arc_w4a16_forward_native",
      [](std::uintptr_t activations_ptr, std::uintptr_t packets_ptr, std::uintptr_t output_ptr,
         std::uintptr_t workspace_ptr, std::size_t workspace_bytes, int batch, int n, int k,
         int group_size, int packet_format, int activation_dtype, int split_k_slices,
         std::uintptr_t stream_ptr) {
        call([&] {
          return fk_arc_w4a16_forward_native(cp(activations_ptr), cp(packets_ptr), mp(output_ptr),
                                             mp(workspace_ptr), workspace_bytes, batch, n, k,
                                             group_size, packet_format, activation_dtype,
                                             split_k_slices, mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("packets_ptr"), py::arg("output_ptr"),
      py::arg("workspace_ptr"), py::arg("workspace_bytes"), py::arg("batch"), py::arg("n"),
      py::arg("k"), py::arg("group_size"), py::arg("packet_format"), py::arg("activation_dtype"),
      py::arg("split_k_slices"), py::arg("stream_ptr"));
  m.def(
      "w4a16_forward_kernel",
      [](std::uintptr_t activations_ptr, std::uintptr_t packets_ptr, std::uintptr_t output_ptr,
         std::uintptr_t workspace_ptr, std::size_t workspace_bytes, int batch, int n, int k,
         int group_size, int packet_format, int activation_dtype, int split_k_slices, int kernel,
         std::uintptr_t stream_ptr) {
        call([&] {
          return fk_w4a16_forward_kernel(cp(activations_ptr), cp(packets_ptr), mp(output_ptr),
                                         mp(workspace_ptr), workspace_bytes, batch, n, k,
                                         group_size, packet_format, activation_dtype,
                                         split_k_slices, kernel, mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("packets_ptr"), py::arg("output_ptr"),
      py::arg("workspace_ptr"), py::arg("workspace_bytes"), py::arg("batch"), py::arg("n"),
      py::arg("k"), py::arg("group_size"), py::arg("packet_format"), py::arg("activation_dtype"),
      py::arg("split_k_slices"), py::arg("kernel"), py::arg("stream_ptr"));
  m.def(
      "w4a16_plan_rmsnorm",
      [](int batch, int n, int k, int group_size, int activation_dtype, int split_k_slices,
         int cu_count, int packet_format) {
        fk_arc_w4a16_plan plan{};
        check(fk_w4a16_plan_rmsnorm(batch, n, k, group_size, activation_dtype, split_k_slices,
                                    cu_count, packet_format, &plan));
        py::dict d;
        d["m_tile"] = plan.m_tile;
        d["workgroups"] = plan.workgroups;
        d["groups_per_workgroup"] = plan.groups_per_workgroup;
        d["max_tile_contributors"] = plan.max_tile_contributors;
        d["workspace_bytes"] = plan.workspace_bytes;
        d["slice_cols"] = plan.slice_cols;
        d["schedule"] = plan.schedule;
        return d;
      },
      py::arg("batch"), py::arg("n"), py::arg("k"), py::arg("group_size"),
      py::arg("activation_dtype"), py::arg("split_k_slices"), py::arg("cu_count"),
      py::arg("packet_format"));
  m.def(
      "w4a16_forward_rmsnorm",
      [](std::uintptr_t activations_ptr, std::uintptr_t norm_weight_ptr, float eps,
         std::uintptr_t packets_ptr, std::uintptr_t output_ptr, std::uintptr_t workspace_ptr,
         std::size_t workspace_bytes, int batch, int n, int k, int group_size, int packet_format,
         int activation_dtype, int split_k_slices, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_w4a16_forward_rmsnorm(cp(activations_ptr), cp(norm_weight_ptr), eps,
                                          cp(packets_ptr), mp(output_ptr), mp(workspace_ptr),
                                          workspace_bytes, batch, n, k, group_size, packet_format,
                                          activation_dtype, split_k_slices, mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("norm_weight_ptr"), py::arg("eps"),
      py::arg("packets_ptr"), py::arg("output_ptr"), py::arg("workspace_ptr"),
      py::arg("workspace_bytes"), py::arg("batch"), py::arg("n"), py::arg("k"),
      py::arg("group_size"), py::arg("packet_format"), py::arg("activation_dtype"),
      py::arg("split_k_slices"), py::arg("stream_ptr"));
  m.def(
      "w4a16_forward_silu_mul",
      [](std::uintptr_t activations_ptr, std::uintptr_t packets_ptr, std::uintptr_t output_ptr,
         int batch, int n, int k, int group_size, int packet_format, int activation_dtype,
         std::uintptr_t norm_weight_ptr, float eps, std::uintptr_t stream_ptr) {
        call([&] {
          return fk_w4a16_forward_silu_mul(cp(activations_ptr), cp(packets_ptr), mp(output_ptr),
                                           batch, n, k, group_size, packet_format,
                                           activation_dtype, cp(norm_weight_ptr), eps,
                                           mp(stream_ptr));
        });
      },
      py::arg("activations_ptr"), py::arg("packets_ptr"), py::arg("output_ptr"), py::arg("batch"),
      py::arg("n"), py::arg("k"), py::arg("group_size"), py::arg("packet_format"),
      py::arg("activation_dtype"), py::arg("norm_weight_ptr"), py::arg("eps"),
      py::arg("stream_ptr"));
}
