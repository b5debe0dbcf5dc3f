// Python module `_ext`: the reference's native binding surface
// (native/bindings/coords.cpp:414-626, convolution.cpp:12-274) over torch
// device tensors.  Relation builders return the reference's 10-tuple
// (coords.cpp:79-92); the *_with_view variants append the implicit-GEMM view
// (out_in_map, row_masks) computed by the same pass.

#include <torch/extension.h>

#include <array>
#include <vector>

#include "features/convolution/api.h"
#include "features/pooling/api.h"
#include "features/quantization/api.h"
#include "features/coordinates/relations.h"
#include "foundation/runtime.h"
#include "lattice_hip.h"

namespace ln = lattice_native;
namespace py = pybind11;

namespace {

ln::Triple triple_from_values(const std::vector<int>& values, const char* name) {
    if (values.size() == 1) return {values[0], values[0], values[0]};
    if (values.size() != 3) throw std::invalid_argument(std::string(name) + " must be an int or a 3-tuple.");
    return {values[0], values[1], values[2]};
}

py::tuple relation_tuple(const ln::NativeKernelRelation& r) {
    return py::make_tuple(r.in_rows, r.out_rows, r.kernel_ids, r.output_row_offsets, r.out_coords, r.counts,
                          r.in_row_offsets, r.in_edge_ids, r.kernel_row_offsets, r.kernel_edge_ids);
}

// Grouped views are not built here (None); build_relation_grouped_views
// makes them on demand.  The device status word (lattice_relation_flags)
// and the build's workspace (whose block table a later build over the same
// coordinates may reuse: `table=`) follow the implicit-GEMM view.
py::tuple relation_tuple_with_view(const ln::NativeKernelRelation& r) {
    return py::make_tuple(r.in_rows, r.out_rows, r.kernel_ids, r.output_row_offsets, r.out_coords, r.counts,
                          py::none(), py::none(), py::none(), py::none(), r.out_in_map, r.row_masks, r.status,
                          r.table);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "MI355X-native sparse convolution hot path (gfx950 HIP kernels behind a C ABI).";
    m.def("version", []() { return std::string(lattice_hip_version()); });
    m.def("coord_hash_capacity", [](int rows) { return lattice_hip_coord_hash_capacity(rows); }, py::arg("rows"));
    m.def(
        "kernel_offsets",
        [](const std::vector<int>& kernel_size, const std::vector<int>& dilation) {
            return ln::kernel_offsets(triple_from_values(kernel_size, "kernel_size"),
                                      triple_from_values(dilation, "dilation"));
        },
        py::arg("kernel_size"), py::arg("dilation"));

    auto forward = [](bool with_view) {
        return [with_view](const at::Tensor& coords, const at::Tensor& active_rows,
                           const std::vector<int>& kernel_size, const std::vector<int>& stride,
                           const std::vector<int>& padding, const std::vector<int>& dilation,
                           const std::optional<at::Tensor>& table) {
            auto r = ln::make_kernel_relation(coords, active_rows, triple_from_values(kernel_size, "kernel_size"),
                                              triple_from_values(stride, "stride"),
                                              triple_from_values(padding, "padding"),
                                              triple_from_values(dilation, "dilation"), !with_view, table);
            return with_view ? relation_tuple_with_view(r) : relation_tuple(r);
        };
    };
    m.def("build_kernel_relation", forward(false), py::arg("coords"), py::arg("active_rows"),
          py::arg("kernel_size"), py::arg("stride"), py::arg("padding"), py::arg("dilation"), py::kw_only(),
          py::arg("table") = py::none(), "Build a forward sparse kernel relation.");
    m.def("build_kernel_relation_with_view", forward(true), py::arg("coords"), py::arg("active_rows"),
          py::arg("kernel_size"), py::arg("stride"), py::arg("padding"), py::arg("dilation"), py::kw_only(),
          py::arg("table") = py::none());

    auto subm = [](bool with_view) {
        return [with_view](const at::Tensor& coords, const at::Tensor& active_rows,
                           const std::vector<int>& kernel_size, const std::vector<int>& dilation) {
            auto r = ln::make_submanifold_kernel_relation(coords, active_rows,
                                                          triple_from_values(kernel_size, "kernel_size"),
                                                          triple_from_values(dilation, "dilation"), !with_view);
            return with_view ? relation_tuple_with_view(r) : relation_tuple(r);
        };
    };
    m.def("build_submanifold_kernel_relation", subm(false), py::arg("coords"), py::arg("active_rows"),
          py::arg("kernel_size"), py::arg("dilation"),
          "Build a submanifold sparse kernel relation.");
    m.def("build_submanifold_kernel_relation_with_view", subm(true), py::arg("coords"), py::arg("active_rows"),
          py::arg("kernel_size"), py::arg("dilation"));

    auto target = [](bool with_view) {
        return [with_view](const at::Tensor& coords, const at::Tensor& active_rows, const at::Tensor& target_coords,
                           const at::Tensor& target_active_rows, const std::vector<int>& kernel_size,
                           const std::vector<int>& stride, const std::vector<int>& padding,
                           const std::vector<int>& dilation) {
            auto r = ln::make_target_kernel_relation(
                coords, active_rows, target_coords, target_active_rows,
                triple_from_values(kernel_size, "kernel_size"), triple_from_values(stride, "stride"),
                triple_from_values(padding, "padding"), triple_from_values(dilation, "dilation"), !with_view);
            return with_view ? relation_tuple_with_view(r) : relation_tuple(r);
        };
    };
    m.def("build_target_kernel_relation", target(false), py::arg("coords"), py::arg("active_rows"),
          py::arg("target_coords"), py::arg("target_active_rows"), py::arg("kernel_size"), py::arg("stride"),
          py::arg("padding"), py::arg("dilation"),
          "Build a target-aligned sparse kernel relation.");
    m.def("build_target_kernel_relation_with_view", target(true), py::arg("coords"), py::arg("active_rows"),
          py::arg("target_coords"), py::arg("target_active_rows"), py::arg("kernel_size"), py::arg("stride"),
          py::arg("padding"), py::arg("dilation"));

    // Generative / transposed relations.  The *_lazy variants leave the
    // grouped views to build_relation_grouped_views and append the build's
    // device status word (int32 (1,), lattice_relation_flags).
    auto expanded = [](bool generative, bool lazy) {
        return [generative, lazy](const at::Tensor& coords, const at::Tensor& active_rows,
                                  const std::vector<int>& kernel_size, const std::vector<int>& stride,
                                  const std::vector<int>& padding, const std::vector<int>& dilation) -> py::tuple {
            auto r = ln::make_expanded_relation(coords, active_rows, triple_from_values(kernel_size, "kernel_size"),
                                                triple_from_values(stride, "stride"),
                                                triple_from_values(padding, "padding"),
                                                triple_from_values(dilation, "dilation"), generative, !lazy);
            if (!lazy) return relation_tuple(r);
            return py::make_tuple(r.in_rows, r.out_rows, r.kernel_ids, r.output_row_offsets, r.out_coords, r.counts,
                                  py::none(), py::none(), py::none(), py::none(), r.status);
        };
    };
    auto generative = [expanded](bool lazy) {
        auto fn = expanded(true, lazy);
        return [fn](const at::Tensor& coords, const at::Tensor& active_rows, const std::vector<int>& kernel_size,
                    const std::vector<int>& stride) {
            return fn(coords, active_rows, kernel_size, stride, {0}, {1});
        };
    };
    m.def("build_generative_relation", generative(false), py::arg("coords"), py::arg("active_rows"),
          py::arg("kernel_size"), py::arg("stride"),
          "Build a generative sparse kernel relation.");
    m.def("build_generative_relation_lazy", generative(true), py::arg("coords"), py::arg("active_rows"),
          py::arg("kernel_size"), py::arg("stride"));
    m.def("build_transposed_kernel_relation", expanded(false, false), py::arg("coords"), py::arg("active_rows"),
          py::arg("kernel_size"), py::arg("stride"), py::arg("padding"), py::arg("dilation"),
          "Build a transposed sparse kernel relation.");
    m.def("build_transposed_kernel_relation_lazy", expanded(false, true), py::arg("coords"),
          py::arg("active_rows"), py::arg("kernel_size"), py::arg("stride"), py::arg("padding"),
          py::arg("dilation"));

    m.def(
        "build_relation_grouped_views",
        [](const at::Tensor& in_rows, const at::Tensor& kernel_ids, const at::Tensor& counts, int in_capacity,
           int n_kernels) {
            auto r = ln::make_relation_grouped_views(in_rows, kernel_ids, counts, in_capacity, n_kernels);
            return py::make_tuple(std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r));
        },
        py::arg("in_rows"), py::arg("kernel_ids"), py::arg("counts"), py::arg("in_capacity"), py::arg("n_kernels"),
        "Return (in_row_offsets, in_edge_ids, kernel_row_offsets, kernel_edge_ids).");
    m.def(
        "build_relation_implicit_gemm_view",
        [](const at::Tensor& source_coords, const at::Tensor& source_active_rows, const at::Tensor& output_coords,
           const at::Tensor& output_active_rows, const at::Tensor& offsets, const std::vector<int>& stride,
           const std::vector<int>& padding) {
            auto r = ln::make_relation_implicit_gemm_view(source_coords, source_active_rows, output_coords,
                                                          output_active_rows, offsets,
                                                          triple_from_values(stride, "stride"),
                                                          triple_from_values(padding, "padding"));
            return py::make_tuple(std::get<0>(r), std::get<1>(r));
        },
        py::arg("source_coords"), py::arg("source_active_rows"), py::arg("output_coords"),
        py::arg("output_active_rows"), py::arg("offsets"), py::arg("stride"), py::arg("padding"),
        "Build the dense output-to-input implicit-GEMM map.");
    m.def(
        "build_sorted_implicit_gemm_view",
        [](const at::Tensor& out_in_map, const at::Tensor& row_masks) {
            auto r = ln::make_sorted_implicit_gemm_view(out_in_map, row_masks);
            return py::make_tuple(std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r));
        },
        py::arg("out_in_map"), py::arg("row_masks"),
        "Return (reorder_rows, sorted_out_in_map, sorted_kv_out_in_map, tile_masks).");

    m.def("sparse_conv_features", &ln::sparse_conv_features, py::arg("feats"), py::arg("weights"),
          py::arg("in_rows"), py::arg("out_rows"), py::arg("kernel_ids"), py::arg("counts"), py::arg("row_offsets"),
          py::arg("in_row_offsets"), py::arg("in_edge_ids"), py::arg("kernel_row_offsets"),
          py::arg("kernel_edge_ids"), py::arg("out_capacity"), py::arg("n_kernels"), py::kw_only(),
          py::arg("bias") = py::none(), py::arg("relu") = false);
    m.def("sparse_conv_features_expand", &ln::sparse_conv_features_expand, py::arg("feats"), py::arg("weights"),
          py::arg("active_rows"), py::arg("n_kernels"), py::kw_only(), py::arg("bias") = py::none(),
          py::arg("relu") = false);
    m.def("sparse_conv_features_csr", &ln::sparse_conv_features_csr, py::arg("feats"), py::arg("weights"),
          py::arg("in_rows"), py::arg("kernel_ids"), py::arg("counts"), py::arg("row_offsets"),
          py::arg("out_capacity"), py::arg("n_kernels"), py::kw_only(), py::arg("bias") = py::none(),
          py::arg("relu") = false, py::arg("out_in_map") = py::none());
    m.def(
        "sparse_conv_features_sorted_implicit_gemm",
        [](const at::Tensor& feats, const at::Tensor& weights, const at::Tensor& sorted_out_in_map,
           const at::Tensor& sorted_kv_out_in_map, const at::Tensor& reorder_rows, const at::Tensor& tile_masks,
           // The relation arrays of the reference signature are accepted and
           // not read: the sorted view already holds the map.
           const py::object& /*in_rows*/, const py::object& /*out_rows*/, const py::object& /*kernel_ids*/,
           const py::object& /*counts*/, const py::object& /*row_offsets*/, const py::object& /*in_row_offsets*/,
           const py::object& /*in_edge_ids*/, const py::object& /*kernel_row_offsets*/,
           const py::object& /*kernel_edge_ids*/, int out_capacity, int n_kernels, bool store_sorted,
           const std::optional<at::Tensor>& bias, const std::optional<at::Tensor>& tile_order, bool relu,
           const std::optional<at::Tensor>& weight_fragments) {
            return ln::sparse_conv_features_sorted_implicit_gemm(feats, weights, sorted_out_in_map,
                                                                 sorted_kv_out_in_map, reorder_rows, tile_masks,
                                                                 out_capacity, n_kernels, store_sorted, bias,
                                                                 tile_order, relu, weight_fragments);
        },
        py::arg("feats"), py::arg("weights"), py::arg("sorted_out_in_map"), py::arg("sorted_kv_out_in_map"),
        py::arg("reorder_rows"), py::arg("tile_masks"), py::arg("in_rows"), py::arg("out_rows"),
        py::arg("kernel_ids"), py::arg("counts"), py::arg("row_offsets"), py::arg("in_row_offsets"),
        py::arg("in_edge_ids"), py::arg("kernel_row_offsets"), py::arg("kernel_edge_ids"), py::arg("out_capacity"),
        py::arg("n_kernels"), py::arg("store_sorted") = false, py::kw_only(), py::arg("bias") = py::none(),
        py::arg("tile_order") = py::none(), py::arg("relu") = false, py::arg("weight_fragments") = py::none());
    m.def("conv_weight_fragments", &ln::conv_weight_fragments, py::arg("weights"),
          "Fragment-ordered copy of a 5D fp16/bf16 weight for the streamed matrix-core conv (empty when the shape "
          "does not take it).");
    m.def("sparse_quantized_conv_features", &ln::sparse_quantized_conv_features, py::arg("feats"),
          py::arg("weights"), py::arg("scales"), py::arg("biases"), py::arg("in_rows"), py::arg("out_rows"),
          py::arg("kernel_ids"), py::arg("counts"), py::arg("row_offsets"), py::arg("sorted_kv_out_in_map"),
          py::arg("reorder_rows"), py::arg("tile_masks"), py::arg("out_capacity"), py::arg("n_kernels"),
          py::arg("in_channels"), py::arg("out_channels"), py::arg("storage_in_channels"), py::arg("group_size"),
          py::arg("bits"), py::kw_only(), py::arg("bias") = py::none(), py::arg("tile_order") = py::none(),
          py::arg("relu") = false, py::arg("weight_fragments") = py::none(), py::arg("out_in_map") = py::none());
    m.def("quantized_weight_fragments", &ln::quantized_weight_fragments, py::arg("weights"), py::arg("scales"),
          py::arg("biases"), py::arg("in_channels"), py::arg("out_channels"), py::arg("storage_in_channels"),
          py::arg("group_size"), py::arg("bits"),
          "Fragment-ordered packed copy of a quantized weight for the streamed matrix-core conv (empty when the "
          "shape does not take it).");
    m.def("conv_tile_order", &ln::conv_tile_order, py::arg("tile_masks"), py::arg("out_capacity"),
          "Longest-first order of the sorted view's 128-row tiles, for the matrix-core conv's tile_order.");

    m.def("sparse_conv_input_grad", &ln::sparse_conv_input_grad, py::arg("cotangent"), py::arg("weights"),
          py::arg("out_rows"), py::arg("kernel_ids"), py::arg("counts"), py::arg("in_row_offsets"),
          py::arg("in_edge_ids"), py::arg("in_capacity"), py::arg("n_kernels"),
          "Input gradient of the sparse conv over the input-grouped CSR: (in_capacity, C_in).");
    m.def(
        "build_transposed_implicit_gemm_map",
        [](const at::Tensor& in_rows, const at::Tensor& out_rows, const at::Tensor& kernel_ids,
           const at::Tensor& counts, int in_capacity, int n_kernels) {
            auto r = ln::build_transposed_implicit_gemm_map(in_rows, out_rows, kernel_ids, counts, in_capacity,
                                                            n_kernels);
            return py::make_tuple(std::get<0>(r), std::get<1>(r), std::get<2>(r));
        },
        py::arg("in_rows"), py::arg("out_rows"), py::arg("kernel_ids"), py::arg("counts"), py::arg("in_capacity"),
        py::arg("n_kernels"),
        "Return (in_out_map, row_masks, status) of a forward or submanifold relation; status flags an incomplete "
        "map (repeated coordinates).");
    m.def("sparse_conv_weight_grad", &ln::sparse_conv_weight_grad, py::arg("feats"), py::arg("cotangent"),
          py::arg("weights"), py::arg("in_rows"), py::arg("out_rows"), py::arg("counts"),
          py::arg("kernel_row_offsets"), py::arg("kernel_edge_ids"), py::arg("n_kernels"),
          "Weight gradient of the sparse conv over the kernel-grouped CSR, in the layout of `weights`.");

    m.def("sparse_pool_features", &ln::sparse_pool_features, py::arg("feats"), py::arg("in_rows"),
          py::arg("out_rows"), py::arg("kernel_ids"), py::arg("row_offsets"), py::arg("counts"),
          py::arg("input_exclusive"), py::arg("reduce"), py::arg("out_capacity"), py::arg("n_kernels"),
          "Run sparse pooling feature reduction over a kernel relation.");
    m.def("sparse_pool_features_grad", &ln::sparse_pool_features_grad, py::arg("cotangent"), py::arg("feats"),
          py::arg("pooled"), py::arg("in_rows"), py::arg("out_rows"), py::arg("row_offsets"), py::arg("counts"),
          py::arg("in_row_offsets"), py::arg("in_edge_ids"), py::arg("reduce"),
          "Gradient of sparse pooling with respect to the input features.");
    m.def("sparse_quantize", &ln::sparse_quantize, py::arg("points"), py::arg("batch_indices"),
          py::arg("active_rows"), py::arg("voxel_size"), py::arg("origin"),
          "Voxelize points: (coords, active_rows, inverse_rows, counts).");
    m.def("group_by_key", &ln::group_by_key, py::arg("keys"), py::arg("count"), py::arg("groups"));
    m.def("voxelize_features", &ln::voxelize_features, py::arg("feats"), py::arg("inverse_rows"),
          py::arg("counts"), py::arg("active_rows"), py::arg("reduction"));
    m.def("voxelize_features_grouped", &ln::voxelize_features_grouped, py::arg("feats"), py::arg("counts"),
          py::arg("voxel_offsets"), py::arg("point_ids"), py::arg("reduction"));
    m.def("voxelize_features_grad", &ln::voxelize_features_grad, py::arg("cotangent"), py::arg("inverse_rows"),
          py::arg("counts"), py::arg("active_rows"), py::arg("point_rows"), py::arg("reduction"));
    m.def("build_point_voxel_map", &ln::build_point_voxel_map, py::arg("points"), py::arg("batch_indices"),
          py::arg("point_active_rows"), py::arg("voxel_coords"), py::arg("voxel_active_rows"),
          py::arg("voxel_size"), py::arg("origin"), py::arg("interpolation"));
    m.def("interpolate_point_features", &ln::interpolate_point_features, py::arg("voxel_feats"), py::arg("rows"),
          py::arg("weights"));
    m.def("interpolate_point_features_grad", &ln::interpolate_point_features_grad, py::arg("point_grad"),
          py::arg("weights"), py::arg("voxel_offsets"), py::arg("entry_ids"), py::arg("voxel_rows"));
    m.def("global_pool", &ln::global_pool, py::arg("feats"), py::arg("batch_counts"), py::arg("mode"),
          "Per-batch global pooling: (B, C).");
}
