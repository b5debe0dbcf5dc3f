// Relation builders over torch device tensors: validation, output and
// workspace allocation on the caller's device and current stream, then the
// C-ABI call.  Mirrors native/features/coordinates/api.h:67-136 of the
// reference.
#pragma once

#include <torch/extension.h>

#include <array>
#include <tuple>

namespace lattice_native {

using Triple = std::array<int, 3>;

struct NativeKernelRelation {
    at::Tensor in_rows;
    at::Tensor out_rows;
    at::Tensor kernel_ids;
    at::Tensor output_row_offsets;
    at::Tensor out_coords;
    at::Tensor counts;
    at::Tensor in_row_offsets;
    at::Tensor in_edge_ids;
    at::Tensor kernel_row_offsets;
    at::Tensor kernel_edge_ids;
    // Dense implicit-GEMM view computed by the same query pass.
    at::Tensor out_in_map;
    at::Tensor row_masks;
    // The build's device status word (lattice_relation_flags), left on the
    // device: nothing in a build waits for the device.
    at::Tensor status;
    // The block table of the input coordinates (a buffer of its own): a
    // later build over the same coordinates may reuse it
    // (LATTICE_RELATION_TABLE_READY).
    at::Tensor table;
};

std::vector<Triple> kernel_offsets(Triple kernel_size, Triple dilation);

// Builds never read device memory back: every int32 coordinate is accepted.
// with_views: also build the grouped CSR views (otherwise their tensors
// stay undefined and make_relation_grouped_views builds them on demand).
// table (optional): the `table` of an earlier build over the same coords
// and active_rows; its block table is reused instead of rebuilt.
NativeKernelRelation make_kernel_relation(const at::Tensor& coords, const at::Tensor& active_rows,
                                          Triple kernel_size, Triple stride, Triple padding, Triple dilation,
                                          bool with_views = true,
                                          const std::optional<at::Tensor>& table = std::nullopt);

NativeKernelRelation make_submanifold_kernel_relation(const at::Tensor& coords, const at::Tensor& active_rows,
                                                      Triple kernel_size, Triple dilation,
                                                      bool with_views = true);

NativeKernelRelation make_target_kernel_relation(const at::Tensor& coords, const at::Tensor& active_rows,
                                                 const at::Tensor& target_coords,
                                                 const at::Tensor& target_active_rows, Triple kernel_size,
                                                 Triple stride, Triple padding, Triple dilation,
                                                 bool with_views = true);

// Generative (generative = true; padding and dilation ignored) and
// transposed relations: output and edge capacities rows * K, no dense view.
NativeKernelRelation make_expanded_relation(const at::Tensor& coords, const at::Tensor& active_rows,
                                            Triple kernel_size, Triple stride, Triple padding, Triple dilation,
                                            bool generative, bool with_views = true);

// (in_row_offsets, in_edge_ids, kernel_row_offsets, kernel_edge_ids)
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> make_relation_grouped_views(
    const at::Tensor& in_rows, const at::Tensor& kernel_ids, const at::Tensor& counts, int in_capacity,
    int kernel_count);

std::tuple<at::Tensor, at::Tensor> make_relation_implicit_gemm_view(
    const at::Tensor& source_coords, const at::Tensor& source_active_rows, const at::Tensor& output_coords,
    const at::Tensor& output_active_rows, const at::Tensor& offsets, Triple stride, Triple padding);

// (reorder_rows, sorted_out_in_map, sorted_kv_out_in_map, tile_masks)
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> make_sorted_implicit_gemm_view(
    const at::Tensor& out_in_map, const at::Tensor& row_masks);

}  // namespace lattice_native
