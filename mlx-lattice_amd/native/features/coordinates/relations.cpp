#include "features/coordinates/relations.h"

#include <stdexcept>
#include <string>

#include "foundation/runtime.h"

namespace lattice_native {

namespace {

void validate_coords(const at::Tensor& coords, const char* name = "coords") {
    if (coords.dim() != 2 || coords.size(1) != 4) {
        throw std::invalid_argument(std::string(name) + " must have shape (N, 4).");
    }
    if (coords.scalar_type() != at::kInt && coords.scalar_type() != at::kLong) {
        throw std::invalid_argument(std::string(name) + " must be int32 or int64.");
    }
    if (coords.scalar_type() != at::kInt) {
        throw std::invalid_argument("GPU sparse relations require int32 coordinates.");
    }
}

void validate_active_rows(const at::Tensor& active_rows) {
    if (active_rows.dim() != 1 || active_rows.size(0) != 1 || active_rows.scalar_type() != at::kInt) {
        throw std::invalid_argument("active_rows must have shape (1,) and int32 dtype.");
    }
}

void require_on_device(std::initializer_list<std::pair<const at::Tensor*, const char*>> tensors) {
    for (const auto& [t, name] : tensors) require_device(*t, name);
}

void validate_positive(const Triple& v, const char* name) {
    for (int x : v) {
        if (x <= 0) throw std::invalid_argument(std::string(name) + " values must be positive.");
    }
}

void validate_nonnegative(const Triple& v, const char* name) {
    for (int x : v) {
        if (x < 0) throw std::invalid_argument(std::string(name) + " values must be non-negative.");
    }
}

NativeKernelRelation allocate(const at::Tensor& like, int out_capacity, int in_capacity, int K, bool coords,
                              bool views) {
    const int64_t edges = static_cast<int64_t>(out_capacity) * K;
    NativeKernelRelation r;
    r.in_rows = empty_i32({edges}, like);
    r.out_rows = empty_i32({edges}, like);
    r.kernel_ids = empty_i32({edges}, like);
    r.output_row_offsets = empty_i32({out_capacity + 1}, like);
    if (coords) r.out_coords = empty_i32({out_capacity, 4}, like);
    r.counts = empty_i32({2}, like);
    if (views) {
        r.in_row_offsets = empty_i32({in_capacity + 1}, like);
        r.in_edge_ids = empty_i32({edges}, like);
        r.kernel_row_offsets = empty_i32({K + 1}, like);
        r.kernel_edge_ids = empty_i32({edges}, like);
    }
    r.out_in_map = empty_i32({out_capacity, K}, like);
    r.row_masks = empty_i32({out_capacity, (K + 31) / 32}, like);
    return r;
}

lattice_relation_outputs outputs_of(NativeKernelRelation& r, at::Tensor& status) {
    lattice_relation_outputs o{};
    o.in_rows = i32(r.in_rows);
    o.out_rows = i32(r.out_rows);
    o.kernel_ids = i32(r.kernel_ids);
    o.row_offsets = i32(r.output_row_offsets);
    o.out_coords = r.out_coords.defined() ? i32(r.out_coords) : nullptr;
    o.counts = i32(r.counts);
    const bool views = r.in_edge_ids.defined();
    o.in_row_offsets = views ? i32(r.in_row_offsets) : nullptr;
    o.in_edge_ids = views ? i32(r.in_edge_ids) : nullptr;
    o.kernel_row_offsets = views ? i32(r.kernel_row_offsets) : nullptr;
    o.kernel_edge_ids = views ? i32(r.kernel_edge_ids) : nullptr;
    o.out_in_map = i32(r.out_in_map);
    o.row_masks = i32(r.row_masks);
    o.status = i32(status);
    return o;
}

}  // namespace

std::vector<Triple> kernel_offsets(Triple kernel_size, Triple dilation) {
    validate_positive(kernel_size, "kernel_size");
    validate_positive(dilation, "dilation");
    const int K = lattice_hip_kernel_offsets(kernel_size.data(), dilation.data(), nullptr);
    std::vector<int32_t> flat(static_cast<size_t>(K) * 3);
    lattice_hip_kernel_offsets(kernel_size.data(), dilation.data(), flat.data());
    std::vector<Triple> out(static_cast<size_t>(K));
    for (int k = 0; k < K; ++k) out[k] = {flat[3 * k], flat[3 * k + 1], flat[3 * k + 2]};
    return out;
}

NativeKernelRelation make_kernel_relation(const at::Tensor& coords_in, const at::Tensor& active_rows,
                                          Triple kernel_size, Triple stride, Triple padding, Triple dilation,
                                          bool with_views, const std::optional<at::Tensor>& table) {
    validate_coords(coords_in);
    validate_active_rows(active_rows);
    validate_positive(kernel_size, "kernel_size");
    validate_positive(stride, "stride");
    validate_nonnegative(padding, "padding");
    validate_positive(dilation, "dilation");
    require_on_device({{&coords_in, "coords"}, {&active_rows, "active_rows"}});
    const at::Tensor coords = coords_in.contiguous();
    const int rows = static_cast<int>(coords.size(0));
    const int K = kernel_size[0] * kernel_size[1] * kernel_size[2];
    NativeKernelRelation r = allocate(coords, rows, rows, K, true, with_views);
    at::Tensor status = empty_i32({1}, coords);
    lattice_relation_outputs o = outputs_of(r, status);
    // The block table lives in a buffer of its own, so a caller keeping it
    // for the next relation over the same coordinates keeps only the table;
    // an earlier build's table over these coordinates is reused as it is.
    const size_t tneed = lattice_hip_block_table_bytes(rows);
    const size_t need = lattice_hip_kernel_relation_workspace_bytes(rows, K) - tneed;
    const bool reuse = table.has_value() && table->defined() && table->scalar_type() == at::kByte &&
                       table->is_contiguous() && table->device() == coords.device() &&
                       static_cast<size_t>(table->numel()) >= tneed;
    at::Tensor tb = reuse ? *table : workspace(tneed, coords);
    at::Tensor ws = workspace(need, coords);
    size_t tb_bytes = static_cast<size_t>(tb.numel());
    if (reuse) tb_bytes |= LATTICE_RELATION_TABLE_READY;
    check_status(lattice_hip_build_kernel_relation_with_table(
        ci32(coords), rows, ci32(active_rows), kernel_size.data(), stride.data(), padding.data(), dilation.data(),
        &o, tb.data_ptr(), tb_bytes, ws.data_ptr(), static_cast<size_t>(ws.numel()), current_stream(coords)));
    r.status = status;
    r.table = tb;
    return r;
}

NativeKernelRelation make_submanifold_kernel_relation(const at::Tensor& coords, const at::Tensor& active_rows,
                                                      Triple kernel_size, Triple dilation, bool with_views) {
    return make_kernel_relation(coords, active_rows, kernel_size, {1, 1, 1}, {0, 0, 0}, dilation, with_views);
}

NativeKernelRelation make_target_kernel_relation(const at::Tensor& coords_in, const at::Tensor& active_rows,
                                                 const at::Tensor& target_in, const at::Tensor& target_active_rows,
                                                 Triple kernel_size, Triple stride, Triple padding,
                                                 Triple dilation, bool with_views) {
    validate_coords(coords_in);
    validate_coords(target_in, "target_coords");
    validate_active_rows(active_rows);
    validate_active_rows(target_active_rows);
    validate_positive(kernel_size, "kernel_size");
    validate_positive(stride, "stride");
    validate_nonnegative(padding, "padding");
    validate_positive(dilation, "dilation");
    require_on_device({{&coords_in, "coords"},
                       {&active_rows, "active_rows"},
                       {&target_in, "target_coords"},
                       {&target_active_rows, "target_active_rows"}});
    const at::Tensor coords = coords_in.contiguous();
    const at::Tensor target = target_in.contiguous();
    const int rows = static_cast<int>(coords.size(0));
    const int target_rows = static_cast<int>(target.size(0));
    const int K = kernel_size[0] * kernel_size[1] * kernel_size[2];
    NativeKernelRelation r = allocate(coords, target_rows, rows, K, false, with_views);
    r.out_coords = target;
    at::Tensor status = empty_i32({1}, coords);
    lattice_relation_outputs o = outputs_of(r, status);
    o.out_coords = nullptr;
    at::Tensor ws = workspace(lattice_hip_target_relation_workspace_bytes(rows, target_rows, K), coords);
    check_status(lattice_hip_build_target_kernel_relation(
        ci32(coords), rows, ci32(active_rows), ci32(target), target_rows, ci32(target_active_rows),
        kernel_size.data(), stride.data(), padding.data(), dilation.data(), &o, ws.data_ptr(),
        static_cast<size_t>(ws.numel()), current_stream(coords)));
    r.status = status;
    return r;
}

NativeKernelRelation make_expanded_relation(const at::Tensor& coords_in, const at::Tensor& active_rows,
                                            Triple kernel_size, Triple stride, Triple padding, Triple dilation,
                                            bool generative, bool with_views) {
    validate_coords(coords_in);
    validate_active_rows(active_rows);
    validate_positive(kernel_size, "kernel_size");
    validate_positive(stride, "stride");
    if (generative) {
        padding = {0, 0, 0};
        dilation = {1, 1, 1};
    }
    validate_nonnegative(padding, "padding");
    validate_positive(dilation, "dilation");
    require_on_device({{&coords_in, "coords"}, {&active_rows, "active_rows"}});
    const at::Tensor coords = coords_in.contiguous();
    const int rows = static_cast<int>(coords.size(0));
    const int K = kernel_size[0] * kernel_size[1] * kernel_size[2];
    if (static_cast<int64_t>(rows) * K >= (int64_t{1} << 30)) {
        throw std::invalid_argument("relation capacity rows * K exceeds 2^30.");
    }
    const int cap = rows * K;
    NativeKernelRelation r;
    r.in_rows = empty_i32({cap}, coords);
    r.out_rows = empty_i32({cap}, coords);
    r.kernel_ids = empty_i32({cap}, coords);
    r.output_row_offsets = empty_i32({cap + 1}, coords);
    r.out_coords = empty_i32({cap, 4}, coords);
    r.counts = empty_i32({2}, coords);
    if (with_views) {
        r.in_row_offsets = empty_i32({rows + 1}, coords);
        r.in_edge_ids = empty_i32({cap}, coords);
        r.kernel_row_offsets = empty_i32({K + 1}, coords);
        r.kernel_edge_ids = empty_i32({cap}, coords);
    }
    at::Tensor status = empty_i32({1}, coords);
    lattice_relation_outputs o{};
    o.in_rows = i32(r.in_rows);
    o.out_rows = i32(r.out_rows);
    o.kernel_ids = i32(r.kernel_ids);
    o.row_offsets = i32(r.output_row_offsets);
    o.out_coords = i32(r.out_coords);
    o.counts = i32(r.counts);
    if (with_views) {
        o.in_row_offsets = i32(r.in_row_offsets);
        o.in_edge_ids = i32(r.in_edge_ids);
        o.kernel_row_offsets = i32(r.kernel_row_offsets);
        o.kernel_edge_ids = i32(r.kernel_edge_ids);
    }
    o.status = i32(status);
    at::Tensor ws = workspace(lattice_hip_expanded_relation_workspace_bytes(rows, kernel_size.data(), stride.data(),
                                                                           dilation.data(), generative ? 1 : 0),
                              coords);
    if (generative) {
        check_status(lattice_hip_build_generative_relation(ci32(coords), rows, ci32(active_rows), kernel_size.data(),
                                                           stride.data(), &o, ws.data_ptr(),
                                                           static_cast<size_t>(ws.numel()), current_stream(coords)));
    } else {
        check_status(lattice_hip_build_transposed_kernel_relation(
            ci32(coords), rows, ci32(active_rows), kernel_size.data(), stride.data(), padding.data(),
            dilation.data(), &o, ws.data_ptr(), static_cast<size_t>(ws.numel()), current_stream(coords)));
    }
    r.status = status;
    return r;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> make_relation_grouped_views(
    const at::Tensor& in_rows_in, const at::Tensor& kernel_ids_in, const at::Tensor& counts, int in_capacity,
    int kernel_count) {
    if (in_rows_in.dim() != 1 || kernel_ids_in.dim() != 1 || in_rows_in.scalar_type() != at::kInt ||
        kernel_ids_in.scalar_type() != at::kInt || in_rows_in.size(0) != kernel_ids_in.size(0)) {
        throw std::invalid_argument("relation rows and kernel_ids must be equal-length int32 arrays.");
    }
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("relation counts must have shape (2,) and int32 dtype.");
    }
    if (in_capacity < 0 || kernel_count <= 0) {
        throw std::invalid_argument("grouped views need a non-negative input capacity and positive n_kernels.");
    }
    require_on_device({{&in_rows_in, "in_rows"}, {&kernel_ids_in, "kernel_ids"}, {&counts, "counts"}});
    const at::Tensor in_rows = in_rows_in.contiguous();
    const at::Tensor kernel_ids = kernel_ids_in.contiguous();
    const int edges = static_cast<int>(in_rows.size(0));
    at::Tensor in_offsets = empty_i32({in_capacity + 1}, in_rows);
    at::Tensor in_ids = empty_i32({edges}, in_rows);
    at::Tensor k_offsets = empty_i32({kernel_count + 1}, in_rows);
    at::Tensor k_ids = empty_i32({edges}, in_rows);
    at::Tensor ws = workspace(lattice_hip_relation_grouped_views_workspace_bytes(edges), in_rows);
    check_status(lattice_hip_build_relation_grouped_views(
        ci32(in_rows), ci32(kernel_ids), ci32(counts), edges, in_capacity, kernel_count, i32(in_offsets),
        i32(in_ids), i32(k_offsets), i32(k_ids), ws.data_ptr(), static_cast<size_t>(ws.numel()),
        current_stream(in_rows)));
    return {in_offsets, in_ids, k_offsets, k_ids};
}

std::tuple<at::Tensor, at::Tensor> make_relation_implicit_gemm_view(
    const at::Tensor& source_in, const at::Tensor& source_active_rows, const at::Tensor& output_in,
    const at::Tensor& output_active_rows, const at::Tensor& offsets_in, Triple stride, Triple padding) {
    validate_coords(source_in, "source_coords");
    validate_coords(output_in, "output_coords");
    validate_active_rows(source_active_rows);
    validate_active_rows(output_active_rows);
    if (offsets_in.dim() != 2 || offsets_in.size(1) != 3 || offsets_in.scalar_type() != at::kInt) {
        throw std::invalid_argument("offsets must have shape (K, 3) and int32 dtype.");
    }
    validate_positive(stride, "stride");
    validate_nonnegative(padding, "padding");
    require_on_device({{&source_in, "source_coords"},
                       {&source_active_rows, "source_active_rows"},
                       {&output_in, "output_coords"},
                       {&output_active_rows, "output_active_rows"}});
    const at::Tensor source = source_in.contiguous();
    const at::Tensor output = output_in.contiguous();
    const at::Tensor offsets = offsets_in.to(source.device()).contiguous();
    const int source_rows = static_cast<int>(source.size(0));
    const int output_rows = static_cast<int>(output.size(0));
    const int K = static_cast<int>(offsets.size(0));
    if (K <= 0) throw std::invalid_argument("offsets must have shape (K, 3) with K > 0.");
    at::Tensor out_in_map = empty_i32({output_rows, K}, source);
    at::Tensor row_masks = empty_i32({output_rows, (K + 31) / 32}, source);
    at::Tensor status = empty_i32({1}, source);
    at::Tensor ws = workspace(lattice_hip_implicit_gemm_view_workspace_bytes(source_rows), source);
    check_status(lattice_hip_build_relation_implicit_gemm_view(
        ci32(source), source_rows, ci32(source_active_rows), ci32(output), output_rows,
        ci32(output_active_rows), ci32(offsets), K, stride.data(), padding.data(), i32(out_in_map),
        i32(row_masks), i32(status), ws.data_ptr(), static_cast<size_t>(ws.numel()), current_stream(source)));
    return {out_in_map, row_masks};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> make_sorted_implicit_gemm_view(
    const at::Tensor& out_in_map_in, const at::Tensor& row_masks_in) {
    if (out_in_map_in.dim() != 2 || out_in_map_in.scalar_type() != at::kInt) {
        throw std::invalid_argument("out_in_map must have shape (Nout, K) and int32 dtype.");
    }
    if (row_masks_in.dim() != 2 || row_masks_in.scalar_type() != at::kInt ||
        row_masks_in.size(0) != out_in_map_in.size(0)) {
        throw std::invalid_argument("row_masks must have one row per out_in_map row.");
    }
    if (row_masks_in.size(1) != 1) {
        throw std::invalid_argument("sorted implicit GEMM view currently supports K <= 32.");
    }
    require_device(out_in_map_in, "out_in_map");
    const at::Tensor map = out_in_map_in.contiguous();
    const at::Tensor masks = row_masks_in.contiguous();
    const int rows = static_cast<int>(map.size(0));
    const int K = static_cast<int>(map.size(1));
    at::Tensor reorder = empty_i32({rows}, map);
    at::Tensor kv = empty_i32({K, rows}, map);
    at::Tensor tiles = empty_i32({((rows + 63) / 64) * 4}, map);
    at::Tensor ws = workspace(lattice_hip_sorted_view_workspace_bytes(rows), map);
    check_status(lattice_hip_build_sorted_implicit_gemm_view(ci32(map), ci32(masks), rows, K, i32(reorder),
                                                             nullptr, i32(kv), i32(tiles), ws.data_ptr(),
                                                             static_cast<size_t>(ws.numel()), current_stream(map)));
    // The row-major sorted map is the transpose of the K-major one: it is
    // returned as that (non-contiguous) view and copied only by a consumer
    // that needs contiguous rows, the way the reference's lazy graph leaves
    // an unused output unevaluated.
    return {reorder, kv.t(), kv, tiles};
}

}  // namespace lattice_native
