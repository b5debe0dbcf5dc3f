#include "features/quantization/api.h"

#include <stdexcept>

#include "foundation/runtime.h"

namespace lattice_native {

namespace {

std::array<float, 3> float_triple(const std::vector<float>& v, const char* name) {
    if (v.size() == 1) return {v[0], v[0], v[0]};
    if (v.size() != 3) throw std::invalid_argument(std::string(name) + " must contain exactly 3 values.");
    return {v[0], v[1], v[2]};
}

void validate_points(const at::Tensor& points) {
    if (points.dim() != 2 || points.size(1) != 3) throw std::invalid_argument("points must have shape (N, 3).");
    if (points.scalar_type() != at::kFloat) throw std::invalid_argument("points must be float32.");
}

void validate_active(const at::Tensor& t, const char* name) {
    if (t.dim() != 1 || t.size(0) != 1 || t.scalar_type() != at::kInt) {
        throw std::invalid_argument(std::string(name) + " must have shape (1,) and int32 dtype.");
    }
}

void validate_batches(const at::Tensor& b, int64_t rows) {
    if (b.dim() != 1 || b.size(0) != rows || b.scalar_type() != at::kInt) {
        throw std::invalid_argument("batch_indices must have shape (N,) and int32 dtype.");
    }
}

void validate_float_feats(const at::Tensor& t, const char* message) {
    if (t.dim() != 2) throw std::invalid_argument("feats must have shape (N, C).");
    if (t.scalar_type() != at::kFloat) throw std::invalid_argument(message);
}

void validate_i32_vector(const at::Tensor& t, const char* message) {
    if (t.dim() != 1 || t.scalar_type() != at::kInt) throw std::invalid_argument(message);
}

int reduction_code(const std::string& r) {
    if (r == "sum") return 0;
    if (r == "mean") return 1;
    throw std::invalid_argument("reduction must be 'sum' or 'mean'.");
}

}  // namespace

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> sparse_quantize(
    const at::Tensor& points_in, const at::Tensor& batches_in, const at::Tensor& active_rows,
    const std::vector<float>& voxel_size, const std::vector<float>& origin) {
    validate_points(points_in);
    const int64_t rows = points_in.size(0);
    validate_batches(batches_in, rows);
    validate_active(active_rows, "active_rows");
    const auto size = float_triple(voxel_size, "voxel_size");
    const auto org = float_triple(origin, "origin");
    for (float s : size) {
        if (!(s > 0.0f)) throw std::invalid_argument("voxel_size values must be positive.");
    }
    require_device(points_in, "points");
    require_device(batches_in, "batch_indices");
    require_device(active_rows, "active_rows");
    const at::Tensor points = points_in.contiguous();
    const at::Tensor batches = batches_in.contiguous();
    const int n = static_cast<int>(rows);
    at::Tensor coords = empty_i32({rows, 4}, points);
    at::Tensor count = empty_i32({1}, points);
    at::Tensor inverse = empty_i32({rows}, points);
    at::Tensor counts = empty_i32({rows}, points);
    at::Tensor status = empty_i32({1}, points);
    at::Tensor ws = workspace(lattice_hip_sparse_quantize_workspace_bytes(n), points);
    check_status(lattice_hip_sparse_quantize(points.data_ptr<float>(), ci32(batches), n, ci32(active_rows),
                                             size.data(), org.data(), i32(coords), i32(count), i32(inverse),
                                             i32(counts), i32(status), ws.data_ptr(),
                                             static_cast<size_t>(ws.numel()), current_stream(points)));
    return {coords, count, inverse, counts};
}

std::tuple<at::Tensor, at::Tensor> group_by_key(const at::Tensor& keys_in, const std::optional<at::Tensor>& count,
                                                int groups) {
    validate_i32_vector(keys_in, "keys must be a one-dimensional int32 array.");
    if (groups < 0) throw std::invalid_argument("groups must be non-negative.");
    require_device(keys_in, "keys");
    const at::Tensor keys = keys_in.contiguous();
    const int n = static_cast<int>(keys.size(0));
    const int32_t* count_ptr = nullptr;
    if (count.has_value() && count->defined()) {
        validate_active(*count, "count");
        require_device(*count, "count");
        count_ptr = ci32(*count);
    }
    at::Tensor offsets = empty_i32({groups + 1}, keys);
    at::Tensor ids = empty_i32({n}, keys);
    at::Tensor ws = workspace(lattice_hip_group_by_key_workspace_bytes(n), keys);
    check_status(lattice_hip_group_by_key(ci32(keys), n, count_ptr, groups, i32(offsets), i32(ids), ws.data_ptr(),
                                          static_cast<size_t>(ws.numel()), current_stream(keys)));
    return {offsets, ids};
}

at::Tensor voxelize_features_grouped(const at::Tensor& feats_in, const at::Tensor& counts,
                                     const at::Tensor& voxel_offsets, const at::Tensor& point_ids,
                                     const std::string& reduction) {
    const int mode = reduction_code(reduction);
    validate_float_feats(feats_in, "voxelize currently supports float32 features.");
    validate_i32_vector(counts, "counts must be a one-dimensional int32 array.");
    validate_i32_vector(voxel_offsets, "voxel_offsets must be a one-dimensional int32 array.");
    validate_i32_vector(point_ids, "point_ids must be a one-dimensional int32 array.");
    if (voxel_offsets.size(0) != counts.size(0) + 1) {
        throw std::invalid_argument("voxel_offsets must have one entry per voxel plus one.");
    }
    require_device(feats_in, "feats");
    const at::Tensor feats = feats_in.contiguous();
    const int voxel_rows = static_cast<int>(counts.size(0));
    at::Tensor out = at::empty({voxel_rows, feats.size(1)}, feats.options());
    check_status(lattice_hip_voxelize_features(mode, feats.data_ptr<float>(), static_cast<int>(feats.size(1)),
                                               ci32(counts), voxel_rows, ci32(voxel_offsets), ci32(point_ids),
                                               out.data_ptr<float>(), current_stream(feats)));
    return out;
}

at::Tensor voxelize_features(const at::Tensor& feats, const at::Tensor& inverse_rows, const at::Tensor& counts,
                             const at::Tensor& active_rows, const std::string& reduction) {
    reduction_code(reduction);
    validate_float_feats(feats, "voxelize currently supports float32 features.");
    validate_i32_vector(inverse_rows, "inverse_rows must be a one-dimensional int32 array.");
    validate_i32_vector(counts, "counts must be a one-dimensional int32 array.");
    validate_active(active_rows, "active_rows");
    if (feats.size(0) != inverse_rows.size(0)) {
        throw std::invalid_argument("feats and quantization metadata must share rows.");
    }
    auto [offsets, ids] = group_by_key(inverse_rows, active_rows, static_cast<int>(counts.size(0)));
    return voxelize_features_grouped(feats, counts, offsets, ids, reduction);
}

at::Tensor voxelize_features_grad(const at::Tensor& cot_in, const at::Tensor& inverse_rows, const at::Tensor& counts,
                                  const at::Tensor& active_rows, int point_rows, const std::string& reduction) {
    const int mode = reduction_code(reduction);
    validate_float_feats(cot_in, "voxelize currently supports float32 features.");
    validate_i32_vector(inverse_rows, "inverse_rows must be a one-dimensional int32 array.");
    validate_i32_vector(counts, "counts must be a one-dimensional int32 array.");
    validate_active(active_rows, "active_rows");
    if (inverse_rows.size(0) != point_rows) throw std::invalid_argument("inverse_rows must have one entry per point.");
    if (cot_in.size(0) != counts.size(0)) throw std::invalid_argument("cotangent must have one row per voxel.");
    require_device(cot_in, "cotangent");
    const at::Tensor cot = cot_in.contiguous();
    at::Tensor grad = at::empty({point_rows, cot.size(1)}, cot.options());
    check_status(lattice_hip_voxelize_features_grad(mode, cot.data_ptr<float>(), static_cast<int>(cot.size(0)),
                                                    static_cast<int>(cot.size(1)), ci32(inverse_rows), ci32(counts),
                                                    point_rows, ci32(active_rows), grad.data_ptr<float>(),
                                                    current_stream(cot)));
    return grad;
}

std::tuple<at::Tensor, at::Tensor> build_point_voxel_map(
    const at::Tensor& points_in, const at::Tensor& batches_in, const at::Tensor& point_active_rows,
    const at::Tensor& voxel_coords_in, const at::Tensor& voxel_active_rows, const std::vector<float>& voxel_size,
    const std::vector<float>& origin, const std::string& interpolation) {
    int mode;
    if (interpolation == "nearest") {
        mode = 0;
    } else if (interpolation == "linear") {
        mode = 1;
    } else {
        throw std::invalid_argument("interpolation must be 'nearest' or 'linear'.");
    }
    validate_points(points_in);
    const int64_t rows = points_in.size(0);
    validate_batches(batches_in, rows);
    validate_active(point_active_rows, "point_active_rows");
    validate_active(voxel_active_rows, "voxel_active_rows");
    if (voxel_coords_in.dim() != 2 || voxel_coords_in.size(1) != 4 || voxel_coords_in.scalar_type() != at::kInt) {
        throw std::invalid_argument("voxel_coords must have shape (N, 4) and int32 dtype.");
    }
    const auto size = float_triple(voxel_size, "voxel_size");
    const auto org = float_triple(origin, "origin");
    for (float s : size) {
        if (!(s > 0.0f)) throw std::invalid_argument("voxel_size values must be positive.");
    }
    require_device(points_in, "points");
    require_device(voxel_coords_in, "voxel_coords");
    const at::Tensor points = points_in.contiguous();
    const at::Tensor batches = batches_in.contiguous();
    const at::Tensor voxels = voxel_coords_in.contiguous();
    const int voxel_rows = static_cast<int>(voxels.size(0));
    at::Tensor out_rows = empty_i32({rows, 8}, points);
    at::Tensor weights = at::empty({rows, 8}, points.options());
    at::Tensor status = empty_i32({1}, points);
    at::Tensor ws = workspace(lattice_hip_point_voxel_map_workspace_bytes(voxel_rows), points);
    check_status(lattice_hip_build_point_voxel_map(
        points.data_ptr<float>(), ci32(batches), static_cast<int>(rows), ci32(point_active_rows), ci32(voxels),
        voxel_rows, ci32(voxel_active_rows), size.data(), org.data(), mode, i32(out_rows),
        weights.data_ptr<float>(), i32(status), ws.data_ptr(), static_cast<size_t>(ws.numel()),
        current_stream(points)));
    return {out_rows, weights};
}

at::Tensor interpolate_point_features(const at::Tensor& values_in, const at::Tensor& rows, const at::Tensor& weights) {
    if (values_in.dim() != 2) throw std::invalid_argument("voxel_feats must have shape (N, C).");
    if (values_in.scalar_type() != at::kFloat) {
        throw std::invalid_argument("point interpolation currently supports float32.");
    }
    if (rows.dim() != 2 || rows.size(1) != 8 || rows.scalar_type() != at::kInt) {
        throw std::invalid_argument("rows must have shape (N, 8) and int32 dtype.");
    }
    if (weights.sizes() != rows.sizes() || weights.scalar_type() != at::kFloat) {
        throw std::invalid_argument("weights must have the same shape as rows and float32 dtype.");
    }
    require_device(values_in, "voxel_feats");
    const at::Tensor values = values_in.contiguous();
    const at::Tensor r = rows.contiguous();
    const at::Tensor w = weights.contiguous();
    at::Tensor out = at::empty({r.size(0), values.size(1)}, values.options());
    check_status(lattice_hip_interpolate_point_features(values.data_ptr<float>(), static_cast<int>(values.size(0)),
                                                        static_cast<int>(values.size(1)), ci32(r),
                                                        w.data_ptr<float>(), static_cast<int>(r.size(0)),
                                                        out.data_ptr<float>(), current_stream(values)));
    return out;
}

at::Tensor interpolate_point_features_grad(const at::Tensor& grad_in, const at::Tensor& weights,
                                           const at::Tensor& voxel_offsets, const at::Tensor& entry_ids,
                                           int voxel_rows) {
    validate_float_feats(grad_in, "point interpolation currently supports float32.");
    if (weights.dim() != 2 || weights.size(1) != 8 || weights.size(0) != grad_in.size(0) ||
        weights.scalar_type() != at::kFloat) {
        throw std::invalid_argument("weights must have shape (N, 8) and float32 dtype.");
    }
    validate_i32_vector(voxel_offsets, "voxel_offsets must be a one-dimensional int32 array.");
    validate_i32_vector(entry_ids, "entry_ids must be a one-dimensional int32 array.");
    if (voxel_offsets.size(0) != voxel_rows + 1) {
        throw std::invalid_argument("voxel_offsets must have one entry per voxel plus one.");
    }
    require_device(grad_in, "point_grad");
    const at::Tensor g = grad_in.contiguous();
    const at::Tensor w = weights.contiguous();
    at::Tensor out = at::empty({voxel_rows, g.size(1)}, g.options());
    check_status(lattice_hip_interpolate_point_features_grad(g.data_ptr<float>(), static_cast<int>(g.size(1)),
                                                             w.data_ptr<float>(), ci32(voxel_offsets),
                                                             ci32(entry_ids), voxel_rows, out.data_ptr<float>(),
                                                             current_stream(g)));
    return out;
}

}  // namespace lattice_native
