// Point -> voxel quantization over torch device tensors (the reference's
// native/features/coordinates/quantization.cpp and its bindings): validation,
// output allocation on the current stream, then the C-ABI call.
#pragma once

#include <torch/extension.h>

#include <optional>
#include <string>
#include <tuple>
#include <vector>

namespace lattice_native {

// (coords [N, 4], active_rows [1], inverse_rows [N], counts [N]); raises when
// a voxel coordinate does not fit the packed key (one host read).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> sparse_quantize(
    const at::Tensor& points, const at::Tensor& batch_indices, const at::Tensor& active_rows,
    const std::vector<float>& voxel_size, const std::vector<float>& origin);

// Stable grouping of keys by value: (offsets [groups + 1], ids [n]); keys
// outside [0, groups) and positions at or past *count are left out.
std::tuple<at::Tensor, at::Tensor> group_by_key(const at::Tensor& keys, const std::optional<at::Tensor>& count,
                                                int groups);

at::Tensor voxelize_features(const at::Tensor& feats, const at::Tensor& inverse_rows, const at::Tensor& counts,
                             const at::Tensor& active_rows, const std::string& reduction);
at::Tensor voxelize_features_grouped(const at::Tensor& feats, const at::Tensor& counts,
                                     const at::Tensor& voxel_offsets, const at::Tensor& point_ids,
                                     const std::string& reduction);
at::Tensor voxelize_features_grad(const at::Tensor& cotangent, const at::Tensor& inverse_rows,
                                  const at::Tensor& counts, const at::Tensor& active_rows, int point_rows,
                                  const std::string& reduction);

// (rows [N, 8] int32, weights [N, 8] float32)
std::tuple<at::Tensor, at::Tensor> build_point_voxel_map(
    const at::Tensor& points, const at::Tensor& batch_indices, const at::Tensor& point_active_rows,
    const at::Tensor& voxel_coords, const at::Tensor& voxel_active_rows, const std::vector<float>& voxel_size,
    const std::vector<float>& origin, const std::string& interpolation);
at::Tensor interpolate_point_features(const at::Tensor& voxel_feats, const at::Tensor& rows,
                                      const at::Tensor& weights);
at::Tensor interpolate_point_features_grad(const at::Tensor& point_grad, const at::Tensor& weights,
                                           const at::Tensor& voxel_offsets, const at::Tensor& entry_ids,
                                           int voxel_rows);

}  // namespace lattice_native
