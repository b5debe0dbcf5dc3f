// Sparse convolution feature entry points over torch device tensors.
// Mirrors native/features/convolution/api.cpp:119-313 and quantized.cpp:
// 57-268 of the reference: same argument order, validation messages and
// static output capacity (out_capacity, C_out).
#pragma once

#include <torch/extension.h>

namespace lattice_native {

at::Tensor sparse_conv_features(const at::Tensor& feats, const at::Tensor& weights, const at::Tensor& in_rows,
                                const at::Tensor& out_rows, const at::Tensor& kernel_ids, const at::Tensor& counts,
                                const at::Tensor& row_offsets, const at::Tensor& in_row_offsets,
                                const at::Tensor& in_edge_ids, const at::Tensor& kernel_row_offsets,
                                const at::Tensor& kernel_edge_ids, int out_capacity, int n_kernels);

at::Tensor sparse_conv_features_sorted_implicit_gemm(const at::Tensor& feats, const at::Tensor& weights,
                                                     const at::Tensor& sorted_out_in_map,
                                                     const at::Tensor& sorted_kv_out_in_map,
                                                     const at::Tensor& reorder_rows, const at::Tensor& tile_masks,
                                                     int out_capacity, int n_kernels, bool store_sorted);

at::Tensor sparse_quantized_conv_features(const at::Tensor& feats, const at::Tensor& weights,
                                          const at::Tensor& scales, const at::Tensor& biases,
                                          const at::Tensor& in_rows, const at::Tensor& out_rows,
                                          const at::Tensor& kernel_ids, const at::Tensor& counts,
                                          const at::Tensor& row_offsets, const at::Tensor& sorted_kv_out_in_map,
                                          const at::Tensor& reorder_rows, const at::Tensor& tile_masks,
                                          int out_capacity, int n_kernels, int in_channels, int out_channels,
                                          int storage_in_channels, int group_size, int bits);

}  // namespace lattice_native
