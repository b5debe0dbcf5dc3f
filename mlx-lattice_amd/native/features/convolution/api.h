// Sparse convolution feature entry points over torch device tensors.
// Mirrors native/features/convolution/api.cpp:119-313 and quantized.cpp:
// 57-268 of the reference: same argument order, validation messages and
// static output capacity (out_capacity, C_out).
#pragma once

#include <torch/extension.h>

#include <optional>

namespace lattice_native {

at::Tensor sparse_conv_features(const at::Tensor& feats, const at::Tensor& weights, const at::Tensor& in_rows,
                                const at::Tensor& out_rows, const at::Tensor& kernel_ids, const at::Tensor& counts,
                                const at::Tensor& row_offsets, const at::Tensor& in_row_offsets,
                                const at::Tensor& in_edge_ids, const at::Tensor& kernel_row_offsets,
                                const at::Tensor& kernel_edge_ids, int out_capacity, int n_kernels,
                                const std::optional<at::Tensor>& bias = std::nullopt, bool relu = false);

// The CSR conv without the grouped plan views the reference signature
// carries for its gradient (the forward reads only the output CSR).  With
// the relation's dense map (out_in_map, (out_capacity, n_kernels)) and a
// shape the dense-map conv takes (C_in 4 or 8), it runs that instead.
at::Tensor sparse_conv_features_csr(const at::Tensor& feats, const at::Tensor& weights, const at::Tensor& in_rows,
                                    const at::Tensor& kernel_ids, const at::Tensor& counts,
                                    const at::Tensor& row_offsets, int out_capacity, int n_kernels,
                                    const std::optional<at::Tensor>& bias = std::nullopt, bool relu = false,
                                    const std::optional<at::Tensor>& out_in_map = std::nullopt);

// Dense expansion conv over a direct generative / transposed relation:
// (rows * K, C_out), output row in * K + k = feats[in] @ W[k].
at::Tensor sparse_conv_features_expand(const at::Tensor& feats, const at::Tensor& weights,
                                       const at::Tensor& active_rows, int n_kernels,
                                       const std::optional<at::Tensor>& bias = std::nullopt, bool relu = false);

at::Tensor sparse_conv_features_sorted_implicit_gemm(const at::Tensor& feats, const at::Tensor& weights,
                                                     const at::Tensor& sorted_out_in_map,
                                                     const at::Tensor& sorted_kv_out_in_map,
                                                     const at::Tensor& reorder_rows, const at::Tensor& tile_masks,
                                                     int out_capacity, int n_kernels, bool store_sorted,
                                                     const std::optional<at::Tensor>& bias = std::nullopt,
                                                     const std::optional<at::Tensor>& tile_order = std::nullopt,
                                                     bool relu = false,
                                                     const std::optional<at::Tensor>& weight_fragments = std::nullopt);

// The fragment-ordered copy of a 5D fp16/bf16 weight that the streamed
// matrix-core conv reads (lattice_hip_conv_weight_fragments), kept with the
// weight and passed back as `weight_fragments`; an empty tensor when the
// weight's shape does not take that route.
at::Tensor conv_weight_fragments(const at::Tensor& weights);

at::Tensor sparse_quantized_conv_features(const at::Tensor& feats, const at::Tensor& weights,
                                          const at::Tensor& scales, const at::Tensor& biases,
                                          const at::Tensor& in_rows, const at::Tensor& out_rows,
                                          const at::Tensor& kernel_ids, const at::Tensor& counts,
                                          const at::Tensor& row_offsets, const at::Tensor& sorted_kv_out_in_map,
                                          const at::Tensor& reorder_rows, const at::Tensor& tile_masks,
                                          int out_capacity, int n_kernels, int in_channels, int out_channels,
                                          int storage_in_channels, int group_size, int bits,
                                          const std::optional<at::Tensor>& bias = std::nullopt,
                                          const std::optional<at::Tensor>& tile_order = std::nullopt,
                                          bool relu = false,
                                          const std::optional<at::Tensor>& weight_fragments = std::nullopt,
                                          const std::optional<at::Tensor>& out_in_map = std::nullopt);

// The fragment-ordered packed copy of a quantized weight that the streamed
// matrix-core conv reads (lattice_hip_quantized_weight_fragments: codes,
// scale and bias of each lane's 8 input channels in one 16-byte piece),
// kept with the weight and passed back as `weight_fragments`; an empty
// tensor when the shape does not take that route.
at::Tensor quantized_weight_fragments(const at::Tensor& weights, const at::Tensor& scales,
                                      const at::Tensor& biases, int in_channels, int out_channels,
                                      int storage_in_channels, int group_size, int bits);

// Longest-first order of the 128-row tiles of a sorted view
// (lattice_hip_conv_tile_order), kept with the view and passed back as
// `tile_order` so the conv skips its per-call schedule.
at::Tensor conv_tile_order(const at::Tensor& tile_masks, int out_capacity);

// Gradients (the reference conv primitive's vjp, primitive.cpp:137-176):
// input gradient over the input-grouped CSR, (in_capacity, C_in) in the
// cotangent dtype.
at::Tensor sparse_conv_input_grad(const at::Tensor& cot, const at::Tensor& weights, const at::Tensor& out_rows,
                                  const at::Tensor& kernel_ids, const at::Tensor& counts,
                                  const at::Tensor& in_row_offsets, const at::Tensor& in_edge_ids, int in_capacity,
                                  int n_kernels);

// Transposed dense map (in_out_map (in_capacity, K), row_masks, status) of
// a forward or submanifold relation, for the matrix-core input gradient;
// status (1,) gets LATTICE_STATUS_REPEATED_PAIR when the map is incomplete.
std::tuple<at::Tensor, at::Tensor, at::Tensor> build_transposed_implicit_gemm_map(const at::Tensor& in_rows,
                                                                      const at::Tensor& out_rows,
                                                                      const at::Tensor& kernel_ids,
                                                                      const at::Tensor& counts, int in_capacity,
                                                                      int n_kernels);

// Weight gradient over the kernel-grouped CSR, in the shape and layout of
// `weights` (5D or mapped) and the cotangent dtype.
at::Tensor sparse_conv_weight_grad(const at::Tensor& feats, const at::Tensor& cot, const at::Tensor& weights,
                                   const at::Tensor& in_rows, const at::Tensor& out_rows, const at::Tensor& counts,
                                   const at::Tensor& kernel_row_offsets, const at::Tensor& kernel_edge_ids,
                                   int n_kernels);

}  // namespace lattice_native
