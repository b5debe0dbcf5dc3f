// Sparse pooling entry points over torch device tensors.  Mirrors
// native/features/pooling/api.cpp and validation.cpp:8-62 of the reference
// (argument order of bindings/pooling.cpp:15-66, same validation messages).
#pragma once

#include <torch/extension.h>

#include <string>
#include <vector>

namespace lattice_native {

// reduce: "sum", "max" or "avg".  (out_capacity, C) float32.
at::Tensor sparse_pool_features(const at::Tensor& feats, const at::Tensor& in_rows, const at::Tensor& out_rows,
                                const at::Tensor& kernel_ids, const at::Tensor& row_offsets,
                                const at::Tensor& counts, bool input_exclusive, const std::string& reduce,
                                int out_capacity, int n_kernels);

// The pooling vjp over the input-grouped CSR: (N_in, C) float32.
at::Tensor sparse_pool_features_grad(const at::Tensor& cotangent, const at::Tensor& feats,
                                     const at::Tensor& pooled, const at::Tensor& in_rows,
                                     const at::Tensor& out_rows, const at::Tensor& row_offsets,
                                     const at::Tensor& counts, const at::Tensor& in_row_offsets,
                                     const at::Tensor& in_edge_ids, const std::string& reduce);

// Per-batch global pooling of rows grouped by batch_counts: (B, C) float32.
at::Tensor global_pool(const at::Tensor& feats, const std::vector<int64_t>& batch_counts, const std::string& mode);

}  // namespace lattice_native
