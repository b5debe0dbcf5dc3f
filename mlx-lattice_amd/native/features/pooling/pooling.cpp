#include "features/pooling/api.h"

#include <stdexcept>

#include "foundation/runtime.h"

namespace lattice_native {

namespace {

int reduce_code(const std::string& reduce, const char* message) {
    if (reduce == "sum") return 0;
    if (reduce == "max") return 1;
    if (reduce == "avg") return 2;
    throw std::invalid_argument(message);
}

void validate_relation(const at::Tensor& in_rows, const at::Tensor& out_rows, const at::Tensor& kernel_ids,
                       const at::Tensor& row_offsets, const at::Tensor& counts) {
    if (in_rows.dim() != 1 || out_rows.dim() != 1 || kernel_ids.dim() != 1) {
        throw std::invalid_argument("relation rows and kernel_ids must be one-dimensional.");
    }
    if (in_rows.scalar_type() != at::kInt || out_rows.scalar_type() != at::kInt ||
        kernel_ids.scalar_type() != at::kInt) {
        throw std::invalid_argument("relation rows and kernel_ids must use int32 dtype.");
    }
    if (in_rows.size(0) != out_rows.size(0) || in_rows.size(0) != kernel_ids.size(0)) {
        throw std::invalid_argument("relation row arrays and kernel_ids must have equal capacity.");
    }
    if (row_offsets.dim() != 1 || row_offsets.scalar_type() != at::kInt) {
        throw std::invalid_argument("row_offsets must have shape (N_out + 1,) and int32 dtype.");
    }
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("counts must have shape (2,) and int32 dtype.");
    }
}

}  // namespace

at::Tensor sparse_pool_features(const at::Tensor& feats_in, const at::Tensor& in_rows, const at::Tensor& out_rows,
                                const at::Tensor& kernel_ids, const at::Tensor& row_offsets,
                                const at::Tensor& counts, bool /*input_exclusive*/, const std::string& reduce,
                                int out_capacity, int n_kernels) {
    const int mode = reduce_code(reduce, "reduce must be 'sum', 'max', or 'avg'.");
    if (feats_in.dim() != 2) throw std::invalid_argument("feats must have shape (N, C).");
    if (feats_in.scalar_type() != at::kFloat) {
        throw std::invalid_argument("sparse_pool_features currently supports float32 feats.");
    }
    validate_relation(in_rows, out_rows, kernel_ids, row_offsets, counts);
    if (out_capacity < 0 || n_kernels <= 0) {
        throw std::invalid_argument("out_capacity must be nonnegative and n_kernels must be positive.");
    }
    if (row_offsets.size(0) != out_capacity + 1) {
        throw std::invalid_argument("row_offsets length must match out_capacity + 1.");
    }
    require_device(feats_in, "feats");
    const at::Tensor feats = feats_in.contiguous();
    at::Tensor out = at::empty({out_capacity, feats.size(1)}, feats.options());
    check_status(lattice_hip_sparse_pool_features(
        mode, feats.data_ptr<float>(), static_cast<int>(feats.size(0)), static_cast<int>(feats.size(1)),
        ci32(in_rows), static_cast<int>(in_rows.size(0)), ci32(row_offsets), ci32(counts), out_capacity,
        out.data_ptr<float>(), current_stream(feats)));
    return out;
}

at::Tensor sparse_pool_features_grad(const at::Tensor& cot_in, const at::Tensor& feats_in,
                                     const at::Tensor& pooled_in, const at::Tensor& in_rows,
                                     const at::Tensor& out_rows, const at::Tensor& row_offsets,
                                     const at::Tensor& counts, const at::Tensor& in_row_offsets,
                                     const at::Tensor& in_edge_ids, const std::string& reduce) {
    const int mode = reduce_code(reduce, "reduce must be 'sum', 'max', or 'avg'.");
    if (feats_in.dim() != 2 || cot_in.dim() != 2 || pooled_in.dim() != 2) {
        throw std::invalid_argument("feats, pooled and cotangent must have shape (N, C).");
    }
    if (feats_in.scalar_type() != at::kFloat || cot_in.scalar_type() != at::kFloat ||
        pooled_in.scalar_type() != at::kFloat) {
        throw std::invalid_argument("sparse_pool_features currently supports float32 feats.");
    }
    if (cot_in.sizes() != pooled_in.sizes() || cot_in.size(1) != feats_in.size(1)) {
        throw std::invalid_argument("cotangent must match the pooled output shape.");
    }
    validate_relation(in_rows, out_rows, out_rows, row_offsets, counts);
    if (row_offsets.size(0) != cot_in.size(0) + 1) {
        throw std::invalid_argument("row_offsets length must match out_capacity + 1.");
    }
    if (in_row_offsets.dim() != 1 || in_row_offsets.scalar_type() != at::kInt ||
        in_row_offsets.size(0) != feats_in.size(0) + 1) {
        throw std::invalid_argument("in_row_offsets length must match input capacity + 1.");
    }
    if (in_edge_ids.dim() != 1 || in_edge_ids.scalar_type() != at::kInt || in_edge_ids.size(0) != in_rows.size(0)) {
        throw std::invalid_argument("plan edge_ids must match relation edge capacity.");
    }
    require_device(feats_in, "feats");
    const at::Tensor cot = cot_in.contiguous();
    const at::Tensor feats = feats_in.contiguous();
    const at::Tensor pooled = pooled_in.contiguous();
    at::Tensor grad = at::empty(feats.sizes(), feats.options());
    check_status(lattice_hip_sparse_pool_features_grad(
        mode, cot.data_ptr<float>(), feats.data_ptr<float>(), pooled.data_ptr<float>(),
        static_cast<int>(feats.size(0)), static_cast<int>(feats.size(1)), ci32(in_rows), ci32(out_rows),
        static_cast<int>(in_rows.size(0)), ci32(row_offsets), ci32(counts), ci32(in_row_offsets), ci32(in_edge_ids),
        static_cast<int>(cot.size(0)), grad.data_ptr<float>(), current_stream(feats)));
    return grad;
}

at::Tensor global_pool(const at::Tensor& feats_in, const std::vector<int64_t>& batch_counts,
                       const std::string& mode) {
    const int code = reduce_code(mode, "mode must be 'sum', 'max', or 'avg'.");
    if (feats_in.dim() != 2) throw std::invalid_argument("feats must have shape (N, C).");
    if (feats_in.scalar_type() != at::kFloat) {
        throw std::invalid_argument("pooling currently supports float32 tensors.");
    }
    require_device(feats_in, "feats");
    std::vector<int64_t> offsets(batch_counts.size() + 1, 0);
    for (size_t b = 0; b < batch_counts.size(); ++b) {
        if (batch_counts[b] < 0) throw std::invalid_argument("batch_counts must be non-negative.");
        if (code == 1 && batch_counts[b] == 0) {
            throw std::invalid_argument("global_max_pool does not support empty batches.");
        }
        offsets[b + 1] = offsets[b] + batch_counts[b];
    }
    if (offsets.back() > feats_in.size(0)) throw std::invalid_argument("batch_counts must cover all sparse rows.");
    const at::Tensor feats = feats_in.contiguous();
    at::Tensor dev_offsets =
        at::tensor(offsets, at::TensorOptions().dtype(at::kLong)).to(feats.device(), /*non_blocking=*/false);
    at::Tensor out = at::empty({static_cast<int64_t>(batch_counts.size()), feats.size(1)}, feats.options());
    check_status(lattice_hip_global_pool(code, feats.data_ptr<float>(), static_cast<int>(feats.size(1)),
                                         dev_offsets.data_ptr<int64_t>(), static_cast<int>(batch_counts.size()),
                                         out.data_ptr<float>(), current_stream(feats)));
    return out;
}

}  // namespace lattice_native
