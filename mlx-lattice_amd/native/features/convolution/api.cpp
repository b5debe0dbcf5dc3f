#include "features/convolution/api.h"

#include <stdexcept>
#include <string>

#include "foundation/runtime.h"

namespace lattice_native {

namespace {

int dtype_code(const at::Tensor& t, const char* op) {
    switch (t.scalar_type()) {
    case at::kFloat: return LATTICE_F32;
    case at::kHalf: return LATTICE_F16;
    case at::kBFloat16: return LATTICE_BF16;
    default:
        throw std::invalid_argument(std::string(op) + " supports float32 and float16 feats.");
    }
}

void require_i32_vector(const at::Tensor& t, const char* message) {
    if (t.dim() != 1 || t.scalar_type() != at::kInt) throw std::invalid_argument(message);
}

// Optional fused bias: (C_out,) in the feature dtype on the same device, as
// the operator's _with_bias validates it (ops/conv.py:460-469).
const void* bias_ptr(const std::optional<at::Tensor>& bias, const at::Tensor& feats, int64_t c_out,
                     at::Tensor* keep) {
    if (!bias.has_value() || !bias->defined()) return nullptr;
    if (bias->dim() != 1) throw std::invalid_argument("bias must have shape (C_out,).");
    if (bias->size(0) != c_out) throw std::invalid_argument("bias channels must match output channels.");
    if (bias->scalar_type() != feats.scalar_type()) {
        throw std::invalid_argument("bias dtype must match output features.");
    }
    require_device(*bias, "bias");
    *keep = bias->contiguous();
    return keep->data_ptr();
}

void validate_weights(const at::Tensor& feats, const at::Tensor& weights, int n_kernels, const char* op) {
    if (feats.dim() != 2) throw std::invalid_argument("feats must have shape (N, C_in).");
    if (weights.dim() != 3 && weights.dim() != 5) {
        throw std::invalid_argument("weights must have shape (K, C_in, C_out) or (C_out, Kx, Ky, Kz, C_in).");
    }
    dtype_code(feats, op);
    if (weights.scalar_type() != feats.scalar_type()) {
        throw std::invalid_argument(std::string(op) + " weights must match feats dtype.");
    }
    const int64_t w_in = weights.dim() == 3 ? weights.size(1) : weights.size(4);
    if (feats.size(1) != w_in) throw std::invalid_argument("feats channels must match weights input channels.");
    if (n_kernels <= 0) {
        throw std::invalid_argument("out_capacity must be nonnegative and n_kernels must be positive.");
    }
    if (weights.dim() == 3 && weights.size(0) != n_kernels) {
        throw std::invalid_argument("weights kernel rows must match n_kernels.");
    }
    if (weights.dim() == 5 && weights.size(1) * weights.size(2) * weights.size(3) != n_kernels) {
        throw std::invalid_argument("weights kernel rows must match n_kernels.");
    }
    require_device(feats, "feats");
    require_device(weights, "weights");
}

int64_t out_channels_of(const at::Tensor& weights) { return weights.dim() == 3 ? weights.size(2) : weights.size(0); }

// The relation's dense map when the caller passed one and the dense-map
// conv takes the shape (few input channels); an undefined tensor otherwise.
at::Tensor dense_map_for(const std::optional<at::Tensor>& out_in_map, int dtype, const at::Tensor& feats, int c_in,
                         int c_out, int n_kernels, int out_capacity) {
    if (!out_in_map.has_value() || !out_in_map->defined() || out_in_map->numel() == 0) return {};
    if (lattice_hip_conv_dense_map_supported(dtype, c_in, c_out, n_kernels) == 0) return {};
    if (reinterpret_cast<uintptr_t>(feats.data_ptr()) % (static_cast<size_t>(c_in) * feats.element_size()) != 0) {
        return {};
    }
    const at::Tensor& m = *out_in_map;
    if (m.dim() != 2 || m.size(0) != out_capacity || m.size(1) != n_kernels || m.scalar_type() != at::kInt) {
        throw std::invalid_argument("out_in_map must have shape (out_capacity, n_kernels) and int32 dtype.");
    }
    require_device(m, "out_in_map");
    return m.contiguous();
}

}  // namespace

at::Tensor sparse_conv_features(const at::Tensor& feats_in, const at::Tensor& weights_in, const at::Tensor& in_rows,
                                const at::Tensor& out_rows, const at::Tensor& kernel_ids, const at::Tensor& counts,
                                const at::Tensor& row_offsets, const at::Tensor& in_row_offsets,
                                const at::Tensor& in_edge_ids, const at::Tensor& kernel_row_offsets,
                                const at::Tensor& kernel_edge_ids, int out_capacity, int n_kernels,
                                const std::optional<at::Tensor>& bias, bool relu) {
    const char* op = "sparse_conv_features";
    if (out_capacity < 0) {
        throw std::invalid_argument("out_capacity must be nonnegative and n_kernels must be positive.");
    }
    validate_weights(feats_in, weights_in, n_kernels, op);
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
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("counts must have shape (2,) and int32 dtype.");
    }
    require_i32_vector(row_offsets, "row_offsets must be a one-dimensional int32 array.");
    if (in_row_offsets.dim() != 1 || in_row_offsets.scalar_type() != at::kInt || kernel_row_offsets.dim() != 1 ||
        kernel_row_offsets.scalar_type() != at::kInt) {
        throw std::invalid_argument("plan row_offsets must be one-dimensional int32 arrays.");
    }
    if (in_edge_ids.dim() != 1 || kernel_edge_ids.dim() != 1 || in_edge_ids.scalar_type() != at::kInt ||
        kernel_edge_ids.scalar_type() != at::kInt) {
        throw std::invalid_argument("plan edge_ids must be one-dimensional int32 arrays.");
    }
    if (row_offsets.size(0) != out_capacity + 1) {
        throw std::invalid_argument("row_offsets length must match out_capacity + 1.");
    }
    if (in_row_offsets.size(0) != feats_in.size(0) + 1) {
        throw std::invalid_argument("in_row_offsets length must match input capacity + 1.");
    }
    if (kernel_row_offsets.size(0) != n_kernels + 1) {
        throw std::invalid_argument("kernel_row_offsets length must match n_kernels + 1.");
    }
    if (in_edge_ids.size(0) != in_rows.size(0) || kernel_edge_ids.size(0) != in_rows.size(0)) {
        throw std::invalid_argument("plan edge_ids must match relation edge capacity.");
    }
    const at::Tensor feats = feats_in.contiguous();
    const at::Tensor weights = weights_in.contiguous();
    const int64_t c_out = out_channels_of(weights);
    at::Tensor out = at::empty({out_capacity, c_out}, feats.options());
    const int layout = weights.dim() == 3 ? LATTICE_WEIGHT_KERNEL_MAJOR : LATTICE_WEIGHT_DENSE_5D;
    at::Tensor bias_keep;
    const void* b = bias_ptr(bias, feats, c_out, &bias_keep);
    check_status(lattice_hip_sparse_conv_features(
        dtype_code(feats, op), feats.data_ptr(), static_cast<int>(feats.size(0)), static_cast<int>(feats.size(1)),
        weights.data_ptr(), layout, n_kernels, static_cast<int>(c_out), ci32(in_rows), ci32(kernel_ids),
        ci32(counts), static_cast<int>(in_rows.size(0)), ci32(row_offsets), out_capacity, out.data_ptr(), b,
        relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, current_stream(feats)));
    return out;
}

at::Tensor sparse_conv_features_csr(const at::Tensor& feats_in, const at::Tensor& weights_in, const at::Tensor& in_rows,
                                    const at::Tensor& kernel_ids, const at::Tensor& counts,
                                    const at::Tensor& row_offsets, int out_capacity, int n_kernels,
                                    const std::optional<at::Tensor>& bias, bool relu,
                                    const std::optional<at::Tensor>& out_in_map) {
    const char* op = "sparse_conv_features";
    if (out_capacity < 0) {
        throw std::invalid_argument("out_capacity must be nonnegative and n_kernels must be positive.");
    }
    validate_weights(feats_in, weights_in, n_kernels, op);
    require_i32_vector(in_rows, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    require_i32_vector(kernel_ids, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    if (in_rows.size(0) != kernel_ids.size(0)) {
        throw std::invalid_argument("relation row arrays and kernel_ids must have equal capacity.");
    }
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("counts must have shape (2,) and int32 dtype.");
    }
    require_i32_vector(row_offsets, "row_offsets must be a one-dimensional int32 array.");
    if (row_offsets.size(0) != out_capacity + 1) {
        throw std::invalid_argument("row_offsets length must match out_capacity + 1.");
    }
    const at::Tensor feats = feats_in.contiguous();
    const at::Tensor weights = weights_in.contiguous();
    const int64_t c_out = out_channels_of(weights);
    at::Tensor out = at::empty({out_capacity, c_out}, feats.options());
    const int layout = weights.dim() == 3 ? LATTICE_WEIGHT_KERNEL_MAJOR : LATTICE_WEIGHT_DENSE_5D;
    at::Tensor bias_keep;
    const void* b = bias_ptr(bias, feats, c_out, &bias_keep);
    const at::Tensor map = dense_map_for(out_in_map, dtype_code(feats, op), feats, static_cast<int>(feats.size(1)),
                                         static_cast<int>(c_out), n_kernels, out_capacity);
    if (map.defined()) {
        check_status(lattice_hip_sparse_conv_features_dense_map(
            dtype_code(feats, op), feats.data_ptr(), static_cast<int>(feats.size(0)), static_cast<int>(feats.size(1)),
            weights.data_ptr(), layout, n_kernels, static_cast<int>(c_out), ci32(map), ci32(counts), out_capacity,
            out.data_ptr(), b, relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, current_stream(feats)));
        return out;
    }
    check_status(lattice_hip_sparse_conv_features(
        dtype_code(feats, op), feats.data_ptr(), static_cast<int>(feats.size(0)), static_cast<int>(feats.size(1)),
        weights.data_ptr(), layout, n_kernels, static_cast<int>(c_out), ci32(in_rows), ci32(kernel_ids),
        ci32(counts), static_cast<int>(in_rows.size(0)), ci32(row_offsets), out_capacity, out.data_ptr(), b,
        relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, current_stream(feats)));
    return out;
}

at::Tensor sparse_conv_features_expand(const at::Tensor& feats_in, const at::Tensor& weights_in,
                                       const at::Tensor& active_rows, int n_kernels,
                                       const std::optional<at::Tensor>& bias, bool relu) {
    const char* op = "sparse_conv_features_expand";
    validate_weights(feats_in, weights_in, n_kernels, op);
    if (active_rows.dim() != 1 || active_rows.size(0) != 1 || active_rows.scalar_type() != at::kInt) {
        throw std::invalid_argument("active_rows must have shape (1,) and int32 dtype.");
    }
    require_device(active_rows, "active_rows");
    const at::Tensor feats = feats_in.contiguous();
    const at::Tensor weights =
        weights_in.dim() == 5 ? weights_in.contiguous() : weights_in.permute({2, 0, 1}).contiguous();
    const int64_t c_out = out_channels_of(weights_in);
    const int64_t rows = feats.size(0);
    at::Tensor out = at::empty({rows * n_kernels, c_out}, feats.options());
    at::Tensor bias_keep;
    const void* b = bias_ptr(bias, feats, c_out, &bias_keep);
    check_status(lattice_hip_sparse_conv_features_expand(
        dtype_code(feats, op), feats.data_ptr(), static_cast<int>(rows), ci32(active_rows),
        static_cast<int>(feats.size(1)), weights.data_ptr(), n_kernels, static_cast<int>(c_out), out.data_ptr(), b,
        relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, current_stream(feats)));
    return out;
}

// The matrix-core conv's tile schedule: the caller's precomputed order
// (conv_tile_order, flagged LATTICE_CONV_ORDER_READY), or a fresh workspace
// the conv fills itself.
at::Tensor schedule_workspace(const std::optional<at::Tensor>& tile_order, int out_capacity, const at::Tensor& like,
                              size_t* bytes) {
    const size_t need = lattice_hip_conv_workspace_bytes(out_capacity);
    if (tile_order.has_value()) {
        const at::Tensor& t = *tile_order;
        if (t.dim() != 1 || t.scalar_type() != at::kInt || !t.is_contiguous() ||
            static_cast<size_t>(t.numel()) * sizeof(int32_t) < need) {
            throw std::invalid_argument("tile_order must be the contiguous int32 order conv_tile_order returned.");
        }
        require_device(t, "tile_order");
        *bytes = need | LATTICE_CONV_ORDER_READY;
        return t;
    }
    *bytes = need;
    return workspace(need, like);
}

at::Tensor sparse_conv_features_sorted_implicit_gemm(const at::Tensor& feats_in, const at::Tensor& weights_in,
                                                     const at::Tensor& sorted_out_in_map,
                                                     const at::Tensor& sorted_kv_out_in_map,
                                                     const at::Tensor& reorder_rows, const at::Tensor& tile_masks,
                                                     int out_capacity, int n_kernels, bool store_sorted,
                                                     const std::optional<at::Tensor>& bias,
                                                     const std::optional<at::Tensor>& tile_order, bool relu,
                                                     const std::optional<at::Tensor>& weight_fragments) {
    const char* op = "sparse_conv_features_sorted_implicit_gemm";
    if (sorted_out_in_map.dim() != 2 || sorted_out_in_map.scalar_type() != at::kInt) {
        throw std::invalid_argument("sorted_out_in_map must have shape (N_out, K) and int32 dtype.");
    }
    require_i32_vector(reorder_rows, "reorder_rows must have shape (N_out,) and int32 dtype.");
    require_i32_vector(tile_masks, "tile_masks must have shape (ceil(N_out / 64) * 4,) and int32 dtype.");
    if (sorted_out_in_map.size(0) != out_capacity || sorted_out_in_map.size(1) != n_kernels ||
        reorder_rows.size(0) != out_capacity) {
        throw std::invalid_argument("sorted convolution view shape must match out_capacity and n_kernels.");
    }
    if (tile_masks.size(0) != ((out_capacity + 63) / 64) * 4) {
        throw std::invalid_argument("tile_masks length must match ceil(out_capacity / 64) * 4.");
    }
    if (sorted_kv_out_in_map.dim() != 2 || sorted_kv_out_in_map.scalar_type() != at::kInt ||
        sorted_kv_out_in_map.size(0) != n_kernels || sorted_kv_out_in_map.size(1) != out_capacity) {
        throw std::invalid_argument("sorted_kv_out_in_map shape must match out_capacity and n_kernels.");
    }
    if (out_capacity < 0) {
        throw std::invalid_argument("out_capacity must be nonnegative and n_kernels must be positive.");
    }
    validate_weights(feats_in, weights_in, n_kernels, op);
    const at::Tensor feats = feats_in.contiguous();
    // The matrix-core B operand wants C_in contiguous per (C_out, k): the
    // dense 5D layout.  A mapped (K, C_in, C_out) weight is transposed once.
    const at::Tensor weights =
        weights_in.dim() == 5 ? weights_in.contiguous() : weights_in.permute({2, 0, 1}).contiguous();
    const int64_t c_out = out_channels_of(weights_in);
    at::Tensor out = at::empty({out_capacity, c_out}, feats.options());
    const at::Tensor kv = sorted_kv_out_in_map.contiguous();
    const at::Tensor tiles = tile_masks.contiguous();
    const at::Tensor order = reorder_rows.contiguous();
    size_t ws_bytes = 0;
    at::Tensor ws = schedule_workspace(tile_order, out_capacity, feats, &ws_bytes);
    at::Tensor bias_keep;
    const void* b = bias_ptr(bias, feats, c_out, &bias_keep);
    const int dtype = dtype_code(feats, op);
    const int c_in = static_cast<int>(feats.size(1));
    const size_t frag_bytes =
        lattice_hip_conv_weight_fragments_bytes(dtype, n_kernels, c_in, static_cast<int>(c_out));
    const bool small_table = (feats.size(0) + 1) * static_cast<int64_t>(c_in) * 2 <= (int64_t{1} << 32);
    if (frag_bytes > 0 && small_table) {
        // Streamed route: the weight in fragment order (the caller's cached
        // copy, or made now).
        at::Tensor frag;
        if (weight_fragments.has_value() && weight_fragments->numel() > 0) {
            frag = *weight_fragments;
            if (!frag.is_contiguous() || static_cast<size_t>(frag.numel()) * frag.element_size() < frag_bytes ||
                frag.scalar_type() != feats.scalar_type()) {
                throw std::invalid_argument("weight_fragments must be the conv_weight_fragments of this weight.");
            }
            require_device(frag, "weight_fragments");
        } else {
            frag = conv_weight_fragments(weights);
        }
        check_status(lattice_hip_sparse_conv_features_sorted_fragments(
            dtype, feats.data_ptr(), static_cast<int>(feats.size(0)), c_in, frag.data_ptr(), n_kernels,
            static_cast<int>(c_out), ci32(kv), ci32(tiles), store_sorted ? nullptr : ci32(order), out_capacity,
            out.data_ptr(), b, relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, ws.data_ptr(), ws_bytes,
            current_stream(feats)));
        return out;
    }
    check_status(lattice_hip_sparse_conv_features_sorted_implicit_gemm(
        dtype_code(feats, op), feats.data_ptr(), static_cast<int>(feats.size(0)), static_cast<int>(feats.size(1)),
        weights.data_ptr(), LATTICE_WEIGHT_DENSE_5D, n_kernels, static_cast<int>(c_out), ci32(kv), ci32(tiles),
        store_sorted ? nullptr : ci32(order), out_capacity, out.data_ptr(), b,
        relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, ws.data_ptr(), ws_bytes,
        current_stream(feats)));
    return out;
}

at::Tensor conv_weight_fragments(const at::Tensor& weights_in) {
    if (weights_in.dim() != 5 && weights_in.dim() != 3) {
        throw std::invalid_argument("weights must have shape (K, C_in, C_out) or (C_out, Kx, Ky, Kz, C_in).");
    }
    require_device(weights_in, "weights");
    const at::Tensor weights =
        weights_in.dim() == 5 ? weights_in.contiguous() : weights_in.permute({2, 0, 1}).contiguous();
    const int c_out = static_cast<int>(weights.size(0));
    const int c_in = static_cast<int>(weights.size(-1));
    const int k = static_cast<int>(weights.numel() / (static_cast<int64_t>(c_out) * c_in));
    int dtype = -1;
    if (weights.scalar_type() == at::kHalf) dtype = LATTICE_F16;
    if (weights.scalar_type() == at::kBFloat16) dtype = LATTICE_BF16;
    const size_t bytes = dtype < 0 ? 0 : lattice_hip_conv_weight_fragments_bytes(dtype, k, c_in, c_out);
    at::Tensor frag = at::empty({static_cast<int64_t>(bytes / weights.element_size())}, weights.options());
    if (bytes == 0) return frag;
    check_status(lattice_hip_conv_weight_fragments(dtype, weights.data_ptr(), k, c_in, c_out, frag.data_ptr(), bytes,
                                                   current_stream(weights)));
    return frag;
}

at::Tensor quantized_weight_fragments(const at::Tensor& weights_in, const at::Tensor& scales_in,
                                      const at::Tensor& biases_in, int in_channels, int out_channels,
                                      int storage_in_channels, int group_size, int bits) {
    if (weights_in.dim() != 3 || weights_in.scalar_type() != at::kUInt32) {
        throw std::invalid_argument("packed weights must be a three-dimensional uint32 array.");
    }
    if (scales_in.dim() != 3 || biases_in.sizes() != scales_in.sizes() ||
        biases_in.scalar_type() != scales_in.scalar_type()) {
        throw std::invalid_argument("quantized scales and biases must have equal shapes and dtypes.");
    }
    if (bits != 4 && bits != 8) throw std::invalid_argument("quantized convolution bits must be 4 or 8.");
    if (group_size != 32 && group_size != 64 && group_size != 128) {
        throw std::invalid_argument("quantized convolution group_size must be 32, 64, or 128.");
    }
    if (in_channels <= 0 || out_channels <= 0 || storage_in_channels < in_channels ||
        storage_in_channels % group_size != 0) {
        throw std::invalid_argument("quantized convolution channel metadata is invalid.");
    }
    const int k = static_cast<int>(weights_in.size(0));
    if (weights_in.size(1) != static_cast<int64_t>(storage_in_channels) * bits / 32 ||
        weights_in.size(2) != out_channels || scales_in.size(0) != k ||
        scales_in.size(1) != storage_in_channels / group_size || scales_in.size(2) != out_channels) {
        throw std::invalid_argument("packed weight shape does not match quantized convolution metadata.");
    }
    require_device(weights_in, "weights");
    require_device(scales_in, "scales");
    require_device(biases_in, "biases");
    int dtype = -1;
    if (scales_in.scalar_type() == at::kHalf) dtype = LATTICE_F16;
    if (scales_in.scalar_type() == at::kBFloat16) dtype = LATTICE_BF16;
    const size_t bytes =
        dtype < 0 ? 0 : lattice_hip_quantized_weight_fragments_bytes(dtype, k, in_channels, out_channels);
    at::Tensor frag = at::empty({static_cast<int64_t>(bytes / 2)}, scales_in.options());
    if (bytes == 0) return frag;
    const at::Tensor weights = weights_in.contiguous();
    const at::Tensor scales = scales_in.contiguous();
    const at::Tensor biases = biases_in.contiguous();
    check_status(lattice_hip_quantized_weight_fragments(
        dtype, reinterpret_cast<const uint32_t*>(weights.data_ptr()), scales.data_ptr(), biases.data_ptr(), k,
        in_channels, out_channels, storage_in_channels, group_size, bits, frag.data_ptr(), bytes,
        current_stream(weights)));
    return frag;
}

at::Tensor conv_tile_order(const at::Tensor& tile_masks, int out_capacity) {
    require_i32_vector(tile_masks, "tile_masks must have shape (ceil(N_out / 64) * 4,) and int32 dtype.");
    if (out_capacity < 0 || tile_masks.size(0) != ((out_capacity + 63) / 64) * 4) {
        throw std::invalid_argument("tile_masks length must match ceil(out_capacity / 64) * 4.");
    }
    require_device(tile_masks, "tile_masks");
    const at::Tensor tiles = tile_masks.contiguous();
    const size_t bytes = lattice_hip_conv_workspace_bytes(out_capacity);
    at::Tensor order = empty_i32({static_cast<int64_t>(bytes / sizeof(int32_t))}, tiles);
    check_status(lattice_hip_conv_tile_order(ci32(tiles), out_capacity, i32(order), bytes, current_stream(tiles)));
    return order;
}

at::Tensor sparse_quantized_conv_features(const at::Tensor& feats_in, const at::Tensor& weights_in,
                                          const at::Tensor& scales_in, const at::Tensor& biases_in,
                                          const at::Tensor& in_rows, const at::Tensor& out_rows,
                                          const at::Tensor& kernel_ids, const at::Tensor& counts,
                                          const at::Tensor& row_offsets, const at::Tensor& sorted_kv_out_in_map,
                                          const at::Tensor& reorder_rows, const at::Tensor& tile_masks,
                                          int out_capacity, int n_kernels, int in_channels, int out_channels,
                                          int storage_in_channels, int group_size, int bits,
                                          const std::optional<at::Tensor>& bias,
                                          const std::optional<at::Tensor>& tile_order, bool relu,
                                          const std::optional<at::Tensor>& weight_fragments,
                                          const std::optional<at::Tensor>& out_in_map) {
    if (out_capacity < 0 || n_kernels <= 0) {
        throw std::invalid_argument("out_capacity must be nonnegative and n_kernels must be positive.");
    }
    if (feats_in.dim() != 2 || (feats_in.scalar_type() != at::kHalf && feats_in.scalar_type() != at::kFloat &&
                                feats_in.scalar_type() != at::kBFloat16)) {
        throw std::invalid_argument("quantized sparse convolution features must be a float16 or float32 matrix.");
    }
    if (weights_in.dim() != 3 || weights_in.scalar_type() != at::kUInt32) {
        throw std::invalid_argument("packed weights must be a three-dimensional uint32 array.");
    }
    if (scales_in.dim() != 3 || biases_in.sizes() != scales_in.sizes() ||
        scales_in.scalar_type() != feats_in.scalar_type() || biases_in.scalar_type() != feats_in.scalar_type()) {
        throw std::invalid_argument(
            "quantized scales and biases must have shape (K, C_out, G) and match the feature dtype.");
    }
    if (bits != 4 && bits != 8) throw std::invalid_argument("quantized convolution bits must be 4 or 8.");
    if (group_size != 32 && group_size != 64 && group_size != 128) {
        throw std::invalid_argument("quantized convolution group_size must be 32, 64, or 128.");
    }
    if (in_channels <= 0 || out_channels <= 0 || storage_in_channels < in_channels ||
        storage_in_channels % group_size != 0) {
        throw std::invalid_argument("quantized convolution channel metadata is invalid.");
    }
    const int64_t packed_words = static_cast<int64_t>(storage_in_channels) * bits / 32;
    const int64_t groups = storage_in_channels / group_size;
    if (weights_in.size(0) != n_kernels || weights_in.size(1) != packed_words || weights_in.size(2) != out_channels ||
        scales_in.size(0) != n_kernels || scales_in.size(1) != groups || scales_in.size(2) != out_channels) {
        throw std::invalid_argument("packed weight shape does not match quantized convolution metadata.");
    }
    if (feats_in.size(1) != in_channels) {
        throw std::invalid_argument("feature shape does not match quantized convolution metadata.");
    }
    const bool has_plan = sorted_kv_out_in_map.numel() != 0 || reorder_rows.numel() != 0 || tile_masks.numel() != 0;
    if (has_plan) {
        if (sorted_kv_out_in_map.dim() != 2 || sorted_kv_out_in_map.size(0) != n_kernels ||
            sorted_kv_out_in_map.size(1) != out_capacity || sorted_kv_out_in_map.scalar_type() != at::kInt ||
            reorder_rows.dim() != 1 || reorder_rows.size(0) != out_capacity ||
            reorder_rows.scalar_type() != at::kInt || tile_masks.dim() != 1 ||
            tile_masks.size(0) != 4 * ((out_capacity + 63) / 64) || tile_masks.scalar_type() != at::kInt) {
            throw std::invalid_argument("quantized convolution sorted plan shapes are invalid.");
        }
    }
    if (in_rows.dim() != 1 || out_rows.dim() != 1 || kernel_ids.dim() != 1 || in_rows.scalar_type() != at::kInt ||
        out_rows.scalar_type() != at::kInt || kernel_ids.scalar_type() != at::kInt ||
        in_rows.sizes() != out_rows.sizes() || in_rows.sizes() != kernel_ids.sizes()) {
        throw std::invalid_argument(
            "quantized convolution relation edges must be equal-length one-dimensional int32 arrays.");
    }
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("quantized convolution counts must have shape (2,) and int32 dtype.");
    }
    if (row_offsets.dim() != 1 || row_offsets.size(0) != out_capacity + 1 || row_offsets.scalar_type() != at::kInt) {
        throw std::invalid_argument(
            "quantized convolution row_offsets must have length out_capacity + 1 and int32 dtype.");
    }
    require_device(feats_in, "feats");
    const at::Tensor feats = feats_in.contiguous();
    const at::Tensor weights = weights_in.contiguous();
    const at::Tensor scales = scales_in.contiguous();
    const at::Tensor biases = biases_in.contiguous();
    at::Tensor kv;
    at::Tensor order;
    at::Tensor tiles;
    if (has_plan) {
        kv = sorted_kv_out_in_map.contiguous();
        order = reorder_rows.contiguous();
        tiles = tile_masks.contiguous();
    }
    at::Tensor out = at::empty({out_capacity, out_channels}, feats.options());
    size_t ws_bytes = 0;
    at::Tensor ws;
    if (has_plan) ws = schedule_workspace(tile_order, out_capacity, feats, &ws_bytes);
    at::Tensor bias_keep;
    const void* b = bias_ptr(bias, feats, out_channels, &bias_keep);
    const int dtype = dtype_code(feats, "quantized sparse convolution");
    const size_t frag_bytes = dtype == LATTICE_F32 ? 0
                                                   : lattice_hip_quantized_weight_fragments_bytes(
                                                         dtype, n_kernels, in_channels, out_channels);
    const at::Tensor map =
        dense_map_for(out_in_map, dtype, feats, in_channels, out_channels, n_kernels, out_capacity);
    if (map.defined()) {
        check_status(lattice_hip_sparse_quantized_conv_features_dense_map(
            dtype, feats.data_ptr(), static_cast<int>(feats.size(0)), in_channels,
            reinterpret_cast<const uint32_t*>(weights.data_ptr()), scales.data_ptr(), biases.data_ptr(), n_kernels,
            out_channels, storage_in_channels, group_size, bits, ci32(map), ci32(counts), out_capacity,
            out.data_ptr(), b, relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, current_stream(feats)));
        return out;
    }
    const bool small_table = (feats.size(0) + 1) * static_cast<int64_t>(in_channels) * 2 <= (int64_t{1} << 32);
    if (has_plan && frag_bytes > 0 && small_table) {
        // Streamed route: the packed weight in fragment order (the caller's
        // cached copy, or made now), dequantised in registers.
        at::Tensor frag;
        if (weight_fragments.has_value() && weight_fragments->numel() > 0) {
            frag = *weight_fragments;
            if (!frag.is_contiguous() || static_cast<size_t>(frag.numel()) * frag.element_size() < frag_bytes) {
                throw std::invalid_argument("weight_fragments must be the quantized_weight_fragments of this weight.");
            }
            require_device(frag, "weight_fragments");
        } else {
            frag = quantized_weight_fragments(weights, scales, biases, in_channels, out_channels,
                                              storage_in_channels, group_size, bits);
        }
        check_status(lattice_hip_sparse_quantized_conv_features_sorted_fragments(
            dtype, feats.data_ptr(), static_cast<int>(feats.size(0)), in_channels, frag.data_ptr(), bits, n_kernels,
            out_channels, ci32(kv), ci32(tiles), ci32(order), out_capacity, out.data_ptr(), b,
            relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, ws.data_ptr(), ws_bytes, current_stream(feats)));
        return out;
    }
    check_status(lattice_hip_sparse_quantized_conv_features(
        dtype_code(feats, "quantized sparse convolution"), feats.data_ptr(), static_cast<int>(feats.size(0)),
        in_channels, reinterpret_cast<const uint32_t*>(weights.data_ptr()), scales.data_ptr(), biases.data_ptr(),
        n_kernels, out_channels, storage_in_channels, group_size, bits, ci32(in_rows), ci32(kernel_ids),
        ci32(counts), static_cast<int>(in_rows.size(0)), ci32(row_offsets), has_plan ? ci32(kv) : nullptr,
        has_plan ? ci32(tiles) : nullptr, has_plan ? ci32(order) : nullptr, out_capacity, out.data_ptr(), b,
        relu ? LATTICE_EPILOGUE_RELU : LATTICE_EPILOGUE_NONE, has_plan ? ws.data_ptr() : nullptr, ws_bytes,
        current_stream(feats)));
    return out;
}

at::Tensor sparse_conv_input_grad(const at::Tensor& cot_in, const at::Tensor& weights_in, const at::Tensor& out_rows,
                                  const at::Tensor& kernel_ids, const at::Tensor& counts,
                                  const at::Tensor& in_row_offsets, const at::Tensor& in_edge_ids, int in_capacity,
                                  int n_kernels) {
    const char* op = "sparse_conv_input_grad";
    if (cot_in.dim() != 2) throw std::invalid_argument("cotangent must have shape (N_out, C_out).");
    if (weights_in.dim() != 3 && weights_in.dim() != 5) {
        throw std::invalid_argument("weights must have shape (K, C_in, C_out) or (C_out, Kx, Ky, Kz, C_in).");
    }
    const int64_t c_out = out_channels_of(weights_in);
    const int64_t c_in = weights_in.dim() == 3 ? weights_in.size(1) : weights_in.size(4);
    if (cot_in.size(1) != c_out) throw std::invalid_argument("cotangent channels must match weights output channels.");
    if (weights_in.scalar_type() != cot_in.scalar_type()) {
        throw std::invalid_argument(std::string(op) + " weights must match the cotangent dtype.");
    }
    if (in_capacity < 0 || n_kernels <= 0) {
        throw std::invalid_argument("in_capacity must be nonnegative and n_kernels must be positive.");
    }
    require_i32_vector(out_rows, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    require_i32_vector(kernel_ids, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    require_i32_vector(in_row_offsets, "plan row_offsets must be one-dimensional int32 arrays.");
    require_i32_vector(in_edge_ids, "plan edge_ids must be one-dimensional int32 arrays.");
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("counts must have shape (2,) and int32 dtype.");
    }
    if (in_row_offsets.size(0) != in_capacity + 1) {
        throw std::invalid_argument("in_row_offsets length must match input capacity + 1.");
    }
    if (out_rows.size(0) != kernel_ids.size(0) || in_edge_ids.size(0) != out_rows.size(0)) {
        throw std::invalid_argument("plan edge_ids must match relation edge capacity.");
    }
    require_device(cot_in, "cotangent");
    require_device(weights_in, "weights");
    const at::Tensor cot = cot_in.contiguous();
    const at::Tensor weights = weights_in.contiguous();
    at::Tensor grad = at::empty({in_capacity, c_in}, cot.options());
    check_status(lattice_hip_sparse_conv_input_grad(
        dtype_code(cot, op), cot.data_ptr(), static_cast<int>(cot.size(0)), static_cast<int>(c_out),
        weights.data_ptr(), weights.dim() == 3 ? LATTICE_WEIGHT_KERNEL_MAJOR : LATTICE_WEIGHT_DENSE_5D, n_kernels,
        static_cast<int>(c_in), ci32(out_rows), ci32(kernel_ids), ci32(counts), static_cast<int>(out_rows.size(0)),
        ci32(in_row_offsets), ci32(in_edge_ids), in_capacity, grad.data_ptr(), current_stream(cot)));
    return grad;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> build_transposed_implicit_gemm_map(const at::Tensor& in_rows,
                                                                      const at::Tensor& out_rows,
                                                                      const at::Tensor& kernel_ids,
                                                                      const at::Tensor& counts, int in_capacity,
                                                                      int n_kernels) {
    require_i32_vector(in_rows, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    require_i32_vector(out_rows, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    require_i32_vector(kernel_ids, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    if (in_rows.size(0) != out_rows.size(0) || in_rows.size(0) != kernel_ids.size(0)) {
        throw std::invalid_argument("relation row arrays and kernel_ids must have equal capacity.");
    }
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("counts must have shape (2,) and int32 dtype.");
    }
    if (in_capacity < 0 || n_kernels <= 0) {
        throw std::invalid_argument("in_capacity must be nonnegative and n_kernels must be positive.");
    }
    require_device(in_rows, "in_rows");
    at::Tensor map = empty_i32({in_capacity, n_kernels}, in_rows);
    at::Tensor masks = empty_i32({in_capacity, (n_kernels + 31) / 32}, in_rows);
    at::Tensor status = empty_i32({1}, in_rows);
    check_status(lattice_hip_build_transposed_implicit_gemm_map(
        ci32(in_rows), ci32(out_rows), ci32(kernel_ids), ci32(counts), static_cast<int>(in_rows.size(0)),
        in_capacity, n_kernels, i32(map), i32(masks), i32(status), current_stream(in_rows)));
    return {map, masks, status};
}

at::Tensor sparse_conv_weight_grad(const at::Tensor& feats_in, const at::Tensor& cot_in, const at::Tensor& weights,
                                   const at::Tensor& in_rows, const at::Tensor& out_rows, const at::Tensor& counts,
                                   const at::Tensor& kernel_row_offsets, const at::Tensor& kernel_edge_ids,
                                   int n_kernels) {
    const char* op = "sparse_conv_weight_grad";
    validate_weights(feats_in, weights, n_kernels, op);
    const int64_t c_out = out_channels_of(weights);
    if (cot_in.dim() != 2 || cot_in.size(1) != c_out) {
        throw std::invalid_argument("cotangent must have shape (N_out, C_out).");
    }
    if (cot_in.scalar_type() != feats_in.scalar_type()) {
        throw std::invalid_argument(std::string(op) + " cotangent must match feats dtype.");
    }
    require_i32_vector(in_rows, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    require_i32_vector(out_rows, "relation rows and kernel_ids must be one-dimensional int32 arrays.");
    require_i32_vector(kernel_row_offsets, "plan row_offsets must be one-dimensional int32 arrays.");
    require_i32_vector(kernel_edge_ids, "plan edge_ids must be one-dimensional int32 arrays.");
    if (counts.dim() != 1 || counts.size(0) != 2 || counts.scalar_type() != at::kInt) {
        throw std::invalid_argument("counts must have shape (2,) and int32 dtype.");
    }
    if (kernel_row_offsets.size(0) != n_kernels + 1) {
        throw std::invalid_argument("kernel_row_offsets length must match n_kernels + 1.");
    }
    if (in_rows.size(0) != out_rows.size(0) || kernel_edge_ids.size(0) != in_rows.size(0)) {
        throw std::invalid_argument("plan edge_ids must match relation edge capacity.");
    }
    require_device(cot_in, "cotangent");
    const at::Tensor feats = feats_in.contiguous();
    const at::Tensor cot = cot_in.contiguous();
    const int dtype = dtype_code(feats, op);
    const int c_in = static_cast<int>(feats.size(1));
    const int edge_cap = static_cast<int>(in_rows.size(0));
    at::Tensor grad = at::empty(weights.sizes(), cot.options());
    const size_t ws_bytes =
        lattice_hip_conv_weight_grad_workspace_bytes(dtype, n_kernels, c_in, static_cast<int>(c_out), edge_cap);
    at::Tensor ws = workspace(ws_bytes, feats);
    check_status(lattice_hip_sparse_conv_weight_grad(
        dtype, feats.data_ptr(), static_cast<int>(feats.size(0)), c_in, cot.data_ptr(), static_cast<int>(cot.size(0)),
        static_cast<int>(c_out), weights.dim() == 3 ? LATTICE_WEIGHT_KERNEL_MAJOR : LATTICE_WEIGHT_DENSE_5D,
        n_kernels, ci32(in_rows), ci32(out_rows), ci32(counts), edge_cap, ci32(kernel_row_offsets),
        ci32(kernel_edge_ids), grad.data_ptr(), ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, current_stream(feats)));
    return grad;
}

}  // namespace lattice_native
