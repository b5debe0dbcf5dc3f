// Host-side plumbing shared by the native feature layer: the current torch
// HIP stream, C-ABI status translation and tensor checks.
#pragma once

#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <stdexcept>
#include <string>

#include "lattice_hip.h"

namespace lattice_native {

inline void* current_stream(const at::Tensor& on) {
    return static_cast<void*>(c10::hip::getCurrentHIPStream(on.device().index()).stream());
}

// LATTICE_ERROR_INVALID_ARGUMENT -> std::invalid_argument (ValueError in
// Python, as the reference's validation raises); anything else ->
// std::runtime_error.
inline void check_status(int rc) {
    if (rc == LATTICE_OK) return;
    std::string message = lattice_hip_last_error();
    if (rc == LATTICE_ERROR_INVALID_ARGUMENT) throw std::invalid_argument(message);
    throw std::runtime_error(message);
}

inline void require(bool cond, const char* message) {
    if (!cond) throw std::invalid_argument(message);
}

inline void require_device(const at::Tensor& t, const char* name) {
    if (!t.is_cuda()) {
        throw std::invalid_argument(std::string(name) +
                                    " must be a HIP device tensor (the lattice native path runs on the GPU).");
    }
}

inline int32_t* i32(at::Tensor& t) { return t.data_ptr<int32_t>(); }
inline const int32_t* ci32(const at::Tensor& t) { return t.data_ptr<int32_t>(); }

inline at::Tensor empty_i32(at::IntArrayRef shape, const at::Tensor& like) {
    return at::empty(shape, like.options().dtype(at::kInt));
}

inline at::Tensor workspace(size_t bytes, const at::Tensor& like) {
    return at::empty({static_cast<int64_t>(bytes)}, like.options().dtype(at::kByte));
}

}  // namespace lattice_native
