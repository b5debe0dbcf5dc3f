// Sparse pooling over a kernel relation (native/features/pooling/
// primitive.cpp; CPU routines pooling/cpu/algorithms.cpp:180-331) and the
// per-batch global pools (mlx_lattice/ops/pool.py:198-236).
//
// Pooling reads each contributing feature row once per edge and writes each
// output row once: HBM-bound integer-indexed gathers, one lane per
// (row, channel) so the lanes of a row read consecutive channels.
//  * forward: output rows start at the reduction identity (-inf for max, 0
//    otherwise); rows below counts[1] reduce their CSR edges' input rows;
//    avg divides by max(degree, 1).
//  * gradient: one lane per (input row, channel) over the input-grouped CSR;
//    max routes the cotangent to the inputs equal to the pooled value,
//    split evenly over ties (the reference's tie policy).
//  * global pools: one block per (batch, 64-channel tile), four row groups
//    reduced through LDS.

#include <algorithm>
#include <cmath>

#include "lattice_common.h"

namespace lattice {
namespace {

constexpr int kPoolSum = 0;
constexpr int kPoolMax = 1;
constexpr int kPoolAvg = 2;

// One lane per (output row, V-channel chunk): V = 4 (16-byte loads and
// stores) when the channel count allows, else 1; each channel reduces its
// edges in CSR order either way.
// Outputs are written with non-temporal stores (streamed past the caches;
// max_pool3d k2s2 over 400k rows, 64 channels: 33.8 -> 32.2 us).
typedef float f32x4v_t __attribute__((ext_vector_type(4)));
template <int V> struct PoolVec;
template <> struct PoolVec<1> {
    float v[1];
    __device__ static PoolVec load(const float* p) { return {{p[0]}}; }
    __device__ void store(float* p) const { __builtin_nontemporal_store(v[0], p); }
};
template <> struct PoolVec<4> {
    float v[4];
    __device__ static PoolVec load(const float* p) {
        const float4 f = *reinterpret_cast<const float4*>(p);
        return {{f.x, f.y, f.z, f.w}};
    }
    __device__ void store(float* p) const {
        __builtin_nontemporal_store(f32x4v_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4v_t*>(p));
    }
};

template <int V>
__global__ void __launch_bounds__(256)
pool_forward(int mode, const float* __restrict__ feats, int n_in, int channels, const int32_t* __restrict__ in_rows,
             int edge_capacity, const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ counts,
             int out_capacity, float* __restrict__ out) {
    const int out_count = min(counts[1], out_capacity);
    const int chunks = channels / V;
    const long long total = static_cast<long long>(out_capacity) * chunks;
    const float identity = mode == kPoolMax ? -INFINITY : 0.0f;
    for (long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(t / chunks);
        const int c = static_cast<int>(t - static_cast<long long>(row) * chunks) * V;
        PoolVec<V> acc;
#pragma unroll
        for (int j = 0; j < V; ++j) acc.v[j] = identity;
        if (row < out_count) {
            const int lo = row_offsets[row];
            const int hi = row_offsets[row + 1];
            for (int e = lo; e < hi; ++e) {
                if (e < 0 || e >= edge_capacity) continue;
                const int in = in_rows[e];
                if (in < 0 || in >= n_in) continue;
                const PoolVec<V> x = PoolVec<V>::load(feats + static_cast<long long>(in) * channels + c);
#pragma unroll
                for (int j = 0; j < V; ++j) acc.v[j] = mode == kPoolMax ? fmaxf(acc.v[j], x.v[j]) : acc.v[j] + x.v[j];
            }
            if (mode == kPoolAvg) {
                const float scale = 1.0f / static_cast<float>(max(hi - lo, 1));
#pragma unroll
                for (int j = 0; j < V; ++j) acc.v[j] *= scale;
            }
        }
        acc.store(out + static_cast<long long>(row) * channels + c);
    }
}

__global__ void __launch_bounds__(256)
pool_grad(int mode, const float* __restrict__ cot, const float* __restrict__ feats,
          const float* __restrict__ pooled, int n_in, int channels, const int32_t* __restrict__ in_rows,
          const int32_t* __restrict__ out_rows, int edge_capacity, const int32_t* __restrict__ row_offsets,
          const int32_t* __restrict__ counts, const int32_t* __restrict__ in_row_offsets,
          const int32_t* __restrict__ in_edge_ids, int out_capacity, float* __restrict__ grad) {
    const int out_count = min(counts[1], out_capacity);
    const long long total = static_cast<long long>(n_in) * channels;
    for (long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int in = static_cast<int>(t / channels);
        const int c = static_cast<int>(t - static_cast<long long>(in) * channels);
        float value = 0.0f;
        for (int cur = in_row_offsets[in]; cur < in_row_offsets[in + 1]; ++cur) {
            const int e = in_edge_ids[cur];
            if (e < 0 || e >= edge_capacity) continue;
            const int o = out_rows[e];
            if (o < 0 || o >= out_count) continue;
            const int lo = row_offsets[o];
            const int hi = row_offsets[o + 1];
            float scale = 1.0f;
            if (mode == kPoolMax) {
                const float pv = pooled[static_cast<long long>(o) * channels + c];
                if (feats[t] != pv) continue;
                int ties = 0;
                for (int e2 = lo; e2 < hi; ++e2) {
                    if (e2 < 0 || e2 >= edge_capacity) continue;
                    const int i2 = in_rows[e2];
                    if (i2 >= 0 && i2 < n_in && feats[static_cast<long long>(i2) * channels + c] == pv) ++ties;
                }
                if (ties == 0) continue;
                scale = 1.0f / static_cast<float>(ties);
            } else if (mode == kPoolAvg) {
                scale = 1.0f / static_cast<float>(max(hi - lo, 1));
            }
            value += cot[static_cast<long long>(o) * channels + c] * scale;
        }
        grad[t] = value;
    }
}

// Block (batch b, 64-channel tile): rows batch_offsets[b] .. [b+1].
__global__ void __launch_bounds__(256)
global_pool(int mode, const float* __restrict__ feats, int channels, const int64_t* __restrict__ batch_offsets,
            float* __restrict__ out) {
    __shared__ float part[4][64];
    const int b = blockIdx.x;
    const int c = blockIdx.y * 64 + (threadIdx.x & 63);
    const int group = threadIdx.x >> 6;
    const long long lo = batch_offsets[b];
    const long long hi = batch_offsets[b + 1];
    float acc = mode == kPoolMax ? -INFINITY : 0.0f;
    if (c < channels) {
        for (long long r = lo + group; r < hi; r += 4) {
            const float v = feats[r * channels + c];
            acc = mode == kPoolMax ? fmaxf(acc, v) : acc + v;
        }
    }
    part[group][threadIdx.x & 63] = acc;
    __syncthreads();
    if (group == 0 && c < channels) {
        float r = part[0][threadIdx.x];
        for (int g = 1; g < 4; ++g) r = mode == kPoolMax ? fmaxf(r, part[g][threadIdx.x]) : r + part[g][threadIdx.x];
        if (mode == kPoolAvg && hi > lo) r /= static_cast<float>(hi - lo);
        out[static_cast<long long>(b) * channels + c] = r;
    }
}

}  // namespace
}  // namespace lattice

using namespace lattice;

extern "C" int lattice_hip_sparse_pool_features(int mode, const float* feats, int n_in, int channels,
                                                const int32_t* in_rows, int edge_capacity,
                                                const int32_t* row_offsets, const int32_t* counts, int out_capacity,
                                                float* out, void* stream_ptr) {
    LATTICE_REQUIRE(mode == kPoolSum || mode == kPoolMax || mode == kPoolAvg, "reduce must be 'sum', 'max', or 'avg'.");
    LATTICE_REQUIRE(n_in >= 0 && channels > 0 && edge_capacity >= 0 && out_capacity >= 0,
                    "pooling shapes must be nonnegative with positive channels.");
    if (out_capacity == 0) return LATTICE_OK;
    LATTICE_REQUIRE(out && row_offsets && counts && (edge_capacity == 0 || in_rows) && (feats || n_in == 0),
                    "pooling pointers must be non-null.");
    if (channels % 4 == 0) {
        const long long total = static_cast<long long>(out_capacity) * (channels / 4);
        pool_forward<4><<<grid_for(total, 256, 1u << 16), 256, 0, as_stream(stream_ptr)>>>(
            mode, feats, n_in, channels, in_rows, edge_capacity, row_offsets, counts, out_capacity, out);
    } else {
        const long long total = static_cast<long long>(out_capacity) * channels;
        pool_forward<1><<<grid_for(total, 256, 1u << 16), 256, 0, as_stream(stream_ptr)>>>(
            mode, feats, n_in, channels, in_rows, edge_capacity, row_offsets, counts, out_capacity, out);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_sparse_pool_features_grad(int mode, const float* cot, const float* feats,
                                                     const float* pooled, int n_in, int channels,
                                                     const int32_t* in_rows, const int32_t* out_rows,
                                                     int edge_capacity, const int32_t* row_offsets,
                                                     const int32_t* counts, const int32_t* in_row_offsets,
                                                     const int32_t* in_edge_ids, int out_capacity, float* grad,
                                                     void* stream_ptr) {
    LATTICE_REQUIRE(mode == kPoolSum || mode == kPoolMax || mode == kPoolAvg, "reduce must be 'sum', 'max', or 'avg'.");
    LATTICE_REQUIRE(n_in >= 0 && channels > 0 && edge_capacity >= 0 && out_capacity >= 0,
                    "pooling shapes must be nonnegative with positive channels.");
    if (n_in == 0) return LATTICE_OK;
    LATTICE_REQUIRE(grad && feats && row_offsets && counts && in_row_offsets && in_edge_ids &&
                        (edge_capacity == 0 || (in_rows && out_rows)) && (cot || out_capacity == 0) &&
                        (pooled || mode != kPoolMax),
                    "pooling gradient pointers must be non-null.");
    const long long total = static_cast<long long>(n_in) * channels;
    pool_grad<<<grid_for(total, 256, 1u << 16), 256, 0, as_stream(stream_ptr)>>>(
        mode, cot, feats, pooled, n_in, channels, in_rows, out_rows, edge_capacity, row_offsets, counts,
        in_row_offsets, in_edge_ids, out_capacity, grad);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_global_pool(int mode, const float* feats, int channels, const int64_t* batch_offsets,
                                       int batches, float* out, void* stream_ptr) {
    LATTICE_REQUIRE(mode == kPoolSum || mode == kPoolMax || mode == kPoolAvg, "mode must be 'sum', 'max', or 'avg'.");
    LATTICE_REQUIRE(channels > 0 && batches >= 0, "global pooling shapes must be positive.");
    if (batches == 0) return LATTICE_OK;
    LATTICE_REQUIRE(out && batch_offsets, "global pooling pointers must be non-null.");
    dim3 grid(static_cast<unsigned>(batches), static_cast<unsigned>((channels + 63) / 64));
    global_pool<<<grid, 256, 0, as_stream(stream_ptr)>>>(mode, feats, channels, batch_offsets, out);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}
