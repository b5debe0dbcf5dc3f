// Sparse convolution feature kernels for gfx950.
//
// Two routes:
//  * CSR route (bandwidth path): one lane per (output row, output channel)
//    walks the row's edges (row_offsets / in_rows / kernel_ids) with an fp32
//    accumulator; lanes of a row read the same feature values (broadcast)
//    and consecutive output channels of the weight (coalesced).  Follows
//    the output-stationary loop of cpu/algorithms.cpp:180-302 and, for packed
//    weights, cpu/quantized.cpp:64-141.  Used for fp32, for channel counts
//    that do not tile the matrix cores, and for small problems.
//  * Implicit-GEMM route (MFMA path): output rows are visited in the
//    mask-sorted order of the sorted view (core/relations/views.py:467-510),
//    64 rows per 256-thread block.  For every kernel offset that any row of
//    the tile uses, the block gathers the 64 input rows into LDS (zeros for
//    misses) and multiplies them by W[k] with v_mfma_f32_16x16x32_{f16,bf16}
//    (fp32 accumulate).  Packed int4/int8 weights are dequantised
//    (w = q*scale + bias) while the B operand is loaded, so no dequantised
//    weight is ever materialised.

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <climits>

#include "lattice_common.h"
#include "scan.h"

namespace lattice {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ element IO --

template <typename T> struct Elem;
template <> struct Elem<float> {
    __device__ static float load(const float* p, long long i) { return p[i]; }
    __device__ static void store(float* p, long long i, float v) { p[i] = v; }
};
template <> struct Elem<_Float16> {
    __device__ static float load(const _Float16* p, long long i) { return static_cast<float>(p[i]); }
    __device__ static void store(_Float16* p, long long i, float v) { p[i] = static_cast<_Float16>(v); }
};
template <> struct Elem<__bf16> {
    __device__ static float load(const __bf16* p, long long i) { return static_cast<float>(p[i]); }
    __device__ static void store(__bf16* p, long long i, float v) { p[i] = static_cast<__bf16>(v); }
};

// ------------------------------------------------------------- CSR route --

struct WeightIndex {
    int layout;  // LATTICE_WEIGHT_*
    int K, c_in, c_out;
    __device__ inline long long operator()(int k, int ci, int co) const {
        if (layout == LATTICE_WEIGHT_KERNEL_MAJOR) return (static_cast<long long>(k) * c_in + ci) * c_out + co;
        return (static_cast<long long>(co) * K + k) * c_in + ci;
    }
};

template <typename T>
__global__ void __launch_bounds__(256)
conv_csr(const T* __restrict__ feats, int c_in, const T* __restrict__ weights, WeightIndex widx,
         const int32_t* __restrict__ in_rows, const int32_t* __restrict__ kernel_ids,
         const int32_t* __restrict__ counts, int edge_capacity, const int32_t* __restrict__ row_offsets,
         int out_capacity, T* __restrict__ out) {
    const int c_out = widx.c_out;
    const int E = min(counts[0], edge_capacity);
    const int n_out = min(counts[1], out_capacity);
    const long long total = static_cast<long long>(out_capacity) * c_out;
    for (long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(t / c_out);
        const int co = static_cast<int>(t - static_cast<long long>(row) * c_out);
        float acc = 0.0f;
        if (row < n_out) {
            const int e_end = row_offsets[row + 1];
            for (int e = row_offsets[row]; e < e_end; ++e) {
                if (e < 0 || e >= E) continue;
                const int in = in_rows[e];
                const int k = kernel_ids[e];
                if (in < 0 || k < 0 || k >= widx.K) continue;
                const T* f = feats + static_cast<long long>(in) * c_in;
                for (int ci = 0; ci < c_in; ++ci) {
                    acc += Elem<T>::load(f, ci) * Elem<T>::load(weights, widx(k, ci, co));
                }
            }
        }
        Elem<T>::store(out, t, acc);
    }
}

struct QuantIndex {
    int K, c_in, c_out, packed_words, groups, group_size, bits;
};

template <typename T>
__device__ inline float dequant(const uint32_t* __restrict__ weights, const T* __restrict__ scales,
                                const T* __restrict__ biases, const QuantIndex& q, int k, int ci, int co) {
    const int bit = ci * q.bits;
    const uint32_t word =
        weights[(static_cast<long long>(k) * q.packed_words + (bit >> 5)) * q.c_out + co];
    const uint32_t code = (word >> (bit & 31)) & ((1u << q.bits) - 1u);
    const long long s = (static_cast<long long>(k) * q.groups + ci / q.group_size) * q.c_out + co;
    return static_cast<float>(code) * Elem<T>::load(scales, s) + Elem<T>::load(biases, s);
}

template <typename T>
__global__ void __launch_bounds__(256)
quant_conv_csr(const T* __restrict__ feats, const uint32_t* __restrict__ weights, const T* __restrict__ scales,
               const T* __restrict__ biases, QuantIndex q, const int32_t* __restrict__ in_rows,
               const int32_t* __restrict__ kernel_ids, const int32_t* __restrict__ counts, int edge_capacity,
               const int32_t* __restrict__ row_offsets, int out_capacity, T* __restrict__ out) {
    const int E = min(counts[0], edge_capacity);
    const int n_out = min(counts[1], out_capacity);
    const long long total = static_cast<long long>(out_capacity) * q.c_out;
    for (long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(t / q.c_out);
        const int co = static_cast<int>(t - static_cast<long long>(row) * q.c_out);
        float acc = 0.0f;
        if (row < n_out) {
            const int e_end = row_offsets[row + 1];
            for (int e = row_offsets[row]; e < e_end; ++e) {
                if (e < 0 || e >= E) continue;
                const int in = in_rows[e];
                const int k = kernel_ids[e];
                if (in < 0 || k < 0 || k >= q.K) continue;
                const T* f = feats + static_cast<long long>(in) * q.c_in;
                for (int ci = 0; ci < q.c_in; ++ci) {
                    acc += Elem<T>::load(f, ci) * dequant(weights, scales, biases, q, k, ci, co);
                }
            }
        }
        Elem<T>::store(out, t, acc);
    }
}

// ------------------------------------------------------ implicit GEMM ----

constexpr int kTileRows = 64;
constexpr int kBlock = 256;
constexpr int kLdsPad = 8;  // halves appended to each LDS row (bank spread)

template <typename T> struct MfmaOps;
template <> struct MfmaOps<_Float16> {
    typedef half8_t vec;
    __device__ static float4_t mfma(vec a, vec b, float4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct MfmaOps<__bf16> {
    typedef bf16x8_t vec;
    __device__ static float4_t mfma(vec a, vec b, float4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

// Wave layout over the 64 x C_OUT tile: WN waves across columns.
template <int C_OUT> struct TileShape {
    static constexpr int WN = (C_OUT / 16) >= 4 ? 4 : (C_OUT / 16);
    static constexpr int WM = 4 / WN;
    static constexpr int TM = kTileRows / WM;   // rows per wave
    static constexpr int TN = C_OUT / WN;       // cols per wave
    static constexpr int RB = TM / 16;          // 16-row blocks per wave
    static constexpr int CB = TN / 16;          // 16-col blocks per wave
};

struct MapView {
    const int32_t* map;   // sorted map
    long long row_stride; // elements between consecutive sorted rows
    long long k_stride;   // elements between consecutive kernel offsets
};

// B operand source: float weights (n-major: co stride, k stride, ci
// contiguous) or packed affine codes.
template <typename T> struct FloatB {
    const T* w;
    long long s_co, s_k;
    __device__ inline typename MfmaOps<T>::vec load(int k, int co, int ci0) const {
        return *reinterpret_cast<const typename MfmaOps<T>::vec*>(w + co * s_co + k * s_k + ci0);
    }
};

template <typename T> struct PackedB {
    const uint32_t* w;
    const T* scales;
    const T* biases;
    int packed_words, groups, group_size, c_out, bits;
    __device__ inline typename MfmaOps<T>::vec load(int k, int co, int ci0) const {
        typename MfmaOps<T>::vec out;
        const long long s = (static_cast<long long>(k) * groups + ci0 / group_size) * c_out + co;
        const float sc = Elem<T>::load(scales, s);
        const float bi = Elem<T>::load(biases, s);
        const long long wbase = static_cast<long long>(k) * packed_words * c_out + co;
        if (bits == 4) {
            const uint32_t word = w[wbase + static_cast<long long>(ci0 >> 3) * c_out];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                out[j] = static_cast<T>(static_cast<float>((word >> (4 * j)) & 15u) * sc + bi);
            }
        } else {
            const uint32_t w0 = w[wbase + static_cast<long long>(ci0 >> 2) * c_out];
            const uint32_t w1 = w[wbase + static_cast<long long>((ci0 >> 2) + 1) * c_out];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                out[j] = static_cast<T>(static_cast<float>((w0 >> (8 * j)) & 255u) * sc + bi);
                out[4 + j] = static_cast<T>(static_cast<float>((w1 >> (8 * j)) & 255u) * sc + bi);
            }
        }
        return out;
    }
};

template <typename T, int C_OUT, typename BSource>
__global__ void __launch_bounds__(kBlock)
conv_igemm(const T* __restrict__ feats, int c_in, BSource bsrc, MapView mv, int K,
           const int32_t* __restrict__ reorder_rows, int rows, T* __restrict__ out) {
    using S = TileShape<C_OUT>;
    using V = typename MfmaOps<T>::vec;
    extern __shared__ __align__(16) unsigned char lds_raw[];
    const int lds_row = c_in + kLdsPad;                       // halves per LDS row
    T* a_tile = reinterpret_cast<T*>(lds_raw);                // [64][lds_row]
    int32_t* map_tile = reinterpret_cast<int32_t*>(lds_raw + sizeof(T) * kTileRows * lds_row);  // [64][K]
    __shared__ uint32_t tile_mask;

    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid / kWave;
    const int wm = wave / S::WN;
    const int wn = wave % S::WN;
    const int tile = blockIdx.x;
    const int row0 = tile * kTileRows;

    if (tid == 0) tile_mask = 0;
    __syncthreads();
    uint32_t my_mask = 0;
    for (int i = tid; i < kTileRows * K; i += kBlock) {
        const int r = i / K;
        const int k = i - r * K;
        const int sr = row0 + r;
        int v = -1;
        if (sr < rows) v = mv.map[sr * mv.row_stride + k * mv.k_stride];
        map_tile[i] = v;
        if (v >= 0) my_mask |= 1u << k;
    }
    if (my_mask) atomicOr(&tile_mask, my_mask);
    __syncthreads();
    uint32_t kmask = tile_mask;

    float4_t acc[S::RB][S::CB];
#pragma unroll
    for (int i = 0; i < S::RB; ++i)
#pragma unroll
        for (int j = 0; j < S::CB; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int chunks_per_row = c_in / 8;  // 16-byte chunks
    while (kmask) {
        const int k = __builtin_ctz(kmask);
        kmask &= kmask - 1;
        // Gather the tile's input rows for offset k into LDS.
        for (int i = tid; i < kTileRows * chunks_per_row; i += kBlock) {
            const int r = i / chunks_per_row;
            const int c = i - r * chunks_per_row;
            const int in = map_tile[r * K + k];
            V v;
            if (in >= 0) {
                v = *reinterpret_cast<const V*>(feats + static_cast<long long>(in) * c_in + c * 8);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = static_cast<T>(0.0f);
            }
            *reinterpret_cast<V*>(a_tile + r * lds_row + c * 8) = v;
        }
        __syncthreads();
        const int fr = lane & 15;        // fragment row / col
        const int fk = (lane >> 4) * 8;  // fragment k offset
        for (int ci = 0; ci < c_in; ci += 32) {
            V a[S::RB];
#pragma unroll
            for (int i = 0; i < S::RB; ++i) {
                const int r = wm * S::TM + i * 16 + fr;
                a[i] = *reinterpret_cast<const V*>(a_tile + r * lds_row + ci + fk);
            }
#pragma unroll
            for (int j = 0; j < S::CB; ++j) {
                const int co = wn * S::TN + j * 16 + fr;
                const V b = bsrc.load(k, co, ci + fk);
#pragma unroll
                for (int i = 0; i < S::RB; ++i) acc[i][j] = MfmaOps<T>::mfma(a[i], b, acc[i][j]);
            }
        }
        __syncthreads();
    }

    // Epilogue: lane holds rows 4*(lane/16)+q of each 16x16 block, column lane%16.
    const int col_in_block = lane & 15;
    const int row_in_block = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < S::RB; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int sr = row0 + wm * S::TM + i * 16 + row_in_block + q;
            if (sr >= rows) continue;
            const long long orow = reorder_rows != nullptr ? reorder_rows[sr] : sr;
#pragma unroll
            for (int j = 0; j < S::CB; ++j) {
                const int co = wn * S::TN + j * 16 + col_in_block;
                Elem<T>::store(out, orow * C_OUT + co, acc[i][j][q]);
            }
        }
    }
}

template <typename T, typename BSource>
int launch_igemm(const T* feats, int c_in, int c_out, const BSource& b, MapView mv, int K,
                 const int32_t* reorder_rows, int rows, T* out, hipStream_t stream) {
    if (rows <= 0) return LATTICE_OK;
    const unsigned tiles = static_cast<unsigned>((rows + kTileRows - 1) / kTileRows);
    const size_t lds = sizeof(T) * kTileRows * (c_in + kLdsPad) + sizeof(int32_t) * kTileRows * K;
    switch (c_out) {
    case 16: conv_igemm<T, 16, BSource><<<tiles, kBlock, lds, stream>>>(feats, c_in, b, mv, K, reorder_rows, rows, out); break;
    case 32: conv_igemm<T, 32, BSource><<<tiles, kBlock, lds, stream>>>(feats, c_in, b, mv, K, reorder_rows, rows, out); break;
    case 64: conv_igemm<T, 64, BSource><<<tiles, kBlock, lds, stream>>>(feats, c_in, b, mv, K, reorder_rows, rows, out); break;
    case 128: conv_igemm<T, 128, BSource><<<tiles, kBlock, lds, stream>>>(feats, c_in, b, mv, K, reorder_rows, rows, out); break;
    case 256: conv_igemm<T, 256, BSource><<<tiles, kBlock, lds, stream>>>(feats, c_in, b, mv, K, reorder_rows, rows, out); break;
    default:
        set_error("implicit GEMM supports c_out in {16, 32, 64, 128, 256}.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

bool igemm_shape_ok(int c_in, int c_out, int K) {
    return c_in > 0 && c_in % 32 == 0 && c_in <= 512 && K > 0 && K <= 32 &&
           (c_out == 16 || c_out == 32 || c_out == 64 || c_out == 128 || c_out == 256);
}

int check_dtype(int dtype) {
    LATTICE_REQUIRE(dtype == LATTICE_F32 || dtype == LATTICE_F16 || dtype == LATTICE_BF16,
                    "convolution supports float32, float16 and bfloat16 features.");
    return LATTICE_OK;
}

}  // namespace
}  // namespace lattice

using namespace lattice;

extern "C" int lattice_hip_sparse_conv_features(int dtype, const void* feats, int n_in, int c_in,
                                                const void* weights, int weight_layout, int kernel_count,
                                                int c_out, const int32_t* in_rows, const int32_t* kernel_ids,
                                                const int32_t* counts, int edge_capacity,
                                                const int32_t* row_offsets, int out_capacity, void* out,
                                                void* stream_ptr) {
    int rc = check_dtype(dtype);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(n_in >= 0 && c_in > 0 && c_out > 0, "feats must have shape (N, C_in).");
    LATTICE_REQUIRE(out_capacity >= 0 && kernel_count > 0,
                    "out_capacity must be nonnegative and n_kernels must be positive.");
    LATTICE_REQUIRE(weight_layout == LATTICE_WEIGHT_KERNEL_MAJOR || weight_layout == LATTICE_WEIGHT_DENSE_5D,
                    "weights must have shape (K, C_in, C_out) or (C_out, Kx, Ky, Kz, C_in).");
    LATTICE_REQUIRE(counts && row_offsets && out && weights, "conv pointers must be non-null.");
    if (out_capacity == 0) return LATTICE_OK;
    hipStream_t stream = as_stream(stream_ptr);
    WeightIndex widx{weight_layout, kernel_count, c_in, c_out};
    const long long total = static_cast<long long>(out_capacity) * c_out;
    const unsigned grid = grid_for(total, 256, 1u << 16);
    if (dtype == LATTICE_F32) {
        conv_csr<float><<<grid, 256, 0, stream>>>(static_cast<const float*>(feats), c_in,
                                                  static_cast<const float*>(weights), widx, in_rows, kernel_ids,
                                                  counts, edge_capacity, row_offsets, out_capacity,
                                                  static_cast<float*>(out));
    } else if (dtype == LATTICE_F16) {
        conv_csr<_Float16><<<grid, 256, 0, stream>>>(static_cast<const _Float16*>(feats), c_in,
                                                     static_cast<const _Float16*>(weights), widx, in_rows,
                                                     kernel_ids, counts, edge_capacity, row_offsets, out_capacity,
                                                     static_cast<_Float16*>(out));
    } else {
        conv_csr<__bf16><<<grid, 256, 0, stream>>>(static_cast<const __bf16*>(feats), c_in,
                                                   static_cast<const __bf16*>(weights), widx, in_rows, kernel_ids,
                                                   counts, edge_capacity, row_offsets, out_capacity,
                                                   static_cast<__bf16*>(out));
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_sparse_conv_features_sorted_implicit_gemm(
    int dtype, const void* feats, int n_in, int c_in, const void* weights, int weight_layout, int kernel_count,
    int c_out, const int32_t* sorted_out_in_map, const int32_t* reorder_rows, int out_capacity, void* out,
    void* stream_ptr) {
    int rc = check_dtype(dtype);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(dtype != LATTICE_F32, "the implicit GEMM route runs on fp16/bf16 matrix cores.");
    LATTICE_REQUIRE(n_in >= 0 && out_capacity >= 0, "feats must have shape (N, C_in).");
    LATTICE_REQUIRE(weight_layout == LATTICE_WEIGHT_DENSE_5D,
                    "the implicit GEMM route takes (C_out, Kx, Ky, Kz, C_in) weights.");
    if (!igemm_shape_ok(c_in, c_out, kernel_count)) {
        set_error("implicit GEMM needs c_in % 32 == 0, c_out in {16,32,64,128,256} and K <= 32.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
    LATTICE_REQUIRE(sorted_out_in_map && out && weights && (feats || n_in == 0),
                    "conv pointers must be non-null.");
    hipStream_t stream = as_stream(stream_ptr);
    MapView mv{sorted_out_in_map, kernel_count, 1};
    const long long s_co = static_cast<long long>(kernel_count) * c_in;
    const long long s_k = c_in;
    if (dtype == LATTICE_F16) {
        FloatB<_Float16> b{static_cast<const _Float16*>(weights), s_co, s_k};
        return launch_igemm<_Float16>(static_cast<const _Float16*>(feats), c_in, c_out, b, mv, kernel_count,
                                      reorder_rows, out_capacity, static_cast<_Float16*>(out), stream);
    }
    FloatB<__bf16> b{static_cast<const __bf16*>(weights), s_co, s_k};
    return launch_igemm<__bf16>(static_cast<const __bf16*>(feats), c_in, c_out, b, mv, kernel_count, reorder_rows,
                                out_capacity, static_cast<__bf16*>(out), stream);
}

extern "C" int lattice_hip_sparse_quantized_conv_features(
    int dtype, const void* feats, int n_in, int c_in, const uint32_t* weights, const void* scales,
    const void* biases, int kernel_count, int c_out, int storage_c_in, int group_size, int bits,
    const int32_t* in_rows, const int32_t* kernel_ids, const int32_t* counts, int edge_capacity,
    const int32_t* row_offsets, const int32_t* sorted_kv_out_in_map, const int32_t* reorder_rows,
    int out_capacity, void* out, void* stream_ptr) {
    int rc = check_dtype(dtype);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(bits == 4 || bits == 8, "quantized convolution bits must be 4 or 8.");
    LATTICE_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
                    "quantized convolution group_size must be 32, 64, or 128.");
    LATTICE_REQUIRE(c_in > 0 && c_out > 0 && storage_c_in >= c_in && storage_c_in % group_size == 0,
                    "quantized convolution channel metadata is invalid.");
    LATTICE_REQUIRE(out_capacity >= 0 && kernel_count > 0,
                    "out_capacity must be nonnegative and n_kernels must be positive.");
    LATTICE_REQUIRE(weights && scales && biases && out, "quantized conv pointers must be non-null.");
    if (out_capacity == 0) return LATTICE_OK;
    hipStream_t stream = as_stream(stream_ptr);
    const int packed_words = storage_c_in * bits / 32;
    const int groups = storage_c_in / group_size;
    const bool sorted = sorted_kv_out_in_map != nullptr && reorder_rows != nullptr;
    if (sorted && dtype != LATTICE_F32 && igemm_shape_ok(c_in, c_out, kernel_count)) {
        MapView mv{sorted_kv_out_in_map, 1, out_capacity};
        if (dtype == LATTICE_F16) {
            PackedB<_Float16> b{weights, static_cast<const _Float16*>(scales), static_cast<const _Float16*>(biases),
                                packed_words, groups, group_size, c_out, bits};
            return launch_igemm<_Float16>(static_cast<const _Float16*>(feats), c_in, c_out, b, mv, kernel_count,
                                          reorder_rows, out_capacity, static_cast<_Float16*>(out), stream);
        }
        PackedB<__bf16> b{weights, static_cast<const __bf16*>(scales), static_cast<const __bf16*>(biases),
                          packed_words, groups, group_size, c_out, bits};
        return launch_igemm<__bf16>(static_cast<const __bf16*>(feats), c_in, c_out, b, mv, kernel_count,
                                    reorder_rows, out_capacity, static_cast<__bf16*>(out), stream);
    }
    LATTICE_REQUIRE(in_rows && kernel_ids && counts && row_offsets, "relation pointers must be non-null.");
    QuantIndex q{kernel_count, c_in, c_out, packed_words, groups, group_size, bits};
    const unsigned grid = grid_for(static_cast<long long>(out_capacity) * c_out, 256, 1u << 16);
    if (dtype == LATTICE_F32) {
        quant_conv_csr<float><<<grid, 256, 0, stream>>>(
            static_cast<const float*>(feats), weights, static_cast<const float*>(scales),
            static_cast<const float*>(biases), q, in_rows, kernel_ids, counts, edge_capacity, row_offsets,
            out_capacity, static_cast<float*>(out));
    } else if (dtype == LATTICE_F16) {
        quant_conv_csr<_Float16><<<grid, 256, 0, stream>>>(
            static_cast<const _Float16*>(feats), weights, static_cast<const _Float16*>(scales),
            static_cast<const _Float16*>(biases), q, in_rows, kernel_ids, counts, edge_capacity, row_offsets,
            out_capacity, static_cast<_Float16*>(out));
    } else {
        quant_conv_csr<__bf16><<<grid, 256, 0, stream>>>(
            static_cast<const __bf16*>(feats), weights, static_cast<const __bf16*>(scales),
            static_cast<const __bf16*>(biases), q, in_rows, kernel_ids, counts, edge_capacity, row_offsets,
            out_capacity, static_cast<__bf16*>(out));
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}
