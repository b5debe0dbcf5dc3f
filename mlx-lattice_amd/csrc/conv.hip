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
#include <atomic>
#include <climits>
#include <mutex>
#include <string>
#include <type_traits>

#include "lattice_common.h"
#include "scan.h"



namespace lattice {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Cache-policy operand of the raw buffer stores that write conv outputs:
// non-temporal (the output is streamed past the caches; it is not read
// again by the kernel that writes it).
constexpr int kNonTemporal = 2;

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

// Store-side epilogue shared by every conv route.  The conv result is
// rounded to T; the optional bias is then added and the sum rounded again,
// exactly as `feats + bias` over the stored output computes it
// (ops/conv.py:460-469); the optional ReLU then keeps v where v > 0 or v is
// NaN and stores +0 otherwise, the reference's `maximum(feats, 0)`
// (ops/feature.py:54-56) applied to the stored value.
template <typename T> struct Epilogue {
    const T* bias;  // [c_out] in T, or null
    bool relu;
    // Stored value of output channel co for the fp32 sum acc.
    __device__ inline T apply(float acc, int co) const {
        return finish(acc, bias != nullptr ? Elem<T>::load(bias, co) : 0.0f);
    }
    // The same with the channel's bias value already loaded (b is unused
    // when there is no bias).
    __device__ inline T finish(float acc, float b) const {
        T v = static_cast<T>(acc);
        if (bias != nullptr) v = static_cast<T>(static_cast<float>(v) + b);
        if (relu) {
            const float f = static_cast<float>(v);
            if (!(f > 0.0f) && f == f) v = static_cast<T>(0.0f);
        }
        return v;
    }
    // The epilogue of output channels co0 .. (a column slice of the output).
    __host__ __device__ Epilogue shifted(int co0) const { return Epilogue{bias != nullptr ? bias + co0 : nullptr, relu}; }
};

template <typename T> Epilogue<T> epilogue_of(const void* bias, int flags) {
    return Epilogue<T>{static_cast<const T*>(bias), (flags & LATTICE_EPILOGUE_RELU) != 0};
}

template <typename T>
__device__ inline void store_out(T* out, long long i, float acc, const Epilogue<T>& epi, int co) {
    out[i] = epi.apply(acc, co);
}

// ------------------------------------------------------------- CSR route --

struct WeightIndex {
    int layout;  // LATTICE_WEIGHT_*
    int K, c_in, c_out;
    __device__ inline long long operator()(int k, int ci, int co) const {
        if (layout == LATTICE_WEIGHT_KERNEL_MAJOR) return (static_cast<long long>(k) * c_in + ci) * c_out + co;
        return (static_cast<long long>(co) * K + k) * c_in + ci;
    }
};

// Weights of at most kCsrLdsFloats floats are staged once per block in LDS
// as float32, (k, ci, co) with co fastest, so the lanes of a row read
// consecutive banks; the launch then caps the grid so each block walks many
// rows.  Larger weights are read from global memory at each use.
constexpr int kCsrLdsFloats = 16384;
constexpr unsigned kCsrStagedBlocks = 2048;

template <typename T>
__global__ void __launch_bounds__(256)
conv_csr(const T* __restrict__ feats, int c_in, const T* __restrict__ weights, WeightIndex widx,
         const int32_t* __restrict__ in_rows, const int32_t* __restrict__ kernel_ids,
         const int32_t* __restrict__ counts, int edge_capacity, const int32_t* __restrict__ row_offsets,
         int out_capacity, T* __restrict__ out, Epilogue<T> epi, bool staged) {
    extern __shared__ float wlds[];
    const int c_out = widx.c_out;
    if (staged) {
        const int nw = widx.K * c_in * c_out;
        for (int i = threadIdx.x; i < nw; i += blockDim.x) {
            const int co = i % c_out;
            const int kc = i / c_out;
            wlds[i] = Elem<T>::load(weights, widx(kc / c_in, kc % c_in, co));
        }
        __syncthreads();
    }
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
                if (staged) {
                    const float* wk = wlds + static_cast<long long>(k) * c_in * c_out + co;
                    for (int ci = 0; ci < c_in; ++ci) acc += Elem<T>::load(f, ci) * wk[ci * c_out];
                } else {
                    for (int ci = 0; ci < c_in; ++ci) {
                        acc += Elem<T>::load(f, ci) * Elem<T>::load(weights, widx(k, ci, co));
                    }
                }
            }
        }
        store_out(out, t, acc, epi, co);
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
               const int32_t* __restrict__ row_offsets, int out_capacity, T* __restrict__ out,
               Epilogue<T> epi, bool staged) {
    extern __shared__ float wlds[];
    if (staged) {
        const int nw = q.K * q.c_in * q.c_out;
        for (int i = threadIdx.x; i < nw; i += blockDim.x) {
            const int co = i % q.c_out;
            const int kc = i / q.c_out;
            wlds[i] = dequant(weights, scales, biases, q, kc / q.c_in, kc % q.c_in, co);
        }
        __syncthreads();
    }
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
                if (staged) {
                    const float* wk = wlds + static_cast<long long>(k) * q.c_in * q.c_out + co;
                    for (int ci = 0; ci < q.c_in; ++ci) acc += Elem<T>::load(f, ci) * wk[ci * q.c_out];
                } else {
                    for (int ci = 0; ci < q.c_in; ++ci) {
                        acc += Elem<T>::load(f, ci) * dequant(weights, scales, biases, q, k, ci, co);
                    }
                }
            }
        }
        store_out(out, t, acc, epi, co);
    }
}

// Row-per-lane CSR conv for tiny channel counts (c_in <= 16, c_out 16 or
// 32, weights staged in LDS, e.g. a 4 -> 32 stem): one lane walks one
// output row's edges once and accumulates all c_out channels in registers,
// so the dependent loads of an edge (row offsets, edge row and offset,
// feature row) are paid once per row instead of once per (row, channel).
// Each channel still sums its edges in CSR order and its input channels in
// order with an fp32 accumulator, as the per-channel kernels do.
// QUANT: the staged weight is dequantised from the packed layout.
template <typename T, int CO, bool QUANT>
__global__ void __launch_bounds__(256)
conv_csr_rows(const T* __restrict__ feats, int c_in, const T* __restrict__ fweights, WeightIndex widx,
              const uint32_t* __restrict__ qweights, const T* __restrict__ scales, const T* __restrict__ qbiases,
              QuantIndex q, const int32_t* __restrict__ in_rows, const int32_t* __restrict__ kernel_ids,
              const int32_t* __restrict__ counts, int edge_capacity, const int32_t* __restrict__ row_offsets,
              int out_capacity, T* __restrict__ out, Epilogue<T> epi) {
    // (k, ci, co) with co fastest; each offset's slice is padded by 4 floats
    // so the lanes of a wave, which read different offsets, spread over the
    // LDS banks (16-byte reads).
    extern __shared__ float wlds[];
    const int K = QUANT ? q.K : widx.K;
    const int kstride = c_in * CO + 4;
    const int nw = K * c_in * CO;
    for (int i = threadIdx.x; i < nw; i += blockDim.x) {
        const int co = i % CO;
        const int kc = i / CO;
        const int k = kc / c_in;
        const int ci = kc - k * c_in;
        wlds[k * kstride + ci * CO + co] = QUANT ? dequant(qweights, scales, qbiases, q, k, ci, co)
                                                 : Elem<T>::load(fweights, widx(k, ci, co));
    }
    __syncthreads();
    const int E = min(counts[0], edge_capacity);
    const int n_out = min(counts[1], out_capacity);
    for (int row = blockIdx.x * blockDim.x + threadIdx.x; row < out_capacity; row += gridDim.x * blockDim.x) {
        float acc[CO];
#pragma unroll
        for (int co = 0; co < CO; ++co) acc[co] = 0.0f;
        if (row < n_out) {
            const int e_end = row_offsets[row + 1];
            for (int e = row_offsets[row]; e < e_end; ++e) {
                if (e < 0 || e >= E) continue;
                const int in = in_rows[e];
                const int k = kernel_ids[e];
                if (in < 0 || k < 0 || k >= K) continue;
                const T* f = feats + static_cast<long long>(in) * c_in;
                const float4* wk = reinterpret_cast<const float4*>(wlds + k * kstride);
                for (int ci = 0; ci < c_in; ++ci) {
                    const float x = Elem<T>::load(f, ci);
#pragma unroll
                    for (int c4 = 0; c4 < CO / 4; ++c4) {
                        const float4 w = wk[ci * (CO / 4) + c4];
                        acc[4 * c4 + 0] += x * w.x;
                        acc[4 * c4 + 1] += x * w.y;
                        acc[4 * c4 + 2] += x * w.z;
                        acc[4 * c4 + 3] += x * w.w;
                    }
                }
            }
        }
        // the row's CO outputs as whole 16-byte stores
        T vals[CO];
#pragma unroll
        for (int co = 0; co < CO; ++co) {
            vals[co] = epi.apply(acc[co], co);
        }
        uint4* dst = reinterpret_cast<uint4*>(out + static_cast<long long>(row) * CO);
#pragma unroll
        for (int j = 0; j < static_cast<int>(CO * sizeof(T) / 16); ++j) dst[j] = reinterpret_cast<const uint4*>(vals)[j];
    }
}

// Whether the row-per-lane kernel takes the shape (weights staged).
inline bool csr_rows_ok(int c_in, int c_out, long long nw) {
    return nw <= kCsrLdsFloats && c_in <= 16 && (c_out == 16 || c_out == 32);
}

// ------------------------------------------------------ implicit GEMM ----
//
// Block = WAVES waves.  Each wave owns WAVE_ROWS consecutive rows of the
// mask-sorted order and WAVE_COLS = min(C_OUT, 128) output channels; its
// fp32 accumulators stay in registers for the whole kernel.  The pipeline
// walks stages s = (k, 128-channel chunk of C_in) over the offsets any row
// of the block uses.  During stage s a wave
//   * issues the row indices of stage s+DEPTH+1 (k-major map: one
//     contiguous run of rows per offset),
//   * issues the loads of B(s+1) = W[k][:, chunk] into registers,
//   * issues the gather of A(s+DEPTH) (16 bytes per lane per 32-channel
//     step, straight into MFMA operand registers),
//   * runs the MFMAs of stage s on A(s), loaded DEPTH stages earlier, and
//     on B(s) from LDS, skipping offsets that none of its rows uses,
//   * stores B(s+1) into the other LDS buffer, then meets the block at a
//     barrier.
// With IgemmShape::ALDS (the default for 32..128 output channels) the A
// gather of stage s+1 instead covers whole 128-byte row lines and goes
// through a per-wave LDS buffer (see igemm_stage_alds): half the cache lines
// per load instruction, which the vector-memory path is bound by.
// Every load is an ordinary load the compiler tracks, so it waits only for
// the operands each step uses and the gathers of DEPTH stages stay in flight
// across the MFMAs.  Missing rows (map entry -1) load row 0 and are zeroed
// at use, so every lane issues the same loads.  The epilogue stages the tile
// through LDS and writes whole output rows (16 bytes per lane) to
// out[reorder_rows[row]].


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

// Tile and pipeline shape of the matrix-core kernel.
//   C_OUT      output channels (the block covers all of them);
//   WAVE_ROWS  sorted rows per wave (16-row MFMA blocks: RB = WAVE_ROWS/16);
//   WAVES      waves per block;
//   CHUNK      input channels per stage (64 or 128);
//   DEPTH      stages of A gathers in flight ahead of the computing stage;
//   BPIPE      read the B fragments of the next 32-channel step from LDS
//              while the current step's MFMAs run;
//   OCC        blocks per CU the register allocation must allow;
//   WCOLS      output channels per wave (at most 128).
template <int C_OUT_, int WAVE_ROWS_, int WAVES_, int CHUNK_ = 128, int DEPTH_ = 1, bool BPIPE_ = false,
          int OCC_ = (WAVE_ROWS_ == 32 ? 2 : 1), int WCOLS_ = 128, bool WSKIP_ = false, bool ALDS_ = false>
struct IgemmShape {
    // ALDS: gather A in whole 128-byte lines (8 rows x 64 channels per
    // load) into a per-wave LDS buffer and read the MFMA fragments from
    // there; needs 64-channel stages and one stage of prefetch.
    static constexpr bool ALDS = ALDS_;
    static constexpr int A_LDS = WAVES_ * WAVE_ROWS_ * 64;  // halves, when ALDS
    static constexpr bool WSKIP = WSKIP_;  // gather A only for offsets the wave's own rows use
    static constexpr int OCC = OCC_;
    static constexpr int C_OUT = C_OUT_;
    static constexpr int WAVE_ROWS = WAVE_ROWS_;
    static constexpr int WAVES = WAVES_;
    static constexpr int CHUNK = CHUNK_;
    static constexpr int DEPTH = DEPTH_;
    static constexpr bool BPIPE = BPIPE_;
    static constexpr int WAVE_COLS = C_OUT < WCOLS_ ? C_OUT : WCOLS_;
    static constexpr int THREADS = WAVES * 64;
    static constexpr int CG = C_OUT / WAVE_COLS;  // column groups
    static constexpr int RG = WAVES / CG;         // row groups
    static constexpr int BLOCK_ROWS = WAVE_ROWS * RG;
    static constexpr int CB = WAVE_COLS / 16;     // 16-col blocks per wave
    static constexpr int RB = WAVE_ROWS / 16;     // 16-row blocks per wave
    static constexpr int ST = CHUNK / 32;         // 32-channel steps per stage
    static constexpr int NA = DEPTH + 1;          // A register buffers
    // Unrolled stages per loop trip: a multiple of the two B buffers and
    // of the NA A buffers, so every buffer is a compile-time choice, and
    // long enough that most blocks never take the loop back-edge (where the
    // compiler's wait bookkeeping turns conservative and drains all loads).
    static constexpr int UNROLL = NA == 3 ? 12 : 16;
    static_assert(UNROLL % 2 == 0 && UNROLL % NA == 0, "unroll must cycle every buffer");
    // Staged B: C_OUT rows of CHUNK halves (PIECES 16-byte pieces); piece p
    // of row r lives at slot p ^ (r % PIECES), so the rows read by one MFMA
    // fragment hit distinct bank groups.
    static constexpr int PIECES = CHUNK / 8;
    static constexpr int BROW = CHUNK;
    static constexpr int BBUF = C_OUT * BROW;     // one B buffer (halves)
    static constexpr int EROW = WAVE_COLS;        // epilogue row (halves, swizzled pieces)
    static constexpr int EPIECES = WAVE_COLS / 8;  // 16-byte pieces per epilogue row
    static constexpr int B_PIECES = C_OUT * CHUNK / 8 / THREADS;  // 16-byte pieces per thread
    static constexpr int MAX_STAGES = 32 * (512 / CHUNK);  // K <= 32 offsets x C_in <= 512
    static_assert(CHUNK == 64 || CHUNK == 128, "stage chunk is 64 or 128 channels");
    static_assert(!ALDS_ || (CHUNK_ == 64 && DEPTH_ == 1 && WAVE_ROWS_ % 16 == 0), "ALDS shape");
    static_assert(B_PIECES >= 1, "B tile must cover every thread");
    // One LDS array holds the two B buffers and, after the main loop, the
    // epilogue staging of every wave's tile.
    static constexpr int EPI = WAVES * WAVE_ROWS * EROW;
    // The ALDS A buffers follow the two B buffers; the epilogue reuses all.
    static constexpr int MAIN_HALVES = 2 * BBUF + (ALDS_ ? A_LDS : 0);
    static constexpr int LDS_HALVES = MAIN_HALVES > EPI ? MAIN_HALVES : EPI;
};

template <int PIECES>
__device__ inline int swizzle_piece(int piece, int row) { return piece ^ (row & (PIECES - 1)); }

// B operand sources.  `load(k, co, ci0)` returns 8 consecutive input
// channels ci0..ci0+7 of W[k][:, co] as one 16-byte vector.
template <typename T> struct FloatB {
    static constexpr bool kCoFastest = false;  // C_in is contiguous: 8 lanes read one row's 128 bytes
    const T* w;
    long long s_co, s_k;  // element strides; C_in is contiguous
    __device__ inline typename MfmaOps<T>::vec load(int k, int co, int ci0) const {
        return *reinterpret_cast<const typename MfmaOps<T>::vec*>(w + co * s_co + k * s_k + ci0);
    }
};

// fp16 dequantisation of packed codes with packed half math: a code c
// (0..255) placed in the low byte of the half 0x6400 reads as 1024 + c, so
// subtracting 1024 recovers c exactly; then one fused c * scale + bias per
// half pair (one rounding, to fp16, the MFMA operand's type).
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ inline half2_t code_pair(uint32_t bits) {
    const half2_t biased = __builtin_bit_cast(half2_t, bits | 0x64006400u);
    return biased - half2_t{static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
}

__device__ inline half2_t affine_pair(half2_t c, half2_t s, half2_t b) { return __builtin_elementwise_fma(c, s, b); }

// Packed affine codes: w = q * scale + bias, dequantised while staging B.
template <typename T> struct PackedB {
    // C_out is contiguous in the packed words, scales and biases: lanes take
    // consecutive output channels so each of their loads is one coalesced run.
    static constexpr bool kCoFastest = true;
    const uint32_t* w;
    const T* scales;
    const T* biases;
    int packed_words, groups, group_size, c_out, bits;
    __device__ inline typename MfmaOps<T>::vec load(int k, int co, int ci0) const {
        typename MfmaOps<T>::vec out;
        const long long s = (static_cast<long long>(k) * groups + ci0 / group_size) * c_out + co;
        const long long wbase = static_cast<long long>(k) * packed_words * c_out + co;
        if constexpr (std::is_same<T, _Float16>::value) {
            const half2_t sc = {scales[s], scales[s]};
            const half2_t bi = {biases[s], biases[s]};
            if (bits == 4) {
                // nibble j of the word is code j: pairs (j, j + 4)
                const uint32_t word = w[wbase + static_cast<long long>(ci0 >> 3) * c_out];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const half2_t r = affine_pair(code_pair((word >> (4 * j)) & 0x000F000Fu), sc, bi);
                    out[j] = r[0];
                    out[j + 4] = r[1];
                }
            } else {
                // byte j of word i is code 4i + j: pairs (4i + j, 4i + j + 2)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t word = w[wbase + static_cast<long long>((ci0 >> 2) + i) * c_out];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const half2_t r = affine_pair(code_pair((word >> (8 * j)) & 0x00FF00FFu), sc, bi);
                        out[4 * i + j] = r[0];
                        out[4 * i + j + 2] = r[1];
                    }
                }
            }
            return out;
        } else {
            const float sc = Elem<T>::load(scales, s);
            const float bi = Elem<T>::load(biases, s);
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
    }

    // The raw words, scales and biases of output channels co .. co + N - 1
    // (co a multiple of N) for input channels ci0 .. ci0 + 7: one N-word
    // load per word row and N-half loads of the scales and biases.  They are
    // loaded when a stage starts and dequantised when it stores its B tile,
    // so no wait for them sits before the stage's gathers and MFMAs.
    template <int N> struct Raw {
        using W = typename std::conditional<N == 4, uint4, uint2>::type;
        using H = typename std::conditional<N == 4, uint2, uint32_t>::type;
        W w0, w1;  // w1: the second word row of 8-bit codes
        H s, b;
    };
    template <int N>
    __device__ inline void load_raw_n(int k, int co, int ci0, Raw<N>& r) const {
        static_assert(N == 2 || N == 4, "two or four output channels per thread");
        using W = typename Raw<N>::W;
        using H = typename Raw<N>::H;
        const long long s = (static_cast<long long>(k) * groups + ci0 / group_size) * c_out + co;
        const long long wbase = static_cast<long long>(k) * packed_words * c_out + co;
        r.s = *reinterpret_cast<const H*>(scales + s);
        r.b = *reinterpret_cast<const H*>(biases + s);
        // Both word rows are loaded unconditionally (4-bit codes reread the
        // first and ignore the second): a branch here would leave a load
        // of one path pending into the other's registers, and the wait for
        // it would drain every load in flight.
        const int row0 = bits == 4 ? (ci0 >> 3) : (ci0 >> 2);
        const int row1 = bits == 4 ? row0 : row0 + 1;
        r.w0 = *reinterpret_cast<const W*>(w + wbase + static_cast<long long>(row0) * c_out);
        r.w1 = *reinterpret_cast<const W*>(w + wbase + static_cast<long long>(row1) * c_out);
    }
    template <int N>
    __device__ inline void dequant_n(const Raw<N>& r, typename MfmaOps<T>::vec (&out)[N]) const {
        const T* sv = reinterpret_cast<const T*>(&r.s);
        const T* bv = reinterpret_cast<const T*>(&r.b);
        if (bits == 4) {
            const uint32_t* words = reinterpret_cast<const uint32_t*>(&r.w0);
#pragma unroll
            for (int c = 0; c < N; ++c) {
                if constexpr (std::is_same<T, _Float16>::value) {
                    const half2_t sc = {sv[c], sv[c]};
                    const half2_t bi = {bv[c], bv[c]};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const half2_t h = affine_pair(code_pair((words[c] >> (4 * j)) & 0x000F000Fu), sc, bi);
                        out[c][j] = h[0];
                        out[c][j + 4] = h[1];
                    }
                } else {
                    const float sc = static_cast<float>(sv[c]);
                    const float bi = static_cast<float>(bv[c]);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        out[c][j] = static_cast<T>(static_cast<float>((words[c] >> (4 * j)) & 15u) * sc + bi);
                    }
                }
            }
        } else {
            const uint32_t* lo = reinterpret_cast<const uint32_t*>(&r.w0);
            const uint32_t* hi = reinterpret_cast<const uint32_t*>(&r.w1);
#pragma unroll
            for (int c = 0; c < N; ++c) {
                if constexpr (std::is_same<T, _Float16>::value) {
                    const half2_t sc = {sv[c], sv[c]};
                    const half2_t bi = {bv[c], bv[c]};
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const half2_t a = affine_pair(code_pair((lo[c] >> (8 * j)) & 0x00FF00FFu), sc, bi);
                        const half2_t b = affine_pair(code_pair((hi[c] >> (8 * j)) & 0x00FF00FFu), sc, bi);
                        out[c][j] = a[0];
                        out[c][j + 2] = a[1];
                        out[c][4 + j] = b[0];
                        out[c][4 + j + 2] = b[1];
                    }
                } else {
                    const float sc = static_cast<float>(sv[c]);
                    const float bi = static_cast<float>(bv[c]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        out[c][j] = static_cast<T>(static_cast<float>((lo[c] >> (8 * j)) & 255u) * sc + bi);
                        out[c][4 + j] = static_cast<T>(static_cast<float>((hi[c] >> (8 * j)) & 255u) * sc + bi);
                    }
                }
            }
        }
    }
};

// Row indices of this wave's A operand for offset k: rows row0 + 16*rb +
// lane%16 of the sorted order; -1 where there is no input row.  Rows past
// the end re-read the last row; their result is never stored.
template <int RB>
__device__ inline void load_rows(int (&idx)[RB], const int32_t* __restrict__ kv_map, int rows, int row0, int k,
                                 int lr) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = min(row0 + rb * 16 + lr, rows - 1);
        idx[rb] = kv_map[static_cast<long long>(k) * rows + r];
    }
}

// Feature rows as a raw buffer of n_in * c_in elements (under 2 GiB, which
// the route check enforces).  A row address is a 32-bit byte offset; the
// buffer's range check returns zeros past the end, and a missing input row
// (map entry -1) wraps to an offset past the end, so it reads as zeros with
// no select at use.
template <typename T>
__device__ inline __amdgpu_buffer_rsrc_t feature_rows(const T* feats, int n_in, int c_in) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(feats), 0,
                                             static_cast<int>(static_cast<long long>(n_in) * c_in * sizeof(T)),
                                             0x00020000);
}

// A operand of one stage: RB x ST fragments of 16 bytes per lane (channels
// ci_base + 32*st + 8*(lane/16) .. +7).  Every lane issues the same loads
// (steps past the chunk re-read its first step).
template <typename T, typename V, int RB, int ST>
__device__ inline void load_a(V (&a)[RB][ST], const int (&idx)[RB], __amdgpu_buffer_rsrc_t rows_rsrc, int c_in,
                              int ci_base, int cw, int lk) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const unsigned row = static_cast<unsigned>(idx[rb]) * static_cast<unsigned>(c_in * sizeof(T));
#pragma unroll
        for (int st = 0; st < ST; ++st) {
            const int off = st * 32 < cw ? st * 32 : 0;
            a[rb][st] = __builtin_bit_cast(
                V, __builtin_amdgcn_raw_buffer_load_b128(
                       rows_rsrc, static_cast<int>(row + (ci_base + lk + off) * sizeof(T)), 0, 0));
        }
    }
}

// Register staging of one B tile: thread t holds pieces t + i*THREADS.
// Float weights (C_in contiguous) map a piece to row co = p / PIECES, so a
// wave reads whole rows; packed weights (C_out contiguous) map consecutive
// threads to consecutive output channels.
template <typename S, bool CO_FASTEST>
__device__ inline void b_piece(int p, int& co, int& piece) {
    if (CO_FASTEST) {
        piece = p / S::C_OUT;
        co = p - piece * S::C_OUT;
    } else {
        co = p / S::PIECES;
        piece = p - co * S::PIECES;
    }
}

// Packed weights whose tile gives every thread two or four pieces: thread
// t takes the N consecutive output channels N * (t % (C_OUT / N)) .. + N - 1
// at piece t / (C_OUT / N) and loads them with one N-word load per word row
// (load_n).
template <typename S, typename BSource>
struct MultiB {
    static constexpr int N = S::B_PIECES;
    static constexpr bool value = BSource::kCoFastest && (N == 2 || N == 4) && S::C_OUT % N == 0 &&
                                  S::C_OUT * S::PIECES == N * S::THREADS;
};

template <typename T, typename S, typename BSource, typename V>
__device__ inline void stage_b_load(const BSource& bsrc, int k, int ci0, int cw, V (&breg)[S::B_PIECES]) {
    if constexpr (MultiB<S, BSource>::value) {
        // raw codes, scales and biases, kept in breg's registers until the
        // stage stores its B tile
        constexpr int N = MultiB<S, BSource>::N;
        using Raw = typename BSource::template Raw<N>;
        static_assert(sizeof(Raw) <= sizeof(breg), "the raw words fit the staged pieces");
        const int co = N * (threadIdx.x % (S::C_OUT / N));
        const int piece = threadIdx.x / (S::C_OUT / N);
        Raw raw;
        bsrc.template load_raw_n<N>(k, co, ci0 + (piece * 8 < cw ? piece * 8 : 0), raw);
        __builtin_memcpy(&breg[0], &raw, sizeof(Raw));
    } else {
#pragma unroll
        for (int i = 0; i < S::B_PIECES; ++i) {
            int co, piece;
            b_piece<S, BSource::kCoFastest>(threadIdx.x + i * S::THREADS, co, piece);
            breg[i] = bsrc.load(k, co, ci0 + (piece * 8 < cw ? piece * 8 : 0));
        }
    }
}

template <typename T, typename S, typename BSource, typename V>
__device__ inline void stage_b_store(T* dst, const V (&breg)[S::B_PIECES], const BSource& bsrc) {
    if constexpr (MultiB<S, BSource>::value) {
        constexpr int N = MultiB<S, BSource>::N;
        using Raw = typename BSource::template Raw<N>;
        Raw raw;
        __builtin_memcpy(&raw, &breg[0], sizeof(Raw));
        V vals[N];
        bsrc.template dequant_n<N>(raw, vals);
        const int co0 = N * (threadIdx.x % (S::C_OUT / N));
        const int piece = threadIdx.x / (S::C_OUT / N);
#pragma unroll
        for (int c = 0; c < N; ++c) {
            const int co = co0 + c;
            *reinterpret_cast<V*>(dst + co * S::BROW + swizzle_piece<S::PIECES>(piece, co) * 8) = vals[c];
        }
    } else {
#pragma unroll
        for (int i = 0; i < S::B_PIECES; ++i) {
            int co, piece;
            b_piece<S, BSource::kCoFastest>(threadIdx.x + i * S::THREADS, co, piece);
            *reinterpret_cast<V*>(dst + co * S::BROW + swizzle_piece<S::PIECES>(piece, co) * 8) = breg[i];
        }
    }
}

template <typename T, typename S, typename V>
__device__ inline void read_b_step(V (&b)[S::CB], const T* brow, int st, int lane, int lr) {
    const T* bp = brow + swizzle_piece<S::PIECES>(st * 4 + (lane >> 4), lr) * 8;
#pragma unroll
    for (int cb = 0; cb < S::CB; ++cb) b[cb] = *reinterpret_cast<const V*>(bp + cb * 16 * S::BROW);
}

template <typename T, typename S, typename V>
__device__ inline void mfma_step(float4_t (&acc)[S::RB][S::CB], const V (&a)[S::RB][S::ST], const V (&b)[S::CB],
                                 int st) {
#pragma unroll
    for (int cb = 0; cb < S::CB; ++cb) {
#pragma unroll
        for (int rb = 0; rb < S::RB; ++rb) acc[rb][cb] = MfmaOps<T>::mfma(a[rb][st], b[cb], acc[rb][cb]);
    }
}

// Per-wave pipeline state shared by the stages of one block.
struct StageCtx {
    const unsigned char* stage_k;
    const unsigned char* stage_chunk;
    int nstages, c_in, rows, row0, wc, lane;
    uint32_t wmask;
};

// Stage s.  `a_use` holds A(s); `idx_a` holds the row indices of stage
// s+DEPTH, whose gather goes to `a_fill`; `idx_fill` receives the indices
// of stage s+DEPTH+1.
template <typename T, typename S, typename BSource, typename V>
__device__ inline void igemm_stage(int s, const StageCtx& c, const T* bcur, T* bnext,
                                   __amdgpu_buffer_rsrc_t rows_rsrc, const BSource& bsrc,
                                   const int32_t* __restrict__ kv_map, const int (&idx_a)[S::RB],
                                   int (&idx_fill)[S::RB], const V (&a_use)[S::RB][S::ST], V (&a_fill)[S::RB][S::ST],
                                   float4_t (&acc)[S::RB][S::CB]) {
    const int lr = c.lane & 15;
    const int lk = (c.lane >> 4) * 8;
    const int last = c.nstages - 1;
    const int sb = min(s + 1, last);
    const int sa = min(s + S::DEPTH, last);
    const int si = min(s + S::DEPTH + 1, last);
    if (!S::WSKIP || ((c.wmask >> c.stage_k[si]) & 1u)) {
        load_rows<S::RB>(idx_fill, kv_map, c.rows, c.row0, c.stage_k[si], lr);
    }
    V breg[S::B_PIECES];
    const int cib = c.stage_chunk[sb] * S::CHUNK;
    stage_b_load<T, S>(bsrc, c.stage_k[sb], cib, min(S::CHUNK, c.c_in - cib), breg);
    if (!S::WSKIP || ((c.wmask >> c.stage_k[sa]) & 1u)) {
        const int cia = c.stage_chunk[sa] * S::CHUNK;
        load_a<T, V, S::RB, S::ST>(a_fill, idx_a, rows_rsrc, c.c_in, cia, min(S::CHUNK, c.c_in - cia), lk);
    }

    const int k = c.stage_k[s];
    if ((c.wmask >> k) & 1u) {
        const int nst = min(S::CHUNK, c.c_in - c.stage_chunk[s] * S::CHUNK) / 32;
        // Rows wc*WAVE_COLS + 16*cb + lr all share lr's low bits, so piece
        // 4*st + lane/16 sits in the same slot for every column block.
        const T* brow = bcur + (c.wc * S::WAVE_COLS + lr) * S::BROW;
        if (S::BPIPE && nst == S::ST) {
            V bf[2][S::CB];
            read_b_step<T, S>(bf[0], brow, 0, c.lane, lr);
#pragma unroll
            for (int st = 0; st < S::ST; ++st) {
                if (st + 1 < S::ST) read_b_step<T, S>(bf[(st + 1) & 1], brow, st + 1, c.lane, lr);
                mfma_step<T, S>(acc, a_use, bf[st & 1], st);
            }
        } else {
#pragma unroll
            for (int st = 0; st < S::ST; ++st) {
                if (st < nst) {
                    V b[S::CB];
                    read_b_step<T, S>(b, brow, st, c.lane, lr);
                    mfma_step<T, S>(acc, a_use, b, st);
                }
            }
        }
    }
    stage_b_store<T, S, BSource>(bnext, breg, bsrc);
    __syncthreads();
}


// ---- line-coalesced A through LDS (IgemmShape::ALDS) ----
//
// A gather instruction covers 8 consecutive rows of the wave tile with 8
// lanes per row, so each of its 16-byte lanes lands in one of 8 whole
// 128-byte lines (one 64-channel fp16 row chunk), instead of 16 rows x 64
// bytes in the MFMA fragment layout.  Lane l loads row 8h + l/8 of each
// 16-row block, piece l%8.  The rows go to this wave's LDS buffer with piece
// p of row r at slot p ^ (r % 8); the MFMA fragment reads (16 rows, one
// piece each) then spread over distinct banks.  Only the wave reads its own
// buffer, so no barrier guards it: LDS operations of one wave complete in
// issue order.

template <int RB>
__device__ inline void load_rows_coal(int (&idx)[RB][2], const int32_t* __restrict__ kv_map, int rows, int row0,
                                      int k, int lane) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = min(row0 + rb * 16 + 8 * h + (lane >> 3), rows - 1);
            idx[rb][h] = kv_map[static_cast<long long>(k) * rows + r];
        }
    }
}

template <typename T, typename V, int RB>
__device__ inline void load_a_coal(V (&a)[RB][2], const int (&idx)[RB][2], __amdgpu_buffer_rsrc_t rows_rsrc,
                                   int c_in, int ci_base, int cw, int lane) {
    const int piece = lane & 7;
    const int off = piece * 8 < cw ? piece * 8 : 0;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const unsigned row = static_cast<unsigned>(idx[rb][h]) * static_cast<unsigned>(c_in * sizeof(T));
            a[rb][h] = __builtin_bit_cast(
                V, __builtin_amdgcn_raw_buffer_load_b128(rows_rsrc, static_cast<int>(row + (ci_base + off) * sizeof(T)),
                                                         0, 0));
        }
    }
}

template <typename T, typename V, int RB>
__device__ inline void store_a_coal(T* abuf, const V (&a)[RB][2], int lane) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = rb * 16 + 8 * h + (lane >> 3);
            *reinterpret_cast<V*>(abuf + r * 64 + ((lane & 7) ^ (r & 7)) * 8) = a[rb][h];
        }
    }
}

// Stage s of the ALDS pipeline.  `idx_a` holds the row indices of stage
// s+1, whose gather is issued here and written to the wave's LDS buffer at
// the end of the stage (after this stage's fragment reads, in issue order);
// `idx_fill` receives the indices of stage s+2.
template <typename T, typename S, typename BSource, typename V>
__device__ inline void igemm_stage_alds(int s, const StageCtx& c, const T* bcur, T* bnext, T* abuf,
                                        __amdgpu_buffer_rsrc_t rows_rsrc, const BSource& bsrc,
                                        const int32_t* __restrict__ kv_map, const int (&idx_a)[S::RB][2],
                                        int (&idx_fill)[S::RB][2], float4_t (&acc)[S::RB][S::CB]) {
    const int lr = c.lane & 15;
    const int last = c.nstages - 1;
    const int sb = min(s + 1, last);
    const int si = min(s + 2, last);
    if (!S::WSKIP || ((c.wmask >> c.stage_k[si]) & 1u)) {
        load_rows_coal<S::RB>(idx_fill, kv_map, c.rows, c.row0, c.stage_k[si], c.lane);
    }
    V breg[S::B_PIECES];
    const int cib = c.stage_chunk[sb] * S::CHUNK;
    stage_b_load<T, S>(bsrc, c.stage_k[sb], cib, min(S::CHUNK, c.c_in - cib), breg);
    V areg[S::RB][2];
    const bool need_a = !S::WSKIP || ((c.wmask >> c.stage_k[sb]) & 1u);
    if (need_a) {
        load_a_coal<T, V, S::RB>(areg, idx_a, rows_rsrc, c.c_in, cib, min(S::CHUNK, c.c_in - cib), c.lane);
    }

    const int k = c.stage_k[s];
    if ((c.wmask >> k) & 1u) {
        const int nst = min(S::CHUNK, c.c_in - c.stage_chunk[s] * S::CHUNK) / 32;
        const T* brow = bcur + (c.wc * S::WAVE_COLS + lr) * S::BROW;
#pragma unroll
        for (int st = 0; st < S::ST; ++st) {
            if (st < nst) {
                V af[S::RB][S::ST];
                const int slot = ((st * 4 + (c.lane >> 4)) ^ (lr & 7)) * 8;
#pragma unroll
                for (int rb = 0; rb < S::RB; ++rb) af[rb][st] = *reinterpret_cast<const V*>(abuf + (rb * 16 + lr) * 64 + slot);
                V b[S::CB];
                read_b_step<T, S>(b, brow, st, c.lane, lr);
                mfma_step<T, S>(acc, af, b, st);
                // Scheduling hint: interleave this step's LDS fragment reads
                // with its MFMAs (measured 6% faster on the 128-column shape).
                __builtin_amdgcn_iglp_opt(1);
            }
        }
    }
    stage_b_store<T, S, BSource>(bnext, breg, bsrc);
    if (need_a) store_a_coal<T, V, S::RB>(abuf, areg, c.lane);
    __syncthreads();
}

// A column half of the weight: output channels co_base .. co_base + 127.
template <typename T> __host__ __device__ FloatB<T> column_half(const FloatB<T>& b, int co_base) {
    FloatB<T> h = b;
    h.w += co_base * b.s_co;
    return h;
}
template <typename T> __host__ __device__ PackedB<T> column_half(const PackedB<T>& b, int co_base) {
    PackedB<T> h = b;  // c_out stays the row stride of the packed arrays
    h.w += co_base;
    h.scales += co_base;
    h.biases += co_base;
    return h;
}

template <typename T, typename S, typename BSource>
__global__ void __launch_bounds__(S::THREADS, S::OCC)
conv_igemm(const T* __restrict__ feats, int n_in, int c_in, BSource bsrc, const int32_t* __restrict__ kv_map,
           const int32_t* __restrict__ tile_masks, const int32_t* __restrict__ reorder_rows, int rows,
           const int32_t* __restrict__ block_order, T* __restrict__ out, Epilogue<T> epi, int out_ld,
           int halves) {
    using V = typename MfmaOps<T>::vec;
    constexpr int WAVES = S::WAVES;
    constexpr int WAVE_ROWS = S::WAVE_ROWS;
    constexpr int C_OUT = S::C_OUT;
    __shared__ __align__(16) T lds[S::LDS_HALVES];
    T* const bbuf0 = lds;
    T* const bbuf1 = lds + S::BBUF;
    __shared__ unsigned char stage_k[S::MAX_STAGES];
    __shared__ unsigned char stage_chunk[S::MAX_STAGES];

    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int wr = wave / S::CG;
    const int wc = wave % S::CG;
    // block_order (optional) lists the row tiles longest-first, so the
    // costliest tiles start early and the launch drains evenly.  With two
    // column halves (C_out = 256) consecutive blocks take the two halves of
    // one tile, so the second gathers rows the first just brought into L2.
    const int slot = halves > 1 ? static_cast<int>(blockIdx.x) / 2 : static_cast<int>(blockIdx.x);
    if (halves > 1 && (blockIdx.x & 1u)) {
        bsrc = column_half(bsrc, C_OUT);
        out += C_OUT;
        epi = epi.shifted(C_OUT);
    }
    const int tile = block_order != nullptr ? block_order[slot] : slot;
    const int block_row0 = tile * S::BLOCK_ROWS;
    const int row0 = block_row0 + wr * WAVE_ROWS;
    const int quarters = ((rows + 63) / 64) * 4;

    // tile_masks holds one OR-mask per 16-row quarter of the sorted order.
    uint32_t wmask = 0;
    uint32_t bmask = 0;
#pragma unroll
    for (int q = 0; q < S::BLOCK_ROWS / 16; ++q) {
        const int idx = block_row0 / 16 + q;
        const uint32_t m = idx < quarters ? static_cast<uint32_t>(tile_masks[idx]) : 0u;
        bmask |= m;
        if (q / S::RB == wr) wmask |= m;
    }
    const int nchunks = (c_in + S::CHUNK - 1) / S::CHUNK;
    const int nstages = __popc(bmask) * nchunks;
    if (threadIdx.x == 0) {
        uint32_t m = bmask;
        int s = 0;
        while (m) {
            const int k = __builtin_ctz(m);
            m &= m - 1;
            for (int ch = 0; ch < nchunks; ++ch, ++s) {
                stage_k[s] = static_cast<unsigned char>(k);
                stage_chunk[s] = static_cast<unsigned char>(ch);
            }
        }
    }

    float4_t acc[S::RB][S::CB];
#pragma unroll
    for (int i = 0; i < S::RB; ++i)
#pragma unroll
        for (int j = 0; j < S::CB; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int lr = lane & 15;
    const int lk = (lane >> 4) * 8;
    __syncthreads();

    if constexpr (S::ALDS) {
        if (nstages > 0) {
            const StageCtx ctx{stage_k, stage_chunk, nstages, c_in, rows, row0, wc, lane, wmask};
            const int last = nstages - 1;
            T* const abuf = lds + 2 * S::BBUF + wave * WAVE_ROWS * 64;
            const __amdgpu_buffer_rsrc_t rows_rsrc = feature_rows(feats, n_in, c_in);
            int idx[2][S::RB][2];
            load_rows_coal<S::RB>(idx[0], kv_map, rows, row0, stage_k[0], lane);
            load_rows_coal<S::RB>(idx[1], kv_map, rows, row0, stage_k[min(1, last)], lane);
            {
                V breg[S::B_PIECES];
                stage_b_load<T, S>(bsrc, stage_k[0], 0, min(S::CHUNK, c_in), breg);
                V areg[S::RB][2];
                load_a_coal<T, V, S::RB>(areg, idx[0], rows_rsrc, c_in, 0, min(S::CHUNK, c_in), lane);
                stage_b_store<T, S, BSource>(bbuf0, breg, bsrc);
                store_a_coal<T, V, S::RB>(abuf, areg, lane);
            }
            __syncthreads();
            // Stage base + j gathers with idx[(j + 1) % 2] (stage s+1) and
            // refills idx[j % 2] with stage s+2.
            for (int base = 0; base < nstages; base += S::UNROLL) {
#pragma unroll
                for (int j = 0; j < S::UNROLL; ++j) {
                    if (base + j >= nstages) break;
                    igemm_stage_alds<T, S, BSource, V>(base + j, ctx, (j & 1) ? bbuf1 : bbuf0,
                                                       (j & 1) ? bbuf0 : bbuf1, abuf, rows_rsrc, bsrc, kv_map,
                                                       idx[(j + 1) & 1], idx[j & 1], acc);
                }
            }
        }
    } else if (nstages > 0) {
        const StageCtx ctx{stage_k, stage_chunk, nstages, c_in, rows, row0, wc, lane, wmask};
        const int last = nstages - 1;
        // Prologue: B(0) in LDS; A(0) .. A(DEPTH-1) gathered; indices of
        // stage DEPTH ready for stage 0 to gather A(DEPTH).
        int idx[S::NA][S::RB];
        V a[S::NA][S::RB][S::ST];
        const __amdgpu_buffer_rsrc_t rows_rsrc = feature_rows(feats, n_in, c_in);
#pragma unroll
        for (int j = 0; j <= S::DEPTH; ++j) load_rows<S::RB>(idx[j], kv_map, rows, row0, stage_k[min(j, last)], lr);
        {
            V breg[S::B_PIECES];
            stage_b_load<T, S>(bsrc, stage_k[0], 0, min(S::CHUNK, c_in), breg);
            stage_b_store<T, S, BSource>(bbuf0, breg, bsrc);
        }
#pragma unroll
        for (int j = 0; j < S::DEPTH; ++j) {
            const int sj = min(j, last);
            const int ci = stage_chunk[sj] * S::CHUNK;
            load_a<T, V, S::RB, S::ST>(a[j], idx[j], rows_rsrc, c_in, ci, min(S::CHUNK, c_in - ci), lk);
        }
        __syncthreads();
        // Stage s = base + j uses A buffer j % NA, gathers into (j + DEPTH) %
        // NA with the indices in idx[(j + DEPTH) % NA], and refills idx[j %
        // NA] with the indices of stage s + DEPTH + 1 (buffer j % NA is free
        // once its gather has been issued).
        for (int base = 0; base < nstages; base += S::UNROLL) {
#pragma unroll
            for (int j = 0; j < S::UNROLL; ++j) {
                if (base + j >= nstages) break;
                const int u = j % S::NA;
                const int f = (j + S::DEPTH) % S::NA;
                igemm_stage<T, S, BSource, V>(base + j, ctx, (j & 1) ? bbuf1 : bbuf0, (j & 1) ? bbuf0 : bbuf1,
                                              rows_rsrc, bsrc, kv_map, idx[f], idx[u], a[u], a[f], acc);
            }
        }
    }
    __syncthreads();

    // Epilogue: stage this wave's tile in LDS (pieces swizzled by row), then
    // write whole rows with 16-byte stores to out[reorder_rows[row]].
    T* stage = lds + wave * WAVE_ROWS * S::EROW;
    // Optional bias, added after the conv result is rounded (as a separate
    // `feats + bias` would): one value per column this lane writes.
    float bcol[S::CB];
#pragma unroll
    for (int cb = 0; cb < S::CB; ++cb) {
        bcol[cb] = epi.bias != nullptr ? static_cast<float>(epi.bias[wc * S::WAVE_COLS + cb * 16 + lr]) : 0.0f;
    }
#pragma unroll
    for (int rb = 0; rb < S::RB; ++rb) {
#pragma unroll
        for (int cb = 0; cb < S::CB; ++cb) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = rb * 16 + (lane >> 4) * 4 + q;
                const int piece = (cb * 16 + lr) / 8;
                const int slot = piece ^ (r % S::EPIECES);
                const T v = epi.finish(acc[rb][cb][q], bcol[cb]);
                stage[r * S::EROW + slot * 8 + (lr & 7)] = v;
            }
        }
    }
    __syncthreads();
    for (int p = lane; p < WAVE_ROWS * S::EPIECES; p += kWave) {
        const int r = p / S::EPIECES;
        const int piece = p - r * S::EPIECES;
        const int sr = row0 + r;
        if (sr < rows) {
            const long long orow = reorder_rows != nullptr ? reorder_rows[sr] : sr;
__builtin_nontemporal_store(*reinterpret_cast<const V*>(stage + r * S::EROW + (piece ^ (r % S::EPIECES)) * 8),
                                        reinterpret_cast<V*>(out + orow * out_ld + wc * S::WAVE_COLS + piece * 8));
        }
    }
}

// --------------------------------------------- streamed implicit GEMM ----
//
// The matrix-core conv for fp16/bf16 features and weights with C_out in
// {64, 128, 256} and C_in <= 256 (a multiple of 32).  A block owns a tile
// of 128 mask-sorted rows and 128 (or 64) output channels; its 4 waves
// split the tile by columns (C_out = 128: every wave owns all 128 rows and
// 32 columns; C_out = 64: 64 rows x 32 columns).  A stage is one
// (offset k, 64-channel chunk) pair that some row of the tile uses.
//
//  * A (the gathered input rows) goes global -> LDS with no register
//    staging: `buffer_load_dwordx4 ... lds` copies whole 128-byte row lines
//    (8 rows x 64 channels per instruction, 32 rows per wave) two stages
//    ahead into a ring of three 16 KB buffers.  Lane l of a copy writes slot
//    l % 8 of its row; the slot holds piece slot ^ (row % 8), so the 16-row
//    MFMA fragment reads hit distinct banks.  A missing row (map entry -1)
//    wraps past the buffer's range and reads as zeros.
//  * B never passes through LDS: each wave loads its own fragments (its 32
//    columns x 64 channels, four 1 KB runs) from a fragment-ordered copy of
//    the weight (lattice_hip_conv_weight_fragments), two stages ahead.
//  * LDS therefore carries only A: per 16x16x32 MFMA, the 1 KB A fragment
//    is read once for two column blocks (512 B) plus a 128 B share of the
//    copy, 640 B in all, against 896 B when four waves each read a shared
//    B tile (the register-staged kernel above).
//  * v_mfma_f32_16x16x32 runs the transposed product (B fragment as the
//    first operand), so each lane accumulates 4 consecutive output channels
//    of one row and the results leave as 8-byte stores straight from
//    registers to out[reorder_rows[row]].  16-row blocks whose rows do not
//    use k skip their MFMAs.
//
// The main loop's memory instructions are inline assembly issued in a
// fixed order per stage (row indices of stage s + 3, B(s + 2), the copy of
// A(s + 2)), spread over the stage's 16-row blocks, and the loop waits on
// the vector-memory counter itself: loads complete in issue order, so "at
// most N younger loads outstanding" names exactly the group a stage needs.
// The registers such a load writes are tied to the wait that covers them
// (an asm operand), so the compiler places no read of them earlier; no
// value written by these loads is copied or spilled before its wait (checked
// in the generated code: the loads only ever feed the tied waits).
// The stages of one offset form a trip of NCH = ceil(C_in / 64) stages; the
// offsets are popped from the tile's mask once per trip into a small ring of
// scalars, so every stage's offset, chunk and lead resolve at compile time
// in the unrolled loop.

typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v_t __attribute__((ext_vector_type(2)));

// Buffer resource of `bytes` bytes at `base` (raw, no stride): loads past
// the range return zeros.
__device__ inline u32x4v_t raw_rsrc(const void* base, unsigned bytes) {
    const unsigned long long a = reinterpret_cast<unsigned long long>(base);
    return u32x4v_t{static_cast<unsigned>(a), static_cast<unsigned>(a >> 32) & 0xFFFFu, bytes, 0x00020000u};
}

__device__ inline int asm_load_i32(u32x4v_t r, unsigned voff) {
    int v;
    asm volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(r));
    return v;
}

template <typename V>
__device__ inline V asm_load_b128(u32x4v_t r, unsigned voff) {
    V v;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(r));
    return v;
}

// 16 bytes per lane from byte offset voff into LDS at lds_base + 16 * lane.
__device__ inline void asm_copy_b128(u32x4v_t r, unsigned voff, unsigned lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(r)
                 : "memory", "m0");
}

// Wait until at most N vector-memory loads are outstanding; the registers
// passed are those the awaited loads write.
template <int N>
__device__ inline void wait_vm_1(int& d) {
    asm volatile("s_waitcnt vmcnt(%1)" : "+v"(d) : "n"(N));
}

template <int N, typename V, int CB, int ST>
__device__ inline void wait_vm_b(V (&b)[CB][ST]) {
    static_assert(CB * ST == 4, "four B fragments");
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(b[0][0]), "+v"(b[0][1]), "+v"(b[1][0]), "+v"(b[1][1]) : "n"(N));
}

// f(integral_constant<J>) for J = B .. E - 1.
template <int B, int E, typename F>
__device__ inline void static_for(F& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}
// The same for J in [lo, hi) (lo and hi fold to constants once the
// caller's loop is unrolled).
template <int B = 0, int MAXN = 64, typename F>
__device__ inline void static_for_range(F& f, int lo, int hi) {
    if constexpr (B < MAXN) {
        if (B >= lo && B < hi) f(std::integral_constant<int, B>{});
        static_for_range<B + 1, MAXN>(f, lo, hi);
    }
}

constexpr int gcd_int(int a, int b) { return b == 0 ? a : gcd_int(b, a % b); }

// Vector-memory ops a streamed stage j issues: the row indices of a trip
// when stage j + li starts one (trips of nch stages), then its B loads and
// A copies (nbd).  stream_wait_a: the ops issued after the copies of
// stage p + 1 - la, which the wait at the end of stage p lets through.
constexpr int stream_ops(int j, int li, int nch, int nbd) {
    return (((j + li) % nch + nch) % nch == 0 ? 1 : 0) + nbd;
}
constexpr int stream_wait_a(int p, int la, int li, int nch, int nbd) {
    int w = 0;
    for (int j = p + 2 - la; j <= p; ++j) w += stream_ops(j, li, nch, nbd);
    return w;
}
constexpr int lcm_int(int a, int b) { return a / gcd_int(a, b) * b; }

// Tile of the streamed kernel: C_OUT output channels per block (a column
// half when C_out = 256), its 4 waves in WR row groups x 4 / WR column
// groups of 32 columns.
template <int C_OUT_, int WR_, int LA_ = 2, int OCC_ = 3>
struct StreamShape {
    static constexpr int C_OUT = C_OUT_;
    static constexpr int WAVES = 4;
    static constexpr int THREADS = WAVES * 64;
    static constexpr int WR = WR_;
    static constexpr int WC = WAVES / WR_;
    static constexpr int ROWS = 128;          // tile rows (the tile order's 128-row tiles)
    static constexpr int WROWS = ROWS / WR;   // rows per wave
    static constexpr int WCOLS = C_OUT / WC;  // columns per wave
    static constexpr int RB = WROWS / 16;     // 16-row MFMA blocks per wave
    static constexpr int CB = WCOLS / 16;     // 16-column MFMA blocks per wave
    static constexpr int CHUNK = 64;          // input channels per stage
    static constexpr int ST = CHUNK / 32;     // 32-channel MFMA steps per stage
    static constexpr int GATHER = ROWS * (CHUNK / 8) / THREADS;  // row-line copies per thread and stage
    static constexpr int ABUF = ROWS * CHUNK;  // halves of one A buffer
    static constexpr int OCC = OCC_;           // blocks per CU
    // A copies lead by LA stages (a ring of LA + 1 buffers).  LA = 2 at
    // three blocks per CU measured fastest: LA = 3 or 4 at two blocks per
    // CU (a third more copies in flight per CU) ran config 3 at 0.200 /
    // 0.204 against 0.188 ms, and C_out = 64 at LA = 1 with four blocks
    // per CU at 0.055 against 0.053 ms.
    static constexpr int LA = LA_;
    static constexpr int LB = 2;               // B loads lead by LB stages
    static constexpr int LI = LA_ + 1;         // row-index loads lead by LI stages
    static constexpr int READ_AHEAD = 2;       // 16-row fragment reads in flight
    static_assert(WCOLS == 32 && WROWS % 16 == 0 && GATHER == 4, "stream tile shape");
};

// Fragment (k, ks, cg, cb) of a weight: the 16 x 32 block of output
// channels cg*32 + cb*16 .. + 15 and input channels ks*32 .. + 31 of offset
// k, as 64 lanes x 8 values: lane (lr, lg) holds W[co = cg*32 + cb*16 + lr]
// [k][ci = ks*32 + lg*8 .. + 7].  Fragments are stored in (k, ks, cg, cb)
// order, 1 KB each.
__host__ __device__ inline long long fragment_piece(int k, int ks, int cg, int cb, int lane, int ksteps, int ncg) {
    return ((((static_cast<long long>(k) * ksteps + ks) * ncg + cg) * 2 + cb) * 64 + lane);
}

template <typename T>
__global__ void __launch_bounds__(256)
weight_fragments(const T* __restrict__ w, int K, int c_in, int c_out, T* __restrict__ frag) {
    const int ksteps = c_in / 32;
    const int ncg = c_out / 32;
    const long long pieces = static_cast<long long>(K) * c_in * c_out / 8;
    for (long long p = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; p < pieces;
         p += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int lane = static_cast<int>(p % 64);
        long long f = p / 64;
        const int cb = static_cast<int>(f % 2);
        f /= 2;
        const int cg = static_cast<int>(f % ncg);
        f /= ncg;
        const int ks = static_cast<int>(f % ksteps);
        const int k = static_cast<int>(f / ksteps);
        const int co = cg * 32 + cb * 16 + (lane & 15);
        const int ci = ks * 32 + (lane >> 4) * 8;
        *reinterpret_cast<uint4*>(frag + p * 8) =
            *reinterpret_cast<const uint4*>(w + (static_cast<long long>(co) * K + k) * c_in + ci);
    }
}

// Packed fragment of a quantized weight (lattice_hip_quantized_weight_
// fragments): the 16 bytes of lane (lr, lg) of fragment (k, ks, cg, cb)
// hold the codes of W[co][k][ci .. ci + 7] (co = cg*32 + cb*16 + lr,
// ci = ks*32 + lg*8) and the affine scale and bias of their group:
// x = 4-bit codes (nibble j = ci + j) or the first four 8-bit codes (byte
// j), y = the last four 8-bit codes, z = scale | bias << 16, w unused.
// Dequantised in registers once the load has landed: w = q * scale + bias,
// one rounding to T (packed fp16 math as in PackedB::load).
// Packed fragments of a quantized weight (layout above dequant_fragment):
// w (K, packed_words, c_out) uint32 codes, scales / biases (K, groups,
// c_out) of type T.
template <typename T>
__global__ void __launch_bounds__(256)
packed_weight_fragments(const uint32_t* __restrict__ w, const T* __restrict__ scales, const T* __restrict__ biases,
                        int K, int c_in, int c_out, int packed_words, int groups, int group_size, int bits,
                        uint4* __restrict__ frag) {
    const int ksteps = c_in / 32;
    const int ncg = c_out / 32;
    const long long pieces = static_cast<long long>(K) * c_in * c_out / 8;
    for (long long p = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; p < pieces;
         p += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int lane = static_cast<int>(p % 64);
        long long f = p / 64;
        const int cb = static_cast<int>(f % 2);
        f /= 2;
        const int cg = static_cast<int>(f % ncg);
        f /= ncg;
        const int ks = static_cast<int>(f % ksteps);
        const int k = static_cast<int>(f / ksteps);
        const int co = cg * 32 + cb * 16 + (lane & 15);
        const int ci = ks * 32 + (lane >> 4) * 8;
        const long long wbase = static_cast<long long>(k) * packed_words * c_out + co;
        const long long sidx = (static_cast<long long>(k) * groups + ci / group_size) * c_out + co;
        uint4 r;
        if (bits == 4) {
            r.x = w[wbase + static_cast<long long>(ci >> 3) * c_out];
            r.y = 0u;
        } else {
            r.x = w[wbase + static_cast<long long>(ci >> 2) * c_out];
            r.y = w[wbase + static_cast<long long>((ci >> 2) + 1) * c_out];
        }
        r.z = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, scales[sidx])) |
              (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, biases[sidx])) << 16);
        r.w = 0u;
        frag[p] = r;
    }
}

template <typename T, int QB>
__device__ inline typename MfmaOps<T>::vec dequant_fragment(typename MfmaOps<T>::vec raw) {
    using V = typename MfmaOps<T>::vec;
    const uint4 r = __builtin_bit_cast(uint4, raw);
    V out;
    if constexpr (std::is_same<T, _Float16>::value) {
        const half2_t sb = __builtin_bit_cast(half2_t, r.z);
        const half2_t sc = {sb[0], sb[0]};
        const half2_t bi = {sb[1], sb[1]};
        if constexpr (QB == 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const half2_t v = affine_pair(code_pair((r.x >> (4 * j)) & 0x000F000Fu), sc, bi);
                out[j] = v[0];
                out[j + 4] = v[1];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t word = i == 0 ? r.x : r.y;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const half2_t v = affine_pair(code_pair((word >> (8 * j)) & 0x00FF00FFu), sc, bi);
                    out[4 * i + j] = v[0];
                    out[4 * i + j + 2] = v[1];
                }
            }
        }
    } else {
        const float sc = static_cast<float>(__builtin_bit_cast(T, static_cast<uint16_t>(r.z & 0xFFFFu)));
        const float bi = static_cast<float>(__builtin_bit_cast(T, static_cast<uint16_t>(r.z >> 16)));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t q = QB == 4 ? (r.x >> (4 * j)) & 15u : ((j < 4 ? r.x : r.y) >> (8 * (j & 3))) & 255u;
            out[j] = static_cast<T>(static_cast<float>(q) * sc + bi);
        }
    }
    return out;
}

template <typename T, typename S, int NCH, int QB>
__global__ void __launch_bounds__(S::THREADS, S::OCC)
conv_igemm_stream(const T* __restrict__ feats, int n_in, int c_in, const T* __restrict__ wfrag, int kernel_count,
                  int c_out_total, const int32_t* __restrict__ kv_map, const int32_t* __restrict__ tile_masks,
                  const int32_t* __restrict__ reorder_rows, int rows, const int32_t* __restrict__ block_order,
                  T* __restrict__ out, Epilogue<T> epi, int halves) {
    using V = typename MfmaOps<T>::vec;
    constexpr int RB = S::RB;
    constexpr int CB = S::CB;
    constexpr int ST = S::ST;
    constexpr int G = S::GATHER;
    constexpr int NB = CB * ST;  // B loads per stage
    constexpr int ND = G;        // LDS copies per stage
    constexpr int ABYTES = S::ABUF * static_cast<int>(sizeof(T));
    __shared__ __align__(16) T lds[(S::LA + 1) * S::ABUF];

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int wr = wave / S::WC;
    const int wc = wave % S::WC;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int col0 = wc * S::WCOLS;
    // Longest-first tile order; with C_out = 256 consecutive blocks take the
    // two column halves of one tile (the second finds its rows in L2).
    const int slot = halves > 1 ? static_cast<int>(blockIdx.x) / 2 : static_cast<int>(blockIdx.x);
    const int half = halves > 1 ? static_cast<int>(blockIdx.x & 1u) : 0;
    const int cg = half * (S::C_OUT / S::WCOLS) + wc;  // 32-column group of the weight
    const int out_ld = S::C_OUT * halves;
    const int tile = block_order != nullptr ? block_order[slot] : slot;
    const int row0 = tile * S::ROWS;
    const int quarters = ((rows + 63) / 64) * 4;
    // Offset masks of the wave's 16-row blocks and of the whole tile.
    uint32_t qm[RB];
    uint32_t bmask = 0;
#pragma unroll
    for (int q = 0; q < S::ROWS / 16; ++q) {
        const int qi = row0 / 16 + q;
        const uint32_t m = qi < quarters ? static_cast<uint32_t>(tile_masks[qi]) : 0u;
        bmask |= m;
        if (q / RB == wr) qm[q % RB] = m;
    }
    const int ntrips = __popc(bmask);

    float4_t acc[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    if (ntrips > 0) {
        const int gp = (lane & 7) ^ ((lane >> 3) & 7);  // piece it copies (its slot ^ row % 8)
        const int ksteps = c_in / 32;
        const int ncg = c_out_total / S::WCOLS;
        const bool partial = (c_in % S::CHUNK) != 0;  // the last chunk holds 32 channels
        const u32x4v_t frs = raw_rsrc(feats, static_cast<unsigned>(static_cast<long long>(n_in) * c_in * sizeof(T)));
        const u32x4v_t krs =
            raw_rsrc(kv_map, static_cast<unsigned>(static_cast<long long>(kernel_count) * rows * sizeof(int32_t)));
        const u32x4v_t wrs = raw_rsrc(
            wfrag, static_cast<unsigned>(static_cast<long long>(kernel_count) * c_in * c_out_total * sizeof(T)));
        const unsigned lds0 = static_cast<unsigned>(reinterpret_cast<unsigned long long>(lds));

        constexpr int LA = S::LA, LB = S::LB, LI = S::LI;
        static_assert(LI - LA == 1, "row indices arrive one stage before their copies");
        // Row indices are loaded once per trip (an offset's NCH stages share
        // them): one dword per lane, lane j < 32 holding copy row j of the
        // wave, at the stage LI stages before the trip's first stage.  At
        // most two trips' indices are in flight when a trip is one stage.
        constexpr int NRS = NCH == 1 ? 2 : 1;  // row-index register sets
        constexpr int NBS = LB + 1;            // B register sets
        // stages per unrolled block: whole trips that cycle every register set
        constexpr int U = lcm_int(NRS * NCH, NBS);
        static_assert(U % NCH == 0, "whole trips per unrolled block");
        constexpr int TPU = U / NCH;                 // trips per unrolled block
        constexpr int R = TPU + (U - 1 + LI) / NCH;  // ring entries a block reaches
        // Offset ring: kr[i] is the offset of trip t + i (t = the block's
        // first trip); past the last trip it repeats the last offset, whose
        // prefetched operands are never used.
        uint32_t rem = bmask;
        int klast = 0;
        auto pop = [&]() {
            if (rem) {
                klast = __builtin_ctz(rem);
                rem &= rem - 1;
            }
            return klast;
        };
        int kr[R];
#pragma unroll
        for (int i = 0; i < R; ++i) kr[i] = pop();

        // Lanes j and j + 32 load the index of copy row j of the wave.
        auto idx_load = [&](int& raw, int k) {
            const int r = min(row0 + wave * (8 * G) + (lane & 31), rows - 1);
            raw = asm_load_i32(krs, static_cast<unsigned>((k * rows + r) * 4));
        };
        // Copy i of this lane reads row 8 i + lane / 8 of the wave's 32.
        auto idx_expand = [&](int (&d)[G], int raw) {
#pragma unroll
            for (int i = 0; i < G; ++i) d[i] = __builtin_amdgcn_ds_bpermute((8 * i + (lane >> 3)) << 2, raw);
        };
        auto b_load = [&](V (&b)[CB][ST], int k, int ch, int cb, int st) {
            b[cb][st] = asm_load_b128<V>(
                wrs, static_cast<unsigned>(fragment_piece(k, ch * ST + st, cg, cb, lane, ksteps, ncg) * 16));
        };
        auto a_copy = [&](const int (&d)[G], int ch, int buf, int i) {
            const int ci = ch * S::CHUNK;
            // a partial last chunk copies its four pieces twice
            const int off = (partial && ch == NCH - 1 && gp >= 4) ? (gp - 4) * 8 : gp * 8;
            const unsigned dst = lds0 + buf * ABYTES + (wave * (8 * G) + 8 * i) * S::CHUNK * sizeof(T);
            const unsigned row = static_cast<unsigned>(d[i]) * static_cast<unsigned>(c_in * sizeof(T));
            asm_copy_b128(frs, row + (ci + off) * sizeof(T), __builtin_amdgcn_readfirstlane(dst));
        };

        // Memory ops of stage j: the trip's row indices when stage j + LI
        // starts a trip, then NB B loads, then ND copies.
        constexpr auto has_idx = [](int j) { return ((j + LI) % NCH + NCH) % NCH == 0; };
        constexpr auto ops = [](int j) { return (((j + LI) % NCH + NCH) % NCH == 0 ? 1 : 0) + NB + ND; };
        constexpr int W_IDX = NB + ND;  // indices of stage s + LA's trip, at stage s (issued first in s - 1)
        static_assert(W_IDX < 64 && ND + ops(0) < 64, "waits fit the counter");
        int raw[NRS];
        int d[G];
        V b[NBS][CB][ST];
        // Prologue: indices of stages 0 .. LI - 1, A(0) .. A(LA - 1), B(0) ..
        // B(LB - 1), all complete before stage 0.
#pragma unroll
        for (int u = 0; u < LI; ++u) {
            if (u % NCH == 0) idx_load(raw[(u / NCH) % NRS], kr[u / NCH]);
            if (u < LA) {
                if (u % NCH == 0) {
                    wait_vm_1<0>(raw[(u / NCH) % NRS]);
                    idx_expand(d, raw[(u / NCH) % NRS]);
                }
#pragma unroll
                for (int i = 0; i < G; ++i) a_copy(d, u % NCH, u, i);
            }
        }
#pragma unroll
        for (int u = 0; u < LB; ++u)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                for (int st = 0; st < ST; ++st) b_load(b[u % NBS], kr[u / NCH], u % NCH, cb, st);
        asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

        int buf = 0;  // LDS buffer of A(s)
        // The stage at position P of the unrolled block.
        auto step = [&](auto P) {
            constexpr int p = decltype(P)::value;
            constexpr int ch = p % NCH;
            constexpr int NI = has_idx(p) ? 1 : 0;
            constexpr int NT = NI + NB + ND;
            constexpr int W_B = ND + ops(p - 1);  // B(s), before stage s issues (LB = 2)
            // A(s + 1), at the end of stage s: the copies of stage s + 1 - LA
            // came last in it, then every op of stages s + 2 - LA .. s
            constexpr int W_A = stream_wait_a(p, LA, LI, NCH, NB + ND);
            static_assert(W_A < 64, "waits fit the counter");
            static_assert(LB == 2, "W_B counts one stage between a B load and its use");
            V (&bcur)[CB][ST] = b[p % NBS];
            V (&bfill)[CB][ST] = b[(p + LB) % NBS];
            const int k = kr[p / NCH];
            const int k_i = kr[(p + LI) / NCH];
            const int k_b = kr[(p + LB) / NCH];
            const int abuf_fill = buf == 0 ? LA : buf - 1;  // (s + LA) % (LA + 1)
            if constexpr ((p + LA) % NCH == 0) {
                int& ra = raw[((p + LA) / NCH) % NRS];
                wait_vm_1<W_IDX>(ra);
                idx_expand(d, ra);
            }
            wait_vm_b<W_B>(bcur);
            if constexpr (QB != 0) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                    for (int st = 0; st < ST; ++st) bcur[cb][st] = dequant_fragment<T, QB>(bcur[cb][st]);
            }
            // Memory op q of this stage, in the fixed order.
            auto issue_op = [&](auto Q) {
                constexpr int q = decltype(Q)::value;
                if constexpr (q < NI) {
                    idx_load(raw[((p + LI) / NCH) % NRS], k_i);
                } else if constexpr (q < NI + NB) {
                    b_load(bfill, k_b, (p + LB) % NCH, (q - NI) / ST, (q - NI) % ST);
                } else {
                    a_copy(d, (p + LA) % NCH, abuf_fill, q - NI - NB);
                }
            };
            const int nst = (partial && ch == NCH - 1) ? 1 : ST;
            const T* arow = lds + buf * S::ABUF + (wr * S::WROWS + lr) * S::CHUNK;
            auto read_a = [&](V (&a)[ST], int rb) {
#pragma unroll
                for (int st = 0; st < ST; ++st) {
                    a[st] = *reinterpret_cast<const V*>(arow + rb * 16 * S::CHUNK + (((st * 4 + lg) ^ (lr & 7)) * 8));
                }
            };
            constexpr int RA = S::READ_AHEAD;
            V af[RA + 1][ST];
#pragma unroll
            for (int r = 0; r < RA && r < RB; ++r) read_a(af[r], r);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                if (rb + RA < RB) read_a(af[(rb + RA) % (RA + 1)], rb + RA);
                // this 16-row block's share of the stage's memory ops
                static_for_range(issue_op, rb * NT / RB, (rb + 1) * NT / RB);
                if ((qm[rb] >> k) & 1u) {
#pragma unroll
                    for (int st = 0; st < ST; ++st) {
                        if (st < nst) {
#pragma unroll
                            for (int cb = 0; cb < CB; ++cb) {
                                // transposed product: lane (lr, lg) accumulates
                                // row rb*16 + lr, columns cb*16 + lg*4 .. + 3
                                acc[rb][cb] = MfmaOps<T>::mfma(bcur[cb][st], af[rb % (RA + 1)][st], acc[rb][cb]);
                            }
                        }
                    }
                }
            }
            // A(s + 1) has landed for this wave; the barrier makes it so for
            // every wave and frees buffer `buf` for the copy of A(s + 3).
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(W_A) : "memory");
            buf = buf == LA ? 0 : buf + 1;
        };
        auto block = [&](int t0) {
            auto guarded = [&](auto P) {
                constexpr int p = decltype(P)::value;
                if (t0 + p / NCH < ntrips) step(P);
            };
            static_for<0, U>(guarded);
#pragma unroll
            for (int i = 0; i < R; ++i) kr[i] = i + TPU < R ? kr[i + TPU] : pop();
        };
        for (int t = 0; t < ntrips; t += TPU) block(t);
        // No copy may land in this block's LDS after it ends.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // The finished tile goes through LDS (the A ring is free once every
    // wave's copies have landed) so that it leaves as 16-byte stores of
    // whole output rows to out[reorder_rows[row]], non-temporal (streamed
    // past the caches: config 2's conv 24.4 -> 21.5 us, config 3's
    // 188 -> 184 us).  Rows with no edges store
    // zeros (plus bias).
    constexpr int LDW = S::C_OUT + 8;  // halves per staged row: rows 16 bytes apart in the banks
    static_assert(S::ROWS * LDW <= (S::LA + 1) * S::ABUF, "the staged tile fits the A ring");
    __syncthreads();
    T* const stage = lds;
    uint2 bias4[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
        bias4[cb] = epi.bias != nullptr
                        ? *reinterpret_cast<const uint2*>(epi.bias + half * S::C_OUT + col0 + cb * 16 + lg * 4)
                        : uint2{0u, 0u};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = wr * S::WROWS + rb * 16 + lr;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const T* bq = reinterpret_cast<const T*>(&bias4[cb]);
            T v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = epi.finish(acc[rb][cb][q], static_cast<float>(bq[q]));
            *reinterpret_cast<uint2*>(stage + r * LDW + col0 + cb * 16 + lg * 4) = *reinterpret_cast<const uint2*>(v);
        }
    }
    __syncthreads();
    constexpr int CPR = S::C_OUT / 8;  // 16-byte pieces per row
    T* const ohalf = out + half * S::C_OUT;
    for (int i = threadIdx.x; i < S::ROWS * CPR; i += S::THREADS) {
        const int r = i / CPR;
        const int piece = i % CPR;
        const int sr = row0 + r;
        if (sr < rows) {
            const int orow = reorder_rows != nullptr ? reorder_rows[sr] : sr;
            __builtin_nontemporal_store(
                *reinterpret_cast<const u32x4v_t*>(stage + r * LDW + piece * 8),
                reinterpret_cast<u32x4v_t*>(ohalf + static_cast<long long>(orow) * out_ld + piece * 8));
        }
    }
}

// ------------------------------------------------- dense-map small C_in --
//
// Convolutions with few input channels (C_in 4 or 8: the stem of an
// encoder) over the relation's dense map out_in_map[row][k]: a row's
// neighbourhood, K offsets x C_in channels, is one contraction of K * C_in
// values (padded to a multiple of 32) against the weight flattened the same
// way, so the whole conv is a GEMM whose A rows are gathered from the map.
// A wave takes 16 rows at a time: lane (lr, lg) gathers, for each 32-wide
// step j, the flat positions j * 32 + lg * 8 .. + 7 of row lr (8 / C_in
// offsets of C_in channels, one 8- or 16-byte row load each); the weight's
// B fragments for every step (CO / 16 column blocks) are built once per
// block in LDS and held in registers (quantized weights dequantised there:
// w = q * scale + bias in fp32, rounded once to T).  A wave walks 16-row
// blocks grid-stride, loading the next block's map entries while the
// current one computes.  The MFMAs accumulate in fp32; the
// store applies the bias and ReLU as the other routes do.  Map entries of
// -1 or out of range, and rows at or past the relation's active output
// count, contribute nothing (rows past it store the bias alone).
template <typename T, int CI, int CO, bool QUANT, int KS_MAX>
__global__ void __launch_bounds__(256)
conv_dense_map(const T* __restrict__ feats, int n_in, const T* __restrict__ fweights, WeightIndex widx,
               const uint32_t* __restrict__ qweights, const T* __restrict__ scales, const T* __restrict__ qbiases,
               QuantIndex q, int K, const int32_t* __restrict__ out_in_map, const int32_t* __restrict__ counts,
               int out_capacity, T* __restrict__ out, Epilogue<T> epi) {
    using V = typename MfmaOps<T>::vec;
    constexpr int CB = CO / 16;
    // KS_MAX: bound on the 32-wide steps (K * CI <= 32 * KS_MAX)
    constexpr int OPL = 8 / CI;  // offsets per lane and step
    constexpr int NFRAG = KS_MAX * CB;
    static_assert(CI == 4 || CI == 8, "8- or 16-byte feature rows");
    __shared__ __align__(16) T wlds[NFRAG * 64 * 8];
    const int KS = (K * CI + 31) / 32;
    const int lane = lane_id();
    const int lr = lane & 15;
    const int lg = lane >> 4;
    // B fragments, built once per block into LDS: fragment (j, cb), lane
    // (lr, lg) holds W[co = cb*16 + lr] at flat positions j*32 + lg*8 .. + 7
    // (flat = k * CI + ci; zero past K), in the order of the MFMA operand.
    for (int slot = threadIdx.x; slot < NFRAG * 64; slot += blockDim.x) {
        const int f = slot / 64, l = slot % 64;
        const int j = f / CB, cb = f % CB;
        const int co = cb * 16 + (l & 15);
        V v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int flat = j * 32 + (l >> 4) * 8 + e;
            const int k = flat / CI;
            const int ci = flat % CI;
            float w = 0.0f;
            if (k < K) {
                w = QUANT ? dequant(qweights, scales, qbiases, q, k, ci, co) : Elem<T>::load(fweights, widx(k, ci, co));
            }
            v[e] = static_cast<T>(w);
        }
        *reinterpret_cast<V*>(wlds + slot * 8) = v;
    }
    __syncthreads();
    V bfrag[KS_MAX][CB];
#pragma unroll
    for (int j = 0; j < KS_MAX; ++j)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) bfrag[j][cb] = *reinterpret_cast<const V*>(wlds + ((j * CB + cb) * 64 + lane) * 8);

    const int n_out = min(max(counts[1], 0), out_capacity);
    const int waves = static_cast<int>(gridDim.x) * (blockDim.x / kWave);
    const int wave_id = static_cast<int>(blockIdx.x) * (blockDim.x / kWave) + static_cast<int>(threadIdx.x) / kWave;
    const int blocks16 = (out_capacity + 15) / 16;
    // map entries of 16-row block b16 for this lane (-1 = none)
    auto load_map = [&](int b16, int (&m)[KS_MAX][OPL]) {
        const int row = b16 * 16 + lr;
        const bool active = row < n_out;
#pragma unroll
        for (int j = 0; j < KS_MAX; ++j)
#pragma unroll
            for (int t = 0; t < OPL; ++t) {
                const int k = (j * 32 + lg * 8) / CI + t;
                m[j][t] = active && j < KS && k < K ? out_in_map[static_cast<long long>(row) * K + k] : -1;
            }
    };
    int mnext[KS_MAX][OPL];
    if (wave_id < blocks16) load_map(wave_id, mnext);
    for (int b16 = wave_id; b16 < blocks16; b16 += waves) {
        const int row = b16 * 16 + lr;
        int m[KS_MAX][OPL];
#pragma unroll
        for (int j = 0; j < KS_MAX; ++j)
#pragma unroll
            for (int t = 0; t < OPL; ++t) m[j][t] = mnext[j][t] >= 0 && mnext[j][t] < n_in ? mnext[j][t] : -1;
        V a[KS_MAX];
#pragma unroll
        for (int j = 0; j < KS_MAX; ++j) {
            if constexpr (CI == 4) {
                uint2 w2[2];
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    w2[t] = m[j][t] >= 0 ? *reinterpret_cast<const uint2*>(feats + static_cast<long long>(m[j][t]) * 4)
                                         : uint2{0u, 0u};
                a[j] = __builtin_bit_cast(V, uint4{w2[0].x, w2[0].y, w2[1].x, w2[1].y});
            } else {
                a[j] = m[j][0] >= 0 ? *reinterpret_cast<const V*>(feats + static_cast<long long>(m[j][0]) * 8)
                                    : __builtin_bit_cast(V, uint4{0u, 0u, 0u, 0u});
            }
        }
        // the next block's map entries load while this block computes
        if (b16 + waves < blocks16) load_map(b16 + waves, mnext);
        float4_t acc[CB];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[cb] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KS_MAX; ++j) {
            if (j < KS) {
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) acc[cb] = MfmaOps<T>::mfma(bfrag[j][cb], a[j], acc[cb]);
            }
        }
        // lane (lr, lg): row lr, columns cb*16 + lg*4 .. + 3
        if (row < out_capacity) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                T v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = epi.apply(acc[cb][i], cb * 16 + lg * 4 + i);
                __builtin_nontemporal_store(*reinterpret_cast<const u32x2v_t*>(v),
                                            reinterpret_cast<u32x2v_t*>(out + static_cast<long long>(row) * CO +
                                                                        cb * 16 + lg * 4));
            }
        }
    }
}

// ------------------------------------------------- direct expansion ----
//
// Conv over a direct generative / transposed relation (output row
// in * K + k has the single edge (in, k)): out[in*K + k] = feats[in] @ W[k],
// a dense GEMM of the input rows against the K weight slices, with no
// gather.  A block owns 128 consecutive input rows (32 per wave) and keeps
// their MFMA A fragments in registers for all K offsets.  Per offset k:
//   * the block's threads hold W[:, k+1, :] in registers (loaded while k
//     computes) and store it to LDS after a barrier, so the weight crosses
//     the vector-memory path once per block instead of once per wave;
//   * B fragments are read from LDS (16-byte pieces XOR-swizzled by row);
//   * each wave stages its 32 x C_OUT tile in its own LDS area and writes
//     whole 16-byte row pieces to out[in * K + k].
// Input rows at or past the active count give zero rows (plus bias), as
// the relation has no edges for them.  Two blocks share a CU, except at
// C_out = 256, whose per-wave staging (4 x 32 x 264 halves) leaves LDS for
// one.
template <typename T, int KSTEPS, int CB>
__global__ void __launch_bounds__(256, CB == 16 ? 1 : 2)
conv_expand(const T* __restrict__ feats, int n_in, const int32_t* __restrict__ active_rows,
            const T* __restrict__ weights, int K, T* __restrict__ out, Epilogue<T> epi) {
    using V = typename MfmaOps<T>::vec;
    constexpr int C_IN = KSTEPS * 32;
    constexpr int C_OUT = CB * 16;
    constexpr int PIECES = C_OUT / 8;       // 16-byte pieces per output row
    constexpr int SROW = C_OUT + 8;         // padded stage row
    constexpr int WPIECES = C_IN / 8;       // 16-byte pieces per weight row (one output channel)
    constexpr int WTOTAL = C_OUT * WPIECES;  // pieces of one W[:, k, :]
    constexpr int WPER = (WTOTAL + 255) / 256;
    __shared__ __align__(16) T wbuf[C_OUT * C_IN];
    __shared__ __align__(16) T stage[4][32 * SROW];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int active = min(max(*active_rows, 0), n_in);
    const int in0 = blockIdx.x * 128 + wave * 32;
    V a[2][KSTEPS];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int row = in0 + rb * 16 + lr;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            a[rb][ks] = row < active
                            ? *reinterpret_cast<const V*>(feats + static_cast<long long>(row) * C_IN + ks * 32 + lg * 8)
                            : V{};
        }
    }
    // bias of the four output channels cb*16 + lg*4 .. +3 this lane stores
    uint2 bias4[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
        bias4[cb] = epi.bias != nullptr ? *reinterpret_cast<const uint2*>(epi.bias + cb * 16 + lg * 4) : uint2{0u, 0u};
    // piece p of W[co, k, :] sits at wbuf[co * C_IN + ((p ^ (co % WPIECES)) * 8)]
    V wreg[WPER];
    auto load_w = [&](int k) {
#pragma unroll
        for (int j = 0; j < WPER; ++j) {
            const int i = j * 256 + threadIdx.x;
            if (WTOTAL % 256 == 0 || i < WTOTAL) {
                const int co = i / WPIECES;
                const int p = i - co * WPIECES;
                wreg[j] = *reinterpret_cast<const V*>(weights + (static_cast<long long>(co) * K + k) * C_IN + p * 8);
            }
        }
    };
    auto store_w = [&]() {
#pragma unroll
        for (int j = 0; j < WPER; ++j) {
            const int i = j * 256 + threadIdx.x;
            if (WTOTAL % 256 == 0 || i < WTOTAL) {
                const int co = i / WPIECES;
                const int p = i - co * WPIECES;
                *reinterpret_cast<V*>(wbuf + co * C_IN + ((p ^ (co % WPIECES)) * 8)) = wreg[j];
            }
        }
    };
    load_w(0);
    store_w();
    __syncthreads();
    T* st = stage[wave];
    // The wave's output rows in0 .. in0 + 31 as a raw buffer: rows past
    // n_in lie beyond its range, so their stores are dropped with no branch.
    const long long out_bytes = (in0 < n_in ? static_cast<long long>(n_in - in0) : 0ll) * K * C_OUT * sizeof(T);
    const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        out + static_cast<long long>(min(in0, n_in)) * K * C_OUT, 0,
        static_cast<int>(min(out_bytes, static_cast<long long>(INT_MAX))), 0x00020000);
    for (int k = 0; k < K; ++k) {
        // W[:, k+1, :] (the last offset reloads its own slice, so the loop
        // body has no branch around its loads and stores) is in flight
        // during this offset's MFMAs.
        load_w(min(k + 1, K - 1));
        float4_t acc[2][CB];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            V b[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const int co = cb * 16 + lr;
                const int p = ks * 4 + lg;
                b[cb] = *reinterpret_cast<const V*>(wbuf + co * C_IN + ((p ^ (co % WPIECES)) * 8));
            }
            // The transposed product W[k]^T-fragment x feats^T-fragment:
            // lane (lr, lg) then holds output channels cb*16 + lg*4 .. +3 of
            // row rb*16 + lr, four consecutive halves for one 8-byte store.
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) acc[rb][cb] = MfmaOps<T>::mfma(b[cb], a[rb][ks], acc[rb][cb]);
        }
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const T* bq = reinterpret_cast<const T*>(&bias4[cb]);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                T v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = epi.finish(acc[rb][cb][q], static_cast<float>(bq[q]));
                *reinterpret_cast<uint2*>(st + (rb * 16 + lr) * SROW + cb * 16 + lg * 4) =
                    *reinterpret_cast<const uint2*>(v);
            }
        }
        __syncthreads();  // every wave has read W[:, k, :] and staged its tile
        // W[:, k+1, :] goes to LDS before this offset's rows are stored: the
        // wait for its loads then covers only stores issued an offset ago,
        // and this offset's stores drain during the next offset's MFMAs.
        store_w();
        {
            // All of the wave's row pieces are read from the stage first,
            // then stored: 32 rows x PIECES pieces over the 64 lanes.
            constexpr int PER = 32 * PIECES / kWave;
            static_assert(32 * PIECES % kWave == 0, "whole pieces per lane");
            V piece_v[PER];
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int p = lane + j * kWave;
                piece_v[j] = *reinterpret_cast<const V*>(st + (p / PIECES) * SROW + (p % PIECES) * 8);
            }
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int p = lane + j * kWave;
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(u32x4_t, piece_v[j]), out_rsrc,
                    static_cast<int>((((p / PIECES) * K + k) * C_OUT + (p % PIECES) * 8) * sizeof(T)), 0,
                    kNonTemporal);
            }
        }
        __syncthreads();  // W[:, k+1, :] in LDS; the stage is free again
    }
}

// Launches conv_expand for c_in * c_out <= 16384 (the weight slice of one
// offset fits a 32 KB LDS buffer next to the four 32-row output stages).
template <typename T, int KSTEPS, int CB>
int launch_expand_shape(const T* feats, int n_in, const int32_t* active, const T* w, int K, T* out, Epilogue<T> epi,
                        hipStream_t stream) {
    static_assert(KSTEPS * 32 * CB * 16 <= 16384, "the weight slice must fit its LDS buffer");
    const unsigned blocks = static_cast<unsigned>((n_in + 127) / 128);
    conv_expand<T, KSTEPS, CB><<<blocks, 256, 0, stream>>>(feats, n_in, active, w, K, out, epi);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

template <typename T>
int launch_expand(const T* feats, int n_in, const int32_t* active, int c_in, const T* w, int K, int c_out, T* out,
                  Epilogue<T> epi, hipStream_t stream) {
    if (n_in <= 0) return LATTICE_OK;
#define LATTICE_EXPAND(CI, CO) \
    if (c_in == CI && c_out == CO) return launch_expand_shape<T, CI / 32, CO / 16>(feats, n_in, active, w, K, out, epi, stream)
    LATTICE_EXPAND(32, 32);
    LATTICE_EXPAND(32, 64);
    LATTICE_EXPAND(32, 128);
    LATTICE_EXPAND(32, 256);
    LATTICE_EXPAND(64, 32);
    LATTICE_EXPAND(64, 64);
    LATTICE_EXPAND(64, 128);
    LATTICE_EXPAND(64, 256);
    LATTICE_EXPAND(128, 32);
    LATTICE_EXPAND(128, 64);
    LATTICE_EXPAND(128, 128);
    LATTICE_EXPAND(256, 32);
    LATTICE_EXPAND(256, 64);
#undef LATTICE_EXPAND
    set_error("the expansion conv supports c_in, c_out in {32, 64, 128, 256} with c_in * c_out <= 16384.");
    return LATTICE_ERROR_UNSUPPORTED;
}

// Longest-first order of the row tiles of one launch: the cost of a tile is
// the number of offsets its rows use (stages it runs); a counting sort by
// descending cost fills `order`.  One workgroup: costs are read with 16-byte
// loads of the quarter masks and kept in LDS between the count and the
// placement pass.  Ties land in any order (a tile's output does not depend
// on when it runs).  Launches with more tiles than kMaxScheduledTiles run in
// order.
constexpr int kScheduleThreads = 1024;
constexpr int kMaxScheduledTiles = 32768;
constexpr int kOrderTileRows = 128;  // rows of the tiles a tile order ranks

template <int QUARTERS>
__global__ void __launch_bounds__(kScheduleThreads)
schedule_tiles(const int32_t* __restrict__ tile_masks, int rows, int nblocks, int32_t* __restrict__ order) {
    static_assert(QUARTERS % 4 == 0, "tiles span whole 64-row mask groups");
    __shared__ int count[33];
    __shared__ int next[33];
    __shared__ unsigned char cost[kMaxScheduledTiles];
    const int quarters = ((rows + 63) / 64) * 4;  // tile_masks length, a multiple of 4
    if (threadIdx.x < 33) count[threadIdx.x] = 0;
    __syncthreads();
    const int4* masks4 = reinterpret_cast<const int4*>(tile_masks);
#pragma unroll 4
    for (int b = threadIdx.x; b < nblocks; b += kScheduleThreads) {
        uint32_t m = 0;
#pragma unroll
        for (int v = 0; v < QUARTERS / 4; ++v) {
            const int q = b * QUARTERS + 4 * v;
            if (q < quarters) {
                const int4 w = masks4[q / 4];
                m |= static_cast<uint32_t>(w.x | w.y | w.z | w.w);
            }
        }
        const int c = __popc(m);
        cost[b] = static_cast<unsigned char>(c);
        atomicAdd(&count[c], 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int start = 0;
        for (int c = 32; c >= 0; --c) {
            next[c] = start;
            start += count[c];
        }
    }
    __syncthreads();
    for (int b = threadIdx.x; b < nblocks; b += kScheduleThreads) order[atomicAdd(&next[cost[b]], 1)] = b;
}

template <typename T, typename S, typename BSource>
int launch_igemm_shape(const T* feats, int n_in, int c_in, const BSource& b, const int32_t* kv_map,
                       const int32_t* tile_masks, const int32_t* reorder_rows, int rows, int32_t* schedule,
                       T* out, Epilogue<T> epi, hipStream_t stream, bool scheduled, int halves = 1) {
    static_assert(S::BLOCK_ROWS == kOrderTileRows, "every shape uses the tile order's 128-row tiles");
    const int blocks = (rows + S::BLOCK_ROWS - 1) / S::BLOCK_ROWS;
    if (blocks > kMaxScheduledTiles) schedule = nullptr;
    if (schedule != nullptr && !scheduled) {
        schedule_tiles<S::BLOCK_ROWS / 16><<<1, kScheduleThreads, 0, stream>>>(tile_masks, rows, blocks, schedule);
        LATTICE_LAUNCH_CHECK();
    }
    conv_igemm<T, S, BSource><<<static_cast<unsigned>(blocks * halves), S::THREADS, 0, stream>>>(
        feats, n_in, c_in, b, kv_map, tile_masks, reorder_rows, rows, schedule, out, epi, S::C_OUT * halves,
        halves);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

template <typename T, typename BSource>
int launch_igemm(const T* feats, int n_in, int c_in, int c_out, const BSource& b, const int32_t* kv_map,
                 const int32_t* tile_masks, const int32_t* reorder_rows, int rows, int32_t* schedule, bool ready,
                 T* out, Epilogue<T> epi, hipStream_t stream) {
    if (rows <= 0) return LATTICE_OK;
#define LATTICE_IGEMM_LAUNCH(...) \
    launch_igemm_shape<T, IgemmShape<__VA_ARGS__>>(feats, n_in, c_in, b, kv_map, tile_masks, reorder_rows, rows, \
                                                   schedule, out, epi, stream, ready)
// Default shape: 32-row wave tiles, four waves, 64-channel stages (the
// smaller B tile and register set let three blocks share a CU); c_out = 16
// keeps 128-channel stages so its B tile still covers every thread.
// c_out = 256 runs the 128-column shape over both column halves (below).
// c_out 32..128 gather A in whole lines through LDS (ALDS), three blocks
// per CU (float and packed weights alike: the packed tile's dequantisation
// from vector loads of consecutive output channels fits the registers).
    constexpr int kAldsOcc = 3;
#define LATTICE_IGEMM_CASE(C)                                                  \
    case C:                                                                    \
        return LATTICE_IGEMM_LAUNCH(C, 32, 4, 64, 1, false, kAldsOcc, 128, false, true);
    switch (c_out) {
    case 16:
        return LATTICE_IGEMM_LAUNCH(16, 32, 4, 128);
        LATTICE_IGEMM_CASE(32)
        LATTICE_IGEMM_CASE(64)
        LATTICE_IGEMM_CASE(128)
    case 256:
        // One launch of the 128-column kernel over both column halves of
        // every tile (row stride 256): its occupancy and B tile beat the
        // 8-wave 256-column shape, at the cost of gathering A twice, and
        // the two halves of a tile run back to back.
        return launch_igemm_shape<T, IgemmShape<128, 32, 4, 64, 1, false, kAldsOcc, 128, false, true>>(
            feats, n_in, c_in, b, kv_map, tile_masks, reorder_rows, rows, schedule, out, epi, stream, ready, 2);
#undef LATTICE_IGEMM_CASE
#undef LATTICE_IGEMM_LAUNCH
    default:
        set_error("implicit GEMM supports c_out in {16, 32, 64, 128, 256}.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
}

// Shapes the streamed kernel takes: fp16/bf16, C_in a multiple of 32 up to
// 256, C_out in {64, 128, 256}, K <= 32, and a feature table whose byte
// offsets (with the wrapped -1 rows above them) fit 32 bits.
bool stream_shape_ok(long long n_in, int c_in, int c_out, int K) {
    const long long row_bytes = static_cast<long long>(c_in) * 2;
    return c_in > 0 && c_in % 32 == 0 && c_in <= 256 && K > 0 && K <= 32 &&
           (c_out == 64 || c_out == 128 || c_out == 256) && n_in >= 0 && (n_in + 1) * row_bytes <= (1ll << 32);
}

size_t fragments_bytes(int K, int c_in, int c_out) {
    return static_cast<size_t>(K) * static_cast<size_t>(c_in) * static_cast<size_t>(c_out) * 2;
}

template <typename T, typename S, int NCH, int QB>
void launch_stream_nch(const T* feats, int n_in, int c_in, const T* frag, int K, int c_out, const int32_t* kv_map,
                       const int32_t* tile_masks, const int32_t* reorder_rows, int rows, const int32_t* order, T* out,
                       Epilogue<T> epi, int halves, hipStream_t stream) {
    const int tiles = (rows + S::ROWS - 1) / S::ROWS;
    conv_igemm_stream<T, S, NCH, QB><<<static_cast<unsigned>(tiles * halves), S::THREADS, 0, stream>>>(
        feats, n_in, c_in, frag, K, c_out, kv_map, tile_masks, reorder_rows, rows, order, out, epi, halves);
}

template <typename T, typename S, int QB>
void launch_stream_shape(const T* feats, int n_in, int c_in, const T* frag, int K, int c_out, const int32_t* kv_map,
                         const int32_t* tile_masks, const int32_t* reorder_rows, int rows, const int32_t* order,
                         T* out, Epilogue<T> epi, int halves, hipStream_t stream) {
    switch ((c_in + S::CHUNK - 1) / S::CHUNK) {
    case 1:
        launch_stream_nch<T, S, 1, QB>(feats, n_in, c_in, frag, K, c_out, kv_map, tile_masks, reorder_rows, rows, order,
                                   out, epi, halves, stream);
        break;
    case 2:
        launch_stream_nch<T, S, 2, QB>(feats, n_in, c_in, frag, K, c_out, kv_map, tile_masks, reorder_rows, rows, order,
                                   out, epi, halves, stream);
        break;
    case 3:
        launch_stream_nch<T, S, 3, QB>(feats, n_in, c_in, frag, K, c_out, kv_map, tile_masks, reorder_rows, rows, order,
                                   out, epi, halves, stream);
        break;
    default:
        launch_stream_nch<T, S, 4, QB>(feats, n_in, c_in, frag, K, c_out, kv_map, tile_masks, reorder_rows, rows, order,
                                   out, epi, halves, stream);
        break;
    }
}

template <typename T, int QB = 0>
int launch_stream(const T* feats, int n_in, int c_in, const T* frag, int K, int c_out, const int32_t* kv_map,
                  const int32_t* tile_masks, const int32_t* reorder_rows, int rows, int32_t* schedule, bool ready,
                  T* out, Epilogue<T> epi, hipStream_t stream) {
    if (rows <= 0) return LATTICE_OK;
    const int tiles = (rows + kOrderTileRows - 1) / kOrderTileRows;
    if (tiles > kMaxScheduledTiles) schedule = nullptr;
    if (schedule != nullptr && !ready) {
        schedule_tiles<kOrderTileRows / 16><<<1, kScheduleThreads, 0, stream>>>(tile_masks, rows, tiles, schedule);
        LATTICE_LAUNCH_CHECK();
    }
    if (c_out == 64) {
        launch_stream_shape<T, StreamShape<64, 2>, QB>(feats, n_in, c_in, frag, K, c_out, kv_map, tile_masks,
                                                   reorder_rows, rows, schedule, out, epi, 1, stream);
    } else {
        launch_stream_shape<T, StreamShape<128, 1>, QB>(feats, n_in, c_in, frag, K, c_out, kv_map, tile_masks,
                                                    reorder_rows, rows, schedule, out, epi, c_out == 256 ? 2 : 1,
                                                    stream);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

// Workspace of the matrix-core conv: the tile schedule, one int per row
// tile (tiles are at least 64 rows).  NULL workspace = tiles in order.
// With LATTICE_CONV_ORDER_READY in workspace_bytes the workspace already
// holds the order (lattice_hip_conv_tile_order) and is only read.
size_t conv_schedule_bytes(int rows) { return (static_cast<size_t>(std::max(rows, 0)) / 64 + 1) * sizeof(int32_t); }

int conv_schedule(void* workspace, size_t workspace_bytes, int rows, int32_t** schedule, bool* ready) {
    *schedule = nullptr;
    *ready = false;
    if (workspace == nullptr) return LATTICE_OK;
    const bool given = (workspace_bytes & LATTICE_CONV_ORDER_READY) != 0;
    workspace_bytes &= ~static_cast<size_t>(LATTICE_CONV_ORDER_READY);
    LATTICE_REQUIRE(workspace_bytes >= conv_schedule_bytes(rows), "conv workspace too small.");
    *schedule = static_cast<int32_t*>(workspace);
    *ready = given;
    return LATTICE_OK;
}

// Shapes the matrix-core kernel handles; the feature table must also fit
// the 32-bit offsets of its buffer loads (under 2 GiB).
bool igemm_shape_ok(int n_in, int c_in, int c_out, int K) {
    return c_in > 0 && c_in % 32 == 0 && c_in <= 512 && K > 0 && K <= 32 &&
           (c_out == 16 || c_out == 32 || c_out == 64 || c_out == 128 || c_out == 256) &&
           static_cast<long long>(n_in) * c_in * 2 < (1ll << 31);
}

int check_dtype(int dtype) {
    LATTICE_REQUIRE(dtype == LATTICE_F32 || dtype == LATTICE_F16 || dtype == LATTICE_BF16,
                    "convolution supports float32, float16 and bfloat16 features.");
    return LATTICE_OK;
}

}  // namespace
}  // namespace lattice

using namespace lattice;

extern "C" size_t lattice_hip_conv_workspace_bytes(int out_capacity) { return conv_schedule_bytes(out_capacity); }

extern "C" int lattice_hip_conv_tile_order(const int32_t* tile_masks, int out_capacity, int32_t* order,
                                           size_t order_bytes, void* stream_ptr) {
    LATTICE_REQUIRE(out_capacity >= 0, "out_capacity must be nonnegative.");
    LATTICE_REQUIRE(order != nullptr && (tile_masks != nullptr || out_capacity == 0),
                    "tile order pointers must be non-null.");
    LATTICE_REQUIRE(order_bytes >= conv_schedule_bytes(out_capacity), "tile order buffer too small.");
    const int blocks = (out_capacity + kOrderTileRows - 1) / kOrderTileRows;
    if (blocks == 0 || blocks > kMaxScheduledTiles) return LATTICE_OK;  // such launches run tiles in order
    schedule_tiles<kOrderTileRows / 16><<<1, kScheduleThreads, 0, as_stream(stream_ptr)>>>(tile_masks, out_capacity,
                                                                                         blocks, order);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_sparse_conv_features(int dtype, const void* feats, int n_in, int c_in,
                                                const void* weights, int weight_layout, int kernel_count,
                                                int c_out, const int32_t* in_rows, const int32_t* kernel_ids,
                                                const int32_t* counts, int edge_capacity,
                                                const int32_t* row_offsets, int out_capacity, void* out,
                                                const void* bias, int epilogue, void* stream_ptr) {
    LATTICE_REQUIRE((epilogue & ~LATTICE_EPILOGUE_RELU) == 0, "unknown conv epilogue flags.");
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
    const long long nw = static_cast<long long>(kernel_count) * c_in * c_out;
    if (csr_rows_ok(c_in, c_out, nw)) {
        const QuantIndex none{};
        const unsigned rgrid = grid_for(out_capacity, 256, 1u << 16);
        const size_t rlds = static_cast<size_t>(nw + 4 * kernel_count) * sizeof(float);
#define LATTICE_CSR_ROWS(T, CO)                                                                                   \
    conv_csr_rows<T, CO, false><<<rgrid, 256, rlds, stream>>>(                                                    \
        static_cast<const T*>(feats), c_in, static_cast<const T*>(weights), widx, nullptr, nullptr, nullptr, none, \
        in_rows, kernel_ids, counts, edge_capacity, row_offsets, out_capacity, static_cast<T*>(out),             \
        epilogue_of<T>(bias, epilogue))
        if (dtype == LATTICE_F32) {
            if (c_out == 16) LATTICE_CSR_ROWS(float, 16); else LATTICE_CSR_ROWS(float, 32);
        } else if (dtype == LATTICE_F16) {
            if (c_out == 16) LATTICE_CSR_ROWS(_Float16, 16); else LATTICE_CSR_ROWS(_Float16, 32);
        } else {
            if (c_out == 16) LATTICE_CSR_ROWS(__bf16, 16); else LATTICE_CSR_ROWS(__bf16, 32);
        }
#undef LATTICE_CSR_ROWS
        LATTICE_LAUNCH_CHECK();
        return LATTICE_OK;
    }
    const bool staged = nw <= kCsrLdsFloats;
    const unsigned grid = grid_for(total, 256, staged ? kCsrStagedBlocks : 1u << 16);
    const size_t lds = staged ? static_cast<size_t>(nw) * sizeof(float) : 0;
    if (dtype == LATTICE_F32) {
        conv_csr<float><<<grid, 256, lds, stream>>>(static_cast<const float*>(feats), c_in,
                                                  static_cast<const float*>(weights), widx, in_rows, kernel_ids,
                                                  counts, edge_capacity, row_offsets, out_capacity,
                                                  static_cast<float*>(out), epilogue_of<float>(bias, epilogue), staged);
    } else if (dtype == LATTICE_F16) {
        conv_csr<_Float16><<<grid, 256, lds, stream>>>(static_cast<const _Float16*>(feats), c_in,
                                                     static_cast<const _Float16*>(weights), widx, in_rows,
                                                     kernel_ids, counts, edge_capacity, row_offsets, out_capacity,
                                                     static_cast<_Float16*>(out),
                                                     epilogue_of<_Float16>(bias, epilogue), staged);
    } else {
        conv_csr<__bf16><<<grid, 256, lds, stream>>>(static_cast<const __bf16*>(feats), c_in,
                                                   static_cast<const __bf16*>(weights), widx, in_rows, kernel_ids,
                                                   counts, edge_capacity, row_offsets, out_capacity,
                                                   static_cast<__bf16*>(out), epilogue_of<__bf16>(bias, epilogue),
                                                   staged);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_sparse_conv_features_sorted_implicit_gemm(
    int dtype, const void* feats, int n_in, int c_in, const void* weights, int weight_layout, int kernel_count,
    int c_out, const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks, const int32_t* reorder_rows,
    int out_capacity, void* out, const void* bias, int epilogue, void* workspace, size_t workspace_bytes,
    void* stream_ptr) {
    LATTICE_REQUIRE((epilogue & ~LATTICE_EPILOGUE_RELU) == 0, "unknown conv epilogue flags.");
    int rc = check_dtype(dtype);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(dtype != LATTICE_F32, "the implicit GEMM route runs on fp16/bf16 matrix cores.");
    LATTICE_REQUIRE(n_in >= 0 && out_capacity >= 0, "feats must have shape (N, C_in).");
    LATTICE_REQUIRE(weight_layout == LATTICE_WEIGHT_DENSE_5D,
                    "the implicit GEMM route takes (C_out, Kx, Ky, Kz, C_in) weights.");
    if (!igemm_shape_ok(n_in, c_in, c_out, kernel_count)) {
        set_error("implicit GEMM needs c_in % 32 == 0 (<= 512), c_out in {16,32,64,128,256}, K <= 32 and "
                  "feats under 2 GiB.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
    LATTICE_REQUIRE(sorted_kv_out_in_map && tile_masks && out && weights && (feats || n_in == 0),
                    "conv pointers must be non-null.");
    int32_t* schedule = nullptr;
    bool ready = false;
    rc = conv_schedule(workspace, workspace_bytes, out_capacity, &schedule, &ready);
    if (rc != LATTICE_OK) return rc;
    hipStream_t stream = as_stream(stream_ptr);
    const long long s_co = static_cast<long long>(kernel_count) * c_in;
    const long long s_k = c_in;
    if (dtype == LATTICE_F16) {
        FloatB<_Float16> b{static_cast<const _Float16*>(weights), s_co, s_k};
        return launch_igemm<_Float16>(static_cast<const _Float16*>(feats), n_in, c_in, c_out, b, sorted_kv_out_in_map,
                                      tile_masks, reorder_rows, out_capacity, schedule, ready,
                                      static_cast<_Float16*>(out), epilogue_of<_Float16>(bias, epilogue), stream);
    }
    FloatB<__bf16> b{static_cast<const __bf16*>(weights), s_co, s_k};
    return launch_igemm<__bf16>(static_cast<const __bf16*>(feats), n_in, c_in, c_out, b, sorted_kv_out_in_map,
                                tile_masks, reorder_rows, out_capacity, schedule, ready, static_cast<__bf16*>(out),
                                epilogue_of<__bf16>(bias, epilogue), stream);
}

extern "C" size_t lattice_hip_conv_weight_fragments_bytes(int dtype, int kernel_count, int c_in, int c_out) {
    if (dtype != LATTICE_F16 && dtype != LATTICE_BF16) return 0;
    if (!stream_shape_ok(0, c_in, c_out, kernel_count)) return 0;
    return fragments_bytes(kernel_count, c_in, c_out);
}

extern "C" int lattice_hip_conv_weight_fragments(int dtype, const void* weights, int kernel_count, int c_in, int c_out,
                                                 void* fragments, size_t fragments_bytes_given, void* stream_ptr) {
    const size_t need = lattice_hip_conv_weight_fragments_bytes(dtype, kernel_count, c_in, c_out);
    if (need == 0) {
        set_error("weight fragments need fp16/bf16 weights with c_in % 32 == 0 (<= 256), c_out in {64, 128, 256} "
                  "and K <= 32.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
    LATTICE_REQUIRE(weights != nullptr && fragments != nullptr, "weight fragment pointers must be non-null.");
    LATTICE_REQUIRE(fragments_bytes_given >= need, "weight fragment buffer too small.");
    hipStream_t stream = as_stream(stream_ptr);
    const long long pieces = static_cast<long long>(need / 16);
    const unsigned grid = grid_for(pieces, 256, 1u << 14);
    if (dtype == LATTICE_F16) {
        weight_fragments<_Float16><<<grid, 256, 0, stream>>>(static_cast<const _Float16*>(weights), kernel_count,
                                                             c_in, c_out, static_cast<_Float16*>(fragments));
    } else {
        weight_fragments<__bf16><<<grid, 256, 0, stream>>>(static_cast<const __bf16*>(weights), kernel_count, c_in,
                                                           c_out, static_cast<__bf16*>(fragments));
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_sparse_conv_features_sorted_fragments(
    int dtype, const void* feats, int n_in, int c_in, const void* weight_fragments, int kernel_count, int c_out,
    const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks, const int32_t* reorder_rows, int out_capacity,
    void* out, const void* bias, int epilogue, void* workspace, size_t workspace_bytes, void* stream_ptr) {
    LATTICE_REQUIRE((epilogue & ~LATTICE_EPILOGUE_RELU) == 0, "unknown conv epilogue flags.");
    LATTICE_REQUIRE(dtype == LATTICE_F16 || dtype == LATTICE_BF16,
                    "the streamed matrix-core conv takes float16 or bfloat16 features.");
    LATTICE_REQUIRE(n_in >= 0 && out_capacity >= 0, "feats must have shape (N, C_in).");
    if (!stream_shape_ok(n_in, c_in, c_out, kernel_count)) {
        set_error("the streamed conv needs c_in % 32 == 0 (<= 256), c_out in {64, 128, 256}, K <= 32 and feats "
                  "under 4 GiB.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
    LATTICE_REQUIRE(sorted_kv_out_in_map && tile_masks && out && weight_fragments && (feats || n_in == 0),
                    "conv pointers must be non-null.");
    int32_t* schedule = nullptr;
    bool ready = false;
    int rc = conv_schedule(workspace, workspace_bytes, out_capacity, &schedule, &ready);
    if (rc != LATTICE_OK) return rc;
    hipStream_t stream = as_stream(stream_ptr);
    if (dtype == LATTICE_F16) {
        return launch_stream<_Float16>(static_cast<const _Float16*>(feats), n_in, c_in,
                                       static_cast<const _Float16*>(weight_fragments), kernel_count, c_out,
                                       sorted_kv_out_in_map, tile_masks, reorder_rows, out_capacity, schedule, ready,
                                       static_cast<_Float16*>(out), epilogue_of<_Float16>(bias, epilogue), stream);
    }
    return launch_stream<__bf16>(static_cast<const __bf16*>(feats), n_in, c_in,
                                 static_cast<const __bf16*>(weight_fragments), kernel_count, c_out,
                                 sorted_kv_out_in_map, tile_masks, reorder_rows, out_capacity, schedule, ready,
                                 static_cast<__bf16*>(out), epilogue_of<__bf16>(bias, epilogue), stream);
}

extern "C" size_t lattice_hip_quantized_weight_fragments_bytes(int dtype, int kernel_count, int c_in, int c_out) {
    return lattice_hip_conv_weight_fragments_bytes(dtype, kernel_count, c_in, c_out);
}

extern "C" int lattice_hip_quantized_weight_fragments(int dtype, const uint32_t* weights, const void* scales,
                                                      const void* biases, int kernel_count, int c_in, int c_out,
                                                      int storage_c_in, int group_size, int bits, void* fragments,
                                                      size_t fragments_bytes_given, void* stream_ptr) {
    const size_t need = lattice_hip_quantized_weight_fragments_bytes(dtype, kernel_count, c_in, c_out);
    if (need == 0) {
        set_error("quantized weight fragments need fp16/bf16 scales with c_in % 32 == 0 (<= 256), c_out in "
                  "{64, 128, 256} and K <= 32.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
    LATTICE_REQUIRE(bits == 4 || bits == 8, "quantized weight bits must be 4 or 8.");
    LATTICE_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
                    "quantized weight group_size must be 32, 64, or 128.");
    LATTICE_REQUIRE(storage_c_in >= c_in && storage_c_in % group_size == 0, "quantized weight channel metadata is invalid.");
    LATTICE_REQUIRE(weights != nullptr && scales != nullptr && biases != nullptr && fragments != nullptr,
                    "quantized weight fragment pointers must be non-null.");
    LATTICE_REQUIRE(fragments_bytes_given >= need, "quantized weight fragment buffer too small.");
    hipStream_t stream = as_stream(stream_ptr);
    const long long pieces = static_cast<long long>(need / 16);
    const unsigned grid = grid_for(pieces, 256, 1u << 14);
    const int packed_words = storage_c_in * bits / 32;
    const int groups = storage_c_in / group_size;
    if (dtype == LATTICE_F16) {
        packed_weight_fragments<_Float16><<<grid, 256, 0, stream>>>(
            weights, static_cast<const _Float16*>(scales), static_cast<const _Float16*>(biases), kernel_count, c_in,
            c_out, packed_words, groups, group_size, bits, static_cast<uint4*>(fragments));
    } else {
        packed_weight_fragments<__bf16><<<grid, 256, 0, stream>>>(
            weights, static_cast<const __bf16*>(scales), static_cast<const __bf16*>(biases), kernel_count, c_in,
            c_out, packed_words, groups, group_size, bits, static_cast<uint4*>(fragments));
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_sparse_quantized_conv_features_sorted_fragments(
    int dtype, const void* feats, int n_in, int c_in, const void* weight_fragments, int bits, int kernel_count,
    int c_out, const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks, const int32_t* reorder_rows,
    int out_capacity, void* out, const void* bias, int epilogue, void* workspace, size_t workspace_bytes,
    void* stream_ptr) {
    LATTICE_REQUIRE((epilogue & ~LATTICE_EPILOGUE_RELU) == 0, "unknown conv epilogue flags.");
    LATTICE_REQUIRE(dtype == LATTICE_F16 || dtype == LATTICE_BF16,
                    "the streamed matrix-core conv takes float16 or bfloat16 features.");
    LATTICE_REQUIRE(bits == 4 || bits == 8, "quantized convolution bits must be 4 or 8.");
    LATTICE_REQUIRE(n_in >= 0 && out_capacity >= 0, "feats must have shape (N, C_in).");
    if (!stream_shape_ok(n_in, c_in, c_out, kernel_count)) {
        set_error("the streamed conv needs c_in % 32 == 0 (<= 256), c_out in {64, 128, 256}, K <= 32 and feats "
                  "under 4 GiB.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
    LATTICE_REQUIRE(sorted_kv_out_in_map && tile_masks && out && weight_fragments && (feats || n_in == 0),
                    "conv pointers must be non-null.");
    int32_t* schedule = nullptr;
    bool ready = false;
    int rc = conv_schedule(workspace, workspace_bytes, out_capacity, &schedule, &ready);
    if (rc != LATTICE_OK) return rc;
    hipStream_t stream = as_stream(stream_ptr);
    if (dtype == LATTICE_F16) {
        auto* f = static_cast<const _Float16*>(feats);
        auto* w = static_cast<const _Float16*>(weight_fragments);
        auto* o = static_cast<_Float16*>(out);
        const Epilogue<_Float16> epi = epilogue_of<_Float16>(bias, epilogue);
        return bits == 4 ? launch_stream<_Float16, 4>(f, n_in, c_in, w, kernel_count, c_out, sorted_kv_out_in_map,
                                                       tile_masks, reorder_rows, out_capacity, schedule, ready, o,
                                                       epi, stream)
                         : launch_stream<_Float16, 8>(f, n_in, c_in, w, kernel_count, c_out, sorted_kv_out_in_map,
                                                       tile_masks, reorder_rows, out_capacity, schedule, ready, o,
                                                       epi, stream);
    }
    auto* f = static_cast<const __bf16*>(feats);
    auto* w = static_cast<const __bf16*>(weight_fragments);
    auto* o = static_cast<__bf16*>(out);
    const Epilogue<__bf16> epi = epilogue_of<__bf16>(bias, epilogue);
    return bits == 4 ? launch_stream<__bf16, 4>(f, n_in, c_in, w, kernel_count, c_out, sorted_kv_out_in_map,
                                                 tile_masks, reorder_rows, out_capacity, schedule, ready, o, epi,
                                                 stream)
                     : launch_stream<__bf16, 8>(f, n_in, c_in, w, kernel_count, c_out, sorted_kv_out_in_map,
                                                 tile_masks, reorder_rows, out_capacity, schedule, ready, o, epi,
                                                 stream);
}

// ------------------------------------------------- allocation-free entry --
//
// The tile schedule of lattice_hip_sparse_conv_features_sorted_implicit_gemm
// for callers that cannot allocate (code under graph capture, serving loops
// that forbid hipMalloc): a file-scope device array of kMaxScheduledTiles
// ints (128 KiB), one copy per GPU, resident until the process ends.  Its
// address on each device is taken once, with the device current, through
// hipGetSymbolAddress; in host code the array's own name is only a
// host-side stand-in and is never passed to a kernel.  schedule_tiles
// writes every entry a launch reads, so nothing needs clearing.
//
// Calls on one GPU share the array.  Outside graph capture they are put in
// submission order: each call's stream first waits for the event recorded
// after the previous call on that device (whatever its stream), and records
// it again after its own launches, under a per-device host mutex; the event
// is created once per device at the first call.  A call made while its
// stream is being captured neither waits nor records (an event recorded
// outside the capture cannot be waited on inside it), so replays of a
// captured graph that overlap another caller's use of the device race.

namespace lattice {
namespace {

static __device__ __align__(256) int32_t scratch[kMaxScheduledTiles];

constexpr int kMaxScratchDevices = 64;
std::atomic<int32_t*> g_scratch_ptr[kMaxScratchDevices];

// Per-device order of the calls that use the scratch.
struct ScratchOrder {
    std::mutex lock;
    hipEvent_t last_use = nullptr;  // recorded after the latest call's launches
    bool recorded = false;
};
ScratchOrder g_scratch_order[kMaxScratchDevices];

// The scratch of the current device, which must be the stream's device
// (hipGetSymbolAddress answers for the current device).
int scratch_on_current_device(hipStream_t stream, int32_t** ptr, int* device_out) {
    int device = 0;
    LATTICE_HIP_TRY(hipGetDevice(&device));
    if (stream != nullptr) {
        int stream_device = 0;
        LATTICE_HIP_TRY(hipStreamGetDevice(stream, &stream_device));
        LATTICE_REQUIRE(stream_device == device,
                        "the allocation-free conv's stream belongs to another device than the current one.");
    }
    LATTICE_REQUIRE(device >= 0 && device < kMaxScratchDevices, "device index out of range for the conv scratch.");
    int32_t* p = g_scratch_ptr[device].load(std::memory_order_acquire);
    if (p == nullptr) {
        LATTICE_HIP_TRY(hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(scratch)));
        g_scratch_ptr[device].store(p, std::memory_order_release);
    }
    *ptr = p;
    *device_out = device;
    return LATTICE_OK;
}

}  // namespace
}  // namespace lattice

extern "C" int lattice_hip_sparse_conv_features_sorted_implicit_gemm_noalloc(
    int dtype, const void* feats, int n_in, int c_in, const void* weights, int weight_layout, int kernel_count,
    int c_out, const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks, const int32_t* reorder_rows,
    int out_capacity, void* out, const void* bias, int epilogue, void* stream_ptr) {
    LATTICE_REQUIRE(out_capacity <= LATTICE_NOALLOC_CONV_MAX_ROWS,
                    "out_capacity exceeds the allocation-free conv's limit of " +
                        std::to_string(LATTICE_NOALLOC_CONV_MAX_ROWS) +
                        " rows; use lattice_hip_sparse_conv_features_sorted_implicit_gemm with a workspace.");
    static_assert(static_cast<size_t>(LATTICE_NOALLOC_CONV_MAX_ROWS) / 64 + 1 <= kMaxScheduledTiles,
                  "the scratch holds the schedule of the largest allowed launch");
    int32_t* schedule = nullptr;
    int device = 0;
    const hipStream_t stream = as_stream(stream_ptr);
    int rc = scratch_on_current_device(stream, &schedule, &device);
    if (rc != LATTICE_OK) return rc;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    LATTICE_HIP_TRY(hipStreamIsCapturing(stream, &capture));
    const bool ordered = capture == hipStreamCaptureStatusNone;
    ScratchOrder& order = g_scratch_order[device];
    std::lock_guard<std::mutex> guard(order.lock);
    if (ordered) {
        if (order.last_use == nullptr)
            LATTICE_HIP_TRY(hipEventCreateWithFlags(&order.last_use, hipEventDisableTiming));
        if (order.recorded) LATTICE_HIP_TRY(hipStreamWaitEvent(stream, order.last_use, 0));
    }
    rc = lattice_hip_sparse_conv_features_sorted_implicit_gemm(
        dtype, feats, n_in, c_in, weights, weight_layout, kernel_count, c_out, sorted_kv_out_in_map, tile_masks,
        reorder_rows, out_capacity, out, bias, epilogue, schedule, sizeof(scratch), stream_ptr);
    if (rc == LATTICE_OK && ordered) {
        LATTICE_HIP_TRY(hipEventRecord(order.last_use, stream));
        order.recorded = true;
    }
    return rc;
}

extern "C" int lattice_hip_sparse_quantized_conv_features(
    int dtype, const void* feats, int n_in, int c_in, const uint32_t* weights, const void* scales,
    const void* biases, int kernel_count, int c_out, int storage_c_in, int group_size, int bits,
    const int32_t* in_rows, const int32_t* kernel_ids, const int32_t* counts, int edge_capacity,
    const int32_t* row_offsets, const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks,
    const int32_t* reorder_rows, int out_capacity, void* out, const void* bias, int epilogue, void* workspace,
    size_t workspace_bytes, void* stream_ptr) {
    LATTICE_REQUIRE((epilogue & ~LATTICE_EPILOGUE_RELU) == 0, "unknown conv epilogue flags.");
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
    const bool sorted = sorted_kv_out_in_map != nullptr && tile_masks != nullptr && reorder_rows != nullptr;
    if (sorted && dtype != LATTICE_F32 && igemm_shape_ok(n_in, c_in, c_out, kernel_count)) {
        int32_t* schedule = nullptr;
        bool ready = false;
        rc = conv_schedule(workspace, workspace_bytes, out_capacity, &schedule, &ready);
        if (rc != LATTICE_OK) return rc;
        if (dtype == LATTICE_F16) {
            PackedB<_Float16> b{weights, static_cast<const _Float16*>(scales), static_cast<const _Float16*>(biases),
                                packed_words, groups, group_size, c_out, bits};
            return launch_igemm<_Float16>(static_cast<const _Float16*>(feats), n_in, c_in, c_out, b, sorted_kv_out_in_map,
                                          tile_masks, reorder_rows, out_capacity, schedule, ready,
                                          static_cast<_Float16*>(out), epilogue_of<_Float16>(bias, epilogue), stream);
        }
        PackedB<__bf16> b{weights, static_cast<const __bf16*>(scales), static_cast<const __bf16*>(biases),
                          packed_words, groups, group_size, c_out, bits};
        return launch_igemm<__bf16>(static_cast<const __bf16*>(feats), n_in, c_in, c_out, b, sorted_kv_out_in_map,
                                    tile_masks, reorder_rows, out_capacity, schedule, ready, static_cast<__bf16*>(out),
                                    epilogue_of<__bf16>(bias, epilogue), stream);
    }
    LATTICE_REQUIRE(in_rows && kernel_ids && counts && row_offsets, "relation pointers must be non-null.");
    QuantIndex q{kernel_count, c_in, c_out, packed_words, groups, group_size, bits};
    const long long nw = static_cast<long long>(kernel_count) * c_in * c_out;
    if (csr_rows_ok(c_in, c_out, nw)) {
        const WeightIndex none{};
        const unsigned rgrid = grid_for(out_capacity, 256, 1u << 16);
        const size_t rlds = static_cast<size_t>(nw + 4 * kernel_count) * sizeof(float);
#define LATTICE_QCSR_ROWS(T, CO)                                                                                 \
    conv_csr_rows<T, CO, true><<<rgrid, 256, rlds, stream>>>(                                                    \
        static_cast<const T*>(feats), c_in, nullptr, none, weights, static_cast<const T*>(scales),              \
        static_cast<const T*>(biases), q, in_rows, kernel_ids, counts, edge_capacity, row_offsets, out_capacity, \
        static_cast<T*>(out), epilogue_of<T>(bias, epilogue))
        if (dtype == LATTICE_F32) {
            if (c_out == 16) LATTICE_QCSR_ROWS(float, 16); else LATTICE_QCSR_ROWS(float, 32);
        } else if (dtype == LATTICE_F16) {
            if (c_out == 16) LATTICE_QCSR_ROWS(_Float16, 16); else LATTICE_QCSR_ROWS(_Float16, 32);
        } else {
            if (c_out == 16) LATTICE_QCSR_ROWS(__bf16, 16); else LATTICE_QCSR_ROWS(__bf16, 32);
        }
#undef LATTICE_QCSR_ROWS
        LATTICE_LAUNCH_CHECK();
        return LATTICE_OK;
    }
    const bool staged = nw <= kCsrLdsFloats;
    const unsigned grid =
        grid_for(static_cast<long long>(out_capacity) * c_out, 256, staged ? kCsrStagedBlocks : 1u << 16);
    const size_t lds = staged ? static_cast<size_t>(nw) * sizeof(float) : 0;
    if (dtype == LATTICE_F32) {
        quant_conv_csr<float><<<grid, 256, lds, stream>>>(
            static_cast<const float*>(feats), weights, static_cast<const float*>(scales),
            static_cast<const float*>(biases), q, in_rows, kernel_ids, counts, edge_capacity, row_offsets,
            out_capacity, static_cast<float*>(out), epilogue_of<float>(bias, epilogue), staged);
    } else if (dtype == LATTICE_F16) {
        quant_conv_csr<_Float16><<<grid, 256, lds, stream>>>(
            static_cast<const _Float16*>(feats), weights, static_cast<const _Float16*>(scales),
            static_cast<const _Float16*>(biases), q, in_rows, kernel_ids, counts, edge_capacity, row_offsets,
            out_capacity, static_cast<_Float16*>(out), epilogue_of<_Float16>(bias, epilogue), staged);
    } else {
        quant_conv_csr<__bf16><<<grid, 256, lds, stream>>>(
            static_cast<const __bf16*>(feats), weights, static_cast<const __bf16*>(scales),
            static_cast<const __bf16*>(biases), q, in_rows, kernel_ids, counts, edge_capacity, row_offsets,
            out_capacity, static_cast<__bf16*>(out), epilogue_of<__bf16>(bias, epilogue), staged);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_sparse_conv_features_expand(int dtype, const void* feats, int n_in,
                                                       const int32_t* active_rows, int c_in, const void* weights,
                                                       int kernel_count, int c_out, void* out, const void* bias, int epilogue,
                                                       void* stream_ptr) {
    LATTICE_REQUIRE((epilogue & ~LATTICE_EPILOGUE_RELU) == 0, "unknown conv epilogue flags.");
    int rc = check_dtype(dtype);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(dtype != LATTICE_F32, "the expansion conv runs on fp16/bf16 matrix cores.");
    LATTICE_REQUIRE(n_in >= 0 && kernel_count > 0, "feats must have shape (N, C_in) and n_kernels be positive.");
    LATTICE_REQUIRE(static_cast<long long>(n_in) * kernel_count < (1ll << 31), "expanded rows exceed int32.");
    if (n_in == 0) return LATTICE_OK;
    LATTICE_REQUIRE(feats && weights && out && active_rows, "conv pointers must be non-null.");
    hipStream_t stream = as_stream(stream_ptr);
    if (dtype == LATTICE_F16) {
        return launch_expand<_Float16>(static_cast<const _Float16*>(feats), n_in, active_rows, c_in,
                                       static_cast<const _Float16*>(weights), kernel_count, c_out,
                                       static_cast<_Float16*>(out), epilogue_of<_Float16>(bias, epilogue), stream);
    }
    return launch_expand<__bf16>(static_cast<const __bf16*>(feats), n_in, active_rows, c_in,
                                 static_cast<const __bf16*>(weights), kernel_count, c_out,
                                 static_cast<__bf16*>(out), epilogue_of<__bf16>(bias, epilogue), stream);
}

// ------------------------------------------------- dense-map small C_in --

namespace lattice {
namespace {

bool dense_map_shape_ok(int dtype, int c_in, int c_out, int kernel_count) {
    return (dtype == LATTICE_F16 || dtype == LATTICE_BF16) && (c_in == 4 || c_in == 8) &&
           (c_out == 16 || c_out == 32) && kernel_count > 0 && kernel_count * c_in <= 256;
}

template <typename T, bool QUANT>
int launch_dense_map(const void* feats, int n_in, int c_in, const void* fweights, WeightIndex widx,
                     const uint32_t* qweights, const void* scales, const void* qbiases, QuantIndex q, int K,
                     const int32_t* out_in_map, const int32_t* counts, int out_capacity, void* out,
                     const void* bias, int epilogue, hipStream_t stream) {
    const long long waves = (static_cast<long long>(out_capacity) + 15) / 16;
    // Blocks: each builds the weight's fragments once, then its waves walk
    // 16-row blocks grid-stride.  1,024 blocks (four per CU) measured
    // fastest on the config-5 stem: 40 us, against 44 / 46 / 51 / 65 us at
    // 2,048 / 512 / 4,096 / 8,192.
    const unsigned grid = static_cast<unsigned>(std::max<long long>(1, std::min<long long>((waves + 3) / 4, 1024)));
    const T* f = static_cast<const T*>(feats);
    const Epilogue<T> epi = epilogue_of<T>(bias, epilogue);
#define LATTICE_DENSE_MAP(CI, CO, KS)                                                                            \
    conv_dense_map<T, CI, CO, QUANT, KS><<<grid, 256, 0, stream>>>(                                             \
        f, n_in, static_cast<const T*>(fweights), widx, qweights, static_cast<const T*>(scales),              \
        static_cast<const T*>(qbiases), q, K, out_in_map, counts, out_capacity, static_cast<T*>(out), epi)
    const bool short_k = K * c_in <= 128;  // at most four 32-wide steps (e.g. 27 offsets x 4 channels)
    if (c_in == 4) {
        if (q.c_out == 16) {
            if (short_k) LATTICE_DENSE_MAP(4, 16, 4); else LATTICE_DENSE_MAP(4, 16, 8);
        } else {
            if (short_k) LATTICE_DENSE_MAP(4, 32, 4); else LATTICE_DENSE_MAP(4, 32, 8);
        }
    } else {
        if (q.c_out == 16) {
            if (short_k) LATTICE_DENSE_MAP(8, 16, 4); else LATTICE_DENSE_MAP(8, 16, 8);
        } else {
            if (short_k) LATTICE_DENSE_MAP(8, 32, 4); else LATTICE_DENSE_MAP(8, 32, 8);
        }
    }
#undef LATTICE_DENSE_MAP
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

int dense_map_common_checks(int dtype, const void* feats, int n_in, int c_in, int c_out, int kernel_count,
                            const int32_t* out_in_map, const int32_t* counts, int out_capacity, void* out,
                            int epilogue) {
    LATTICE_REQUIRE((epilogue & ~LATTICE_EPILOGUE_RELU) == 0, "unknown conv epilogue flags.");
    LATTICE_REQUIRE(dense_map_shape_ok(dtype, c_in, c_out, kernel_count),
                    "the dense-map conv takes float16/bfloat16 features with C_in 4 or 8, C_out 16 or 32 and "
                    "K * C_in <= 256.");
    LATTICE_REQUIRE(n_in >= 0 && out_capacity >= 0, "feats and out_capacity must be nonnegative.");
    LATTICE_REQUIRE(out_capacity == 0 || (out_in_map && counts && out), "dense-map conv pointers must be non-null.");
    LATTICE_REQUIRE(n_in == 0 || feats != nullptr, "feats must be non-null.");
    LATTICE_REQUIRE(reinterpret_cast<uintptr_t>(feats) % (static_cast<size_t>(c_in) * 2) == 0,
                    "the dense-map conv needs feature rows aligned to their size.");
    return LATTICE_OK;
}

}  // namespace
}  // namespace lattice

extern "C" int lattice_hip_conv_dense_map_supported(int dtype, int c_in, int c_out, int kernel_count) {
    return lattice::dense_map_shape_ok(dtype, c_in, c_out, kernel_count) ? 1 : 0;
}

extern "C" int lattice_hip_sparse_conv_features_dense_map(int dtype, const void* feats, int n_in, int c_in,
                                                         const void* weights, int weight_layout, int kernel_count,
                                                         int c_out, const int32_t* out_in_map,
                                                         const int32_t* counts, int out_capacity, void* out,
                                                         const void* bias, int epilogue, void* stream_ptr) {
    int rc = dense_map_common_checks(dtype, feats, n_in, c_in, c_out, kernel_count, out_in_map, counts,
                                     out_capacity, out, epilogue);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(weight_layout == LATTICE_WEIGHT_KERNEL_MAJOR || weight_layout == LATTICE_WEIGHT_DENSE_5D,
                    "unknown weight layout.");
    LATTICE_REQUIRE(weights != nullptr, "weights must be non-null.");
    if (out_capacity == 0) return LATTICE_OK;
    const WeightIndex widx{weight_layout, kernel_count, c_in, c_out};
    const QuantIndex q{kernel_count, c_in, c_out, 0, 0, 0, 0};
    if (dtype == LATTICE_F16)
        return launch_dense_map<_Float16, false>(feats, n_in, c_in, weights, widx, nullptr, nullptr, nullptr, q,
                                                 kernel_count, out_in_map, counts, out_capacity, out, bias, epilogue,
                                                 as_stream(stream_ptr));
    return launch_dense_map<__bf16, false>(feats, n_in, c_in, weights, widx, nullptr, nullptr, nullptr, q,
                                           kernel_count, out_in_map, counts, out_capacity, out, bias, epilogue,
                                           as_stream(stream_ptr));
}

extern "C" int lattice_hip_sparse_quantized_conv_features_dense_map(
    int dtype, const void* feats, int n_in, int c_in, const uint32_t* weights, const void* scales,
    const void* biases, int kernel_count, int c_out, int storage_c_in, int group_size, int bits,
    const int32_t* out_in_map, const int32_t* counts, int out_capacity, void* out, const void* bias, int epilogue,
    void* stream_ptr) {
    int rc = dense_map_common_checks(dtype, feats, n_in, c_in, c_out, kernel_count, out_in_map, counts,
                                     out_capacity, out, epilogue);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(bits == 4 || bits == 8, "quantized convolution bits must be 4 or 8.");
    LATTICE_REQUIRE(group_size == 32 || group_size == 64 || group_size == 128,
                    "quantized convolution group_size must be 32, 64, or 128.");
    LATTICE_REQUIRE(storage_c_in >= c_in && storage_c_in % group_size == 0,
                    "quantized convolution channel metadata is invalid.");
    LATTICE_REQUIRE(weights && scales && biases, "quantized conv pointers must be non-null.");
    if (out_capacity == 0) return LATTICE_OK;
    const QuantIndex q{kernel_count, c_in, c_out, storage_c_in * bits / 32, storage_c_in / group_size, group_size,
                       bits};
    const WeightIndex none{};
    if (dtype == LATTICE_F16)
        return launch_dense_map<_Float16, true>(feats, n_in, c_in, nullptr, none, weights, scales, biases, q,
                                                kernel_count, out_in_map, counts, out_capacity, out, bias, epilogue,
                                                as_stream(stream_ptr));
    return launch_dense_map<__bf16, true>(feats, n_in, c_in, nullptr, none, weights, scales, biases, q, kernel_count,
                                          out_in_map, counts, out_capacity, out, bias, epilogue,
                                          as_stream(stream_ptr));
}
