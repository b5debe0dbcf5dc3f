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
//
// Block = 4 waves.  Each wave owns 64 consecutive rows of the mask-sorted
// order and WAVE_COLS = min(C_OUT, 128) output channels, so its fp32
// accumulators (64 x WAVE_COLS) live in registers for the whole kernel.
// The pipeline walks stages (k, 128-channel chunk of C_in) over the offsets
// any row of the block uses:
//   * B = W[k][co][chunk] is staged once per block into one of two LDS
//     buffers while the previous stage computes (loads issued before the
//     MFMAs, stored after them);
//   * A is gathered per wave straight from global memory into the MFMA
//     operand registers (16 bytes per lane per 32-channel step), zero where
//     the map says -1, so no LDS traffic or barrier is spent on A;
//   * a wave skips the MFMAs of offsets its own 64 rows never use (its mask
//     is the OR of its tile's four quarter masks).
// The epilogue stages the tile through LDS and writes whole output rows
// (16 bytes per lane) to out[reorder_rows[row]].

constexpr int kBlock = 256;
constexpr int kWaveRows = 64;
constexpr int kChunk = 128;  // input channels per pipeline stage
constexpr int kBPad = 8;     // halves of padding per staged B row (bank spread)

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

template <int C_OUT, int WAVE_ROWS> struct IgemmShape {
    static constexpr int WAVE_COLS = C_OUT < 128 ? C_OUT : 128;
    static constexpr int CG = C_OUT / WAVE_COLS;  // column groups
    static constexpr int RG = 4 / CG;             // row groups
    static constexpr int BLOCK_ROWS = WAVE_ROWS * RG;
    static constexpr int CB = WAVE_COLS / 16;     // 16-col blocks per wave
    static constexpr int RB = WAVE_ROWS / 16;     // 16-row blocks per wave
    static constexpr int ST = kChunk / 32;        // 32-channel steps per stage
    // Staged B: C_OUT rows of kChunk halves (256 bytes, sixteen 16-byte
    // pieces); piece p of row r lives at slot p ^ (r % 16), so the sixteen
    // rows read by one MFMA fragment hit sixteen different bank groups.
    static constexpr int BROW = kChunk;
    static constexpr int BBUF = C_OUT * BROW;     // one B buffer (halves)
    static constexpr int EROW = WAVE_COLS;        // epilogue row (halves, swizzled pieces)
    static constexpr int EPIECES = WAVE_COLS / 8;  // 16-byte pieces per epilogue row
    static constexpr int B_PIECES = C_OUT * kChunk / 8 / kBlock;  // 16-byte pieces per thread
    static constexpr int B_DMA = C_OUT / 16;      // direct loads per wave (4 rows each)
    static_assert(2 * WAVE_ROWS * EROW <= BBUF, "epilogue staging must fit one B buffer per wave pair");
};

__device__ inline int swizzle_piece(int piece, int row) { return piece ^ (row & 15); }

// B operand sources.  `load(k, co, ci0)` returns 8 consecutive input
// channels ci0..ci0+7 of W[k][:, co] as one 16-byte vector.
template <typename T> struct FloatB {
    static constexpr bool kDirect = true;  // staged with direct global->LDS loads
    const T* w;
    long long s_co, s_k;  // element strides; C_in is contiguous
    __device__ inline const T* ptr(int k, int co, int ci0) const { return w + co * s_co + k * s_k + ci0; }
    __device__ inline typename MfmaOps<T>::vec load(int k, int co, int ci0) const {
        return *reinterpret_cast<const typename MfmaOps<T>::vec*>(w + co * s_co + k * s_k + ci0);
    }
};

// Packed affine codes: w = q * scale + bias, dequantised while staging B.
template <typename T> struct PackedB {
    static constexpr bool kDirect = false;  // dequantised in registers, then stored
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

template <typename V>
__device__ inline V zero_vec() {
    V v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = 0;
    return v;
}

// Row indices of this wave's A operand for stage (k): rows row0 + 16*rb +
// lane%16 of the sorted order; -1 where there is no input row.
// Rows past the end re-read the last row; their result is never stored.
template <int RB>
__device__ inline void load_rows(int (&idx)[RB], const int32_t* __restrict__ kv_map, int rows, int row0, int k,
                                 int lr) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = min(row0 + rb * 16 + lr, rows - 1);
        idx[rb] = kv_map[static_cast<long long>(k) * rows + r];
    }
}

// A operand of one stage: RB x ST fragments of 16 bytes per lane (channels
// ci_base + 32*st + 8*(lane/16) .. +7).  Every lane issues the same loads
// on every stage (missing rows read row 0, steps past the chunk re-read its
// first step), so the loads in flight are the same on all paths and the
// compiler's waits stay partial; rows without input are zeroed at use.
template <typename T, typename V, int RB, int ST>
__device__ inline void load_a(V (&a)[RB][ST], const int (&idx)[RB], const T* __restrict__ feats, int c_in,
                              int ci_base, int cw, int lk) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const T* src = feats + static_cast<long long>(idx[rb] >= 0 ? idx[rb] : 0) * c_in + ci_base + lk;
#pragma unroll
        for (int st = 0; st < ST; ++st) {
            const int off = st * 32 < cw ? st * 32 : 0;
            a[rb][st] = *reinterpret_cast<const V*>(src + off);
        }
    }
}

constexpr int kMaxStages = 32 * 4;  // K <= 32 offsets x C_in <= 512 in 128-channel chunks

// Direct global->LDS staging of one B tile (float weights): each wave
// issues B_DMA loads; one load moves four 256-byte rows, lane l filling
// slot l%16 of row l/16 with the piece that the swizzle maps there.
template <typename T, int C_OUT, int WAVE_ROWS, typename BSource>
__device__ inline void stage_b_direct(const BSource& bsrc, int k, int ci0, int cw, T* dst, int wave, int lane) {
    using S = IgemmShape<C_OUT, WAVE_ROWS>;
#pragma unroll
    for (int i = 0; i < S::B_DMA; ++i) {
        const int r0 = (i * 4 + wave) * 4;
        const int row = r0 + (lane >> 4);
        const int piece = swizzle_piece(lane & 15, row);
        const int ci = piece * 8 < cw ? piece * 8 : 0;
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(bsrc.ptr(k, row, ci0 + ci)),
                                         (__attribute__((address_space(3))) void*)(dst + r0 * S::BROW),
                                         16, 0, 0);
    }
}

// Register staging of one B tile (packed weights, dequantised on load).
template <typename T, int C_OUT, int WAVE_ROWS, typename BSource, typename VT>
__device__ inline void stage_b_load(const BSource& bsrc, int k, int ci0, int cw,
                                    VT (&breg)[IgemmShape<C_OUT, WAVE_ROWS>::B_PIECES]) {
    using S = IgemmShape<C_OUT, WAVE_ROWS>;
#pragma unroll
    for (int i = 0; i < S::B_PIECES; ++i) {
        const int p = threadIdx.x + i * kBlock;
        const int co = p / (kChunk / 8);
        const int piece = p - co * (kChunk / 8);
        breg[i] = bsrc.load(k, co, ci0 + (piece * 8 < cw ? piece * 8 : 0));
    }
}

template <typename T, int C_OUT, int WAVE_ROWS, typename VT>
__device__ inline void stage_b_store(T* dst, const VT (&breg)[IgemmShape<C_OUT, WAVE_ROWS>::B_PIECES]) {
    using S = IgemmShape<C_OUT, WAVE_ROWS>;
#pragma unroll
    for (int i = 0; i < S::B_PIECES; ++i) {
        const int p = threadIdx.x + i * kBlock;
        const int co = p / (kChunk / 8);
        const int piece = p - co * (kChunk / 8);
        *reinterpret_cast<VT*>(dst + co * S::BROW + swizzle_piece(piece, co) * 8) = breg[i];
    }
}

// s_waitcnt immediate that waits until at most `n` vector-memory operations
// are outstanding and leaves the other counters alone (gfx9 encoding).
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | (((n >> 4) & 3) << 14); }

template <typename T>
__device__ inline uint32_t lds_address(const T* p) {
    return static_cast<uint32_t>(reinterpret_cast<size_t>((const __attribute__((address_space(3))) void*)p));
}

// Reads CB B fragments (16 bytes per lane, STRIDE bytes apart) from LDS and
// waits for them.  The reads are issued as inline assembly: the compiler
// would otherwise treat them as possibly aliasing the direct global->LDS
// loads in flight into the other B buffer and drain every vector-memory
// load first.  The buffer read here was completed by the explicit wait and
// barrier that ended the previous stage.  The empty asm statements tie the
// fragment registers to the wait so no MFMA can be scheduled above it.
template <typename V, int CB, int STRIDE>
__device__ inline void read_b_fragments(V (&b)[CB], uint32_t addr) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(b[cb]) : "v"(addr), "i"(cb * STRIDE));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) asm volatile("" : "+v"(b[cb]));
}

// One pipeline stage.  `bcur` holds this stage's B tile, `bnext` receives
// the next one; the caller alternates two distinct LDS arrays so the
// compiler can tell the direct loads into `bnext` from the reads of `bcur`.
template <typename T, int C_OUT, int WAVE_ROWS, typename BSource, typename V>
__device__ inline void igemm_stage(int s, int nstages, const unsigned char* stage_k, const unsigned char* stage_chunk,
                                   const T* __restrict__ bcur, T* __restrict__ bnext, const T* __restrict__ feats,
                                   int c_in,
                                   const BSource& bsrc, const int32_t* __restrict__ kv_map, int rows, int row0,
                                   int wave, int wc, int lane, uint32_t wmask,
                                   int (&idx_cur)[IgemmShape<C_OUT, WAVE_ROWS>::RB],
                                   int (&idx_next)[IgemmShape<C_OUT, WAVE_ROWS>::RB],
                                   V (&a_cur)[IgemmShape<C_OUT, WAVE_ROWS>::RB][IgemmShape<C_OUT, WAVE_ROWS>::ST],
                                   float4_t (&acc)[IgemmShape<C_OUT, WAVE_ROWS>::RB][IgemmShape<C_OUT, WAVE_ROWS>::CB]) {
    using S = IgemmShape<C_OUT, WAVE_ROWS>;
    const int lr = lane & 15;
    const int lk = (lane >> 4) * 8;
    const int s1 = min(s + 1, nstages - 1);
    const int s2 = min(s + 2, nstages - 1);
    const int k = stage_k[s];
    const int chunk = stage_chunk[s];
    const int k1 = stage_k[s1];
    const int ci1 = stage_chunk[s1] * kChunk;
    const int cw1 = min(kChunk, c_in - ci1);
    // Issue, in this order: row indices two stages ahead, the next B tile,
    // the next A operand.  The scheduling fences keep the order so the wait
    // before the barrier can leave the A loads in flight.
    int idx_next2[S::RB];
    load_rows<S::RB>(idx_next2, kv_map, rows, row0, stage_k[s2], lr);
    V breg[BSource::kDirect ? 1 : S::B_PIECES];
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (BSource::kDirect) {
        stage_b_direct<T, C_OUT, WAVE_ROWS>(bsrc, k1, ci1, cw1, bnext, wave, lane);
    } else {
        stage_b_load<T, C_OUT, WAVE_ROWS>(bsrc, k1, ci1, cw1, breg);
    }
    __builtin_amdgcn_sched_barrier(0);
    V a_next[S::RB][S::ST];
    load_a<T, V, S::RB, S::ST>(a_next, idx_next, feats, c_in, ci1, cw1, lk);
    __builtin_amdgcn_sched_barrier(0);

    if ((wmask >> k) & 1u) {
        const int nst = min(kChunk, c_in - chunk * kChunk) / 32;
        const uint32_t brow = lds_address(bcur + (wc * S::WAVE_COLS + lr) * S::BROW);
        const V zero = zero_vec<V>();
#pragma unroll
        for (int st = 0; st < S::ST; ++st) {
            if (st < nst) {
                // Rows wc*WAVE_COLS + 16*cb + lr all have lr as their low four
                // bits, so piece 4*st + lane/16 sits in the same slot for every
                // column block.
                const uint32_t addr = brow + swizzle_piece(st * 4 + (lane >> 4), lr) * 16;
                V b[S::CB];
                read_b_fragments<V, S::CB, 16 * S::BROW * 2>(b, addr);
                V a[S::RB];
#pragma unroll
                for (int rb = 0; rb < S::RB; ++rb) a[rb] = idx_cur[rb] >= 0 ? a_cur[rb][st] : zero;
#pragma unroll
                for (int cb = 0; cb < S::CB; ++cb) {
#pragma unroll
                    for (int rb = 0; rb < S::RB; ++rb) acc[rb][cb] = MfmaOps<T>::mfma(a[rb], b[cb], acc[rb][cb]);
                }
            }
        }
    }
    if constexpr (BSource::kDirect) {
        // The next B tile must have landed in LDS before any wave reads it;
        // the A loads issued after it may stay in flight.
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(S::RB * S::ST));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    } else {
        stage_b_store<T, C_OUT, WAVE_ROWS>(bnext, breg);
        __syncthreads();
    }
#pragma unroll
    for (int rb = 0; rb < S::RB; ++rb) {
        idx_cur[rb] = idx_next[rb];
        idx_next[rb] = idx_next2[rb];
#pragma unroll
        for (int st = 0; st < S::ST; ++st) a_cur[rb][st] = a_next[rb][st];
    }
}

template <typename T, int C_OUT, int WAVE_ROWS, typename BSource>
__global__ void __launch_bounds__(kBlock, 1)
conv_igemm(const T* __restrict__ feats, int c_in, BSource bsrc, const int32_t* __restrict__ kv_map,
           const int32_t* __restrict__ tile_masks, const int32_t* __restrict__ reorder_rows, int rows,
           T* __restrict__ out) {
    using S = IgemmShape<C_OUT, WAVE_ROWS>;
    using V = typename MfmaOps<T>::vec;
    __shared__ __align__(16) T bbuf0[S::BBUF];
    __shared__ __align__(16) T bbuf1[S::BBUF];
    __shared__ unsigned char stage_k[kMaxStages];
    __shared__ unsigned char stage_chunk[kMaxStages];

    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int wr = wave / S::CG;
    const int wc = wave % S::CG;
    const int block_row0 = blockIdx.x * S::BLOCK_ROWS;
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
    const int nchunks = (c_in + kChunk - 1) / kChunk;
    const int nstages = __popc(bmask) * nchunks;
    if (threadIdx.x == 0) {
        uint32_t m = bmask;
        int s = 0;
        while (m) {
            const int k = __builtin_ctz(m);
            m &= m - 1;
            for (int c = 0; c < nchunks; ++c, ++s) {
                stage_k[s] = static_cast<unsigned char>(k);
                stage_chunk[s] = static_cast<unsigned char>(c);
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

    if (nstages > 0) {
        // Prologue: B tile of stage 0 in LDS, A of stage 0 and row indices
        // of stage 1 in registers.
        const int k0 = stage_k[0];
        const int c0 = min(kChunk, c_in);
        if constexpr (BSource::kDirect) {
            stage_b_direct<T, C_OUT, WAVE_ROWS>(bsrc, k0, 0, c0, bbuf0, wave, lane);
        } else {
            V breg[S::B_PIECES];
            stage_b_load<T, C_OUT, WAVE_ROWS>(bsrc, k0, 0, c0, breg);
            stage_b_store<T, C_OUT, WAVE_ROWS>(bbuf0, breg);
        }
        int idx_cur[S::RB];
        load_rows<S::RB>(idx_cur, kv_map, rows, row0, k0, lr);
        V a_cur[S::RB][S::ST];
        load_a<T, V, S::RB, S::ST>(a_cur, idx_cur, feats, c_in, 0, c0, lk);
        int idx_next[S::RB];
        load_rows<S::RB>(idx_next, kv_map, rows, row0, stage_k[min(1, nstages - 1)], lr);
        __syncthreads();
        for (int s = 0; s < nstages; s += 2) {
            igemm_stage<T, C_OUT, WAVE_ROWS, BSource, V>(s, nstages, stage_k, stage_chunk, bbuf0, bbuf1, feats, c_in,
                                                          bsrc, kv_map, rows, row0, wave, wc, lane, wmask, idx_cur,
                                                          idx_next, a_cur, acc);
            if (s + 1 < nstages) {
                igemm_stage<T, C_OUT, WAVE_ROWS, BSource, V>(s + 1, nstages, stage_k, stage_chunk, bbuf1, bbuf0,
                                                              feats, c_in, bsrc, kv_map, rows, row0, wave, wc, lane,
                                                              wmask, idx_cur, idx_next, a_cur, acc);
            }
        }
    }
    __syncthreads();

    // Epilogue: stage this wave's tile in LDS (pieces swizzled by row), then
    // write whole rows with 16-byte stores to out[reorder_rows[row]].
    T* stage = (wave < 2 ? bbuf0 : bbuf1) + (wave & 1) * WAVE_ROWS * S::EROW;
#pragma unroll
    for (int rb = 0; rb < S::RB; ++rb) {
#pragma unroll
        for (int cb = 0; cb < S::CB; ++cb) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = rb * 16 + (lane >> 4) * 4 + q;
                const int piece = (cb * 16 + lr) / 8;
                const int slot = piece ^ (r % S::EPIECES);
                stage[r * S::EROW + slot * 8 + (lr & 7)] = static_cast<T>(acc[rb][cb][q]);
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
            *reinterpret_cast<V*>(out + orow * C_OUT + wc * S::WAVE_COLS + piece * 8) =
                *reinterpret_cast<const V*>(stage + r * S::EROW + (piece ^ (r % S::EPIECES)) * 8);
        }
    }
}

template <typename T, int C_OUT, int WAVE_ROWS, typename BSource>
int launch_igemm_shape(const T* feats, int c_in, const BSource& b, const int32_t* kv_map,
                       const int32_t* tile_masks, const int32_t* reorder_rows, int rows, T* out,
                       hipStream_t stream) {
    using S = IgemmShape<C_OUT, WAVE_ROWS>;
    const unsigned blocks = static_cast<unsigned>((rows + S::BLOCK_ROWS - 1) / S::BLOCK_ROWS);
    conv_igemm<T, C_OUT, WAVE_ROWS, BSource><<<blocks, kBlock, 0, stream>>>(feats, c_in, b, kv_map, tile_masks,
                                                                           reorder_rows, rows, out);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

// Wave tile rows: 64 doubles B reuse from LDS, 32 halves the registers
// (two waves per SIMD).  Chosen per launch; see igemm_wave_rows().
int g_igemm_wave_rows = 32;

template <typename T, typename BSource>
int launch_igemm(const T* feats, int c_in, int c_out, const BSource& b, const int32_t* kv_map,
                 const int32_t* tile_masks, const int32_t* reorder_rows, int rows, T* out, hipStream_t stream) {
    if (rows <= 0) return LATTICE_OK;
#define LATTICE_IGEMM_CASE(C)                                                                              \
    case C:                                                                                                \
        return g_igemm_wave_rows == 64                                                                     \
                   ? launch_igemm_shape<T, C, 64>(feats, c_in, b, kv_map, tile_masks, reorder_rows, rows, out, \
                                                  stream)                                                  \
                   : launch_igemm_shape<T, C, 32>(feats, c_in, b, kv_map, tile_masks, reorder_rows, rows, out, \
                                                  stream);
    switch (c_out) {
        LATTICE_IGEMM_CASE(16)
        LATTICE_IGEMM_CASE(32)
        LATTICE_IGEMM_CASE(64)
        LATTICE_IGEMM_CASE(128)
        LATTICE_IGEMM_CASE(256)
#undef LATTICE_IGEMM_CASE
    default:
        set_error("implicit GEMM supports c_out in {16, 32, 64, 128, 256}.");
        return LATTICE_ERROR_UNSUPPORTED;
    }
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

extern "C" int lattice_hip_set_conv_tile_rows(int rows) {
    LATTICE_REQUIRE(rows == 32 || rows == 64, "conv tile rows must be 32 or 64.");
    g_igemm_wave_rows = rows;
    return LATTICE_OK;
}

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
    int c_out, const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks, const int32_t* reorder_rows,
    int out_capacity, void* out, void* stream_ptr) {
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
    LATTICE_REQUIRE(sorted_kv_out_in_map && tile_masks && out && weights && (feats || n_in == 0),
                    "conv pointers must be non-null.");
    hipStream_t stream = as_stream(stream_ptr);
    const long long s_co = static_cast<long long>(kernel_count) * c_in;
    const long long s_k = c_in;
    if (dtype == LATTICE_F16) {
        FloatB<_Float16> b{static_cast<const _Float16*>(weights), s_co, s_k};
        return launch_igemm<_Float16>(static_cast<const _Float16*>(feats), c_in, c_out, b, sorted_kv_out_in_map,
                                      tile_masks, reorder_rows, out_capacity, static_cast<_Float16*>(out), stream);
    }
    FloatB<__bf16> b{static_cast<const __bf16*>(weights), s_co, s_k};
    return launch_igemm<__bf16>(static_cast<const __bf16*>(feats), c_in, c_out, b, sorted_kv_out_in_map,
                                tile_masks, reorder_rows, out_capacity, static_cast<__bf16*>(out), stream);
}

extern "C" int lattice_hip_sparse_quantized_conv_features(
    int dtype, const void* feats, int n_in, int c_in, const uint32_t* weights, const void* scales,
    const void* biases, int kernel_count, int c_out, int storage_c_in, int group_size, int bits,
    const int32_t* in_rows, const int32_t* kernel_ids, const int32_t* counts, int edge_capacity,
    const int32_t* row_offsets, const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks,
    const int32_t* reorder_rows, int out_capacity, void* out, void* stream_ptr) {
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
    if (sorted && dtype != LATTICE_F32 && igemm_shape_ok(c_in, c_out, kernel_count)) {
        if (dtype == LATTICE_F16) {
            PackedB<_Float16> b{weights, static_cast<const _Float16*>(scales), static_cast<const _Float16*>(biases),
                                packed_words, groups, group_size, c_out, bits};
            return launch_igemm<_Float16>(static_cast<const _Float16*>(feats), c_in, c_out, b, sorted_kv_out_in_map,
                                          tile_masks, reorder_rows, out_capacity, static_cast<_Float16*>(out),
                                          stream);
        }
        PackedB<__bf16> b{weights, static_cast<const __bf16*>(scales), static_cast<const __bf16*>(biases),
                          packed_words, groups, group_size, c_out, bits};
        return launch_igemm<__bf16>(static_cast<const __bf16*>(feats), c_in, c_out, b, sorted_kv_out_in_map,
                                    tile_masks, reorder_rows, out_capacity, static_cast<__bf16*>(out), stream);
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
