// Gradients of the sparse convolution (the reference's vjp:
// native/features/convolution/primitive.cpp:137-176, 597-680; CPU routines
// cpu/algorithms.cpp:355-481).
//
//  * Input gradient, CSR route: one lane per (input row, input channel)
//    walks the row's edges in the input-grouped CSR (in_row_offsets /
//    in_edge_ids) with an fp32 accumulator over the edges and every output
//    channel, one rounding at the end (eval_input_grad_typed).  Small
//    weights are staged once per block in LDS as fp32, (k, co, ci) with ci
//    fastest, so the lanes of a row read consecutive banks.
//  * Input gradient, matrix-core route: for a forward or submanifold
//    relation every (input row, k) pair has at most one output row, so the
//    relation transposes into a dense map in_out_map[in][k] with the same
//    row masks as the forward's out_in_map.  `transposed_map` scatters it
//    from the edges; the forward's sorted view and implicit-GEMM kernel then
//    compute grad[in][ci] = sum_k sum_co cot[map[in][k]][co] * W[k][ci][co]
//    with the weight transposed to (C_in, K, C_out).
//  * Weight gradient: dW[k] = sum over the edges of k of
//    feats[in]^T cot[out] (eval_weight_grad_typed), a contraction over
//    edges.  The matrix-core kernel splits each offset's kernel-grouped
//    edges (kernel_row_offsets / kernel_edge_ids, in output-row order) into
//    eight parts, one per XCD, and deals an XCD's blocks to the offsets in
//    proportion to their edge counts; an offset's blocks take its part's
//    64-edge chunks in turn, so the XCD's blocks sweep the same output rows
//    together and a cotangent row stays in L2 between the offsets that read
//    it.  Channel tiles are 128 x 128 when the channels fill them (an
//    edge's rows are gathered once for every channel pair).  A block stages
//    64 edges of both operands in LDS as edge rows, reads the MFMA
//    fragments (8 consecutive edges per lane) with transposing LDS reads
//    and accumulates in fp32.  Each block writes its partial tile; a second
//    kernel sums an offset's partials in a fixed order and rounds once, so
//    results are deterministic.  Other dtypes and shapes take a
//    one-lane-per-weight kernel.

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <type_traits>

#include "lattice_common.h"
#include "scan.h"

namespace lattice {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

template <typename T> __device__ inline float to_f(T v) { return static_cast<float>(v); }

struct GradWeightIndex {
    int layout;  // LATTICE_WEIGHT_*
    int K, c_in, c_out;
    __device__ inline long long operator()(int k, int ci, int co) const {
        if (layout == LATTICE_WEIGHT_KERNEL_MAJOR) return (static_cast<long long>(k) * c_in + ci) * c_out + co;
        return (static_cast<long long>(co) * K + k) * c_in + ci;
    }
};

constexpr int kGradLdsFloats = 16384;
constexpr unsigned kGradStagedBlocks = 2048;

// ------------------------------------------------- input gradient (CSR) --

template <typename T>
__global__ void __launch_bounds__(256)
input_grad_csr(const T* __restrict__ cot, int out_capacity, const T* __restrict__ weights, GradWeightIndex widx,
               const int32_t* __restrict__ out_rows, const int32_t* __restrict__ kernel_ids,
               const int32_t* __restrict__ counts, int edge_capacity, const int32_t* __restrict__ in_row_offsets,
               const int32_t* __restrict__ in_edge_ids, int in_capacity, T* __restrict__ grad, bool staged) {
    extern __shared__ float wlds[];
    const int c_in = widx.c_in;
    const int c_out = widx.c_out;
    if (staged) {
        const int nw = widx.K * c_in * c_out;
        for (int i = threadIdx.x; i < nw; i += blockDim.x) {
            const int ci = i % c_in;
            const int kc = i / c_in;  // k * c_out + co
            wlds[i] = to_f(weights[widx(kc / c_out, ci, kc % c_out)]);
        }
        __syncthreads();
    }
    const int E = min(counts[0], edge_capacity);
    const long long total = static_cast<long long>(in_capacity) * c_in;
    for (long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(t / c_in);
        const int ci = static_cast<int>(t - static_cast<long long>(row) * c_in);
        float acc = 0.0f;
        const int end = in_row_offsets[row + 1];
        for (int cur = in_row_offsets[row]; cur < end; ++cur) {
            const int e = in_edge_ids[cur];
            if (e < 0 || e >= E) continue;
            const int o = out_rows[e];
            const int k = kernel_ids[e];
            if (o < 0 || o >= out_capacity || k < 0 || k >= widx.K) continue;
            const T* g = cot + static_cast<long long>(o) * c_out;
            if (staged) {
                const float* wk = wlds + static_cast<long long>(k) * c_out * c_in + ci;
                for (int co = 0; co < c_out; ++co) acc += to_f(g[co]) * wk[co * c_in];
            } else {
                for (int co = 0; co < c_out; ++co) acc += to_f(g[co]) * to_f(weights[widx(k, ci, co)]);
            }
        }
        grad[t] = static_cast<T>(acc);
    }
}

// ---------------------------------------- transposed map (matrix cores) --

__global__ void __launch_bounds__(256)
transposed_map(const int32_t* __restrict__ in_rows, const int32_t* __restrict__ out_rows,
               const int32_t* __restrict__ kernel_ids, const int32_t* __restrict__ counts, int edge_capacity,
               int in_capacity, int K, int32_t* __restrict__ in_out_map, int32_t* __restrict__ status) {
    const int E = min(counts[0], edge_capacity);
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < E; e += gridDim.x * blockDim.x) {
        const int in = in_rows[e];
        const int o = out_rows[e];
        const int k = kernel_ids[e];
        if (in < 0 || in >= in_capacity || o < 0 || k < 0 || k >= K) continue;
        const int prev = atomicCAS(&in_out_map[static_cast<long long>(in) * K + k], -1, o);
        if (prev != -1 && status != nullptr) atomicOr(status, LATTICE_STATUS_REPEATED_PAIR);
    }
}

// Offset bits of each input row, from its row of the transposed map.  A
// block takes `rows_per_block` consecutive rows, copies their contiguous
// map rows into LDS with coalesced loads, and one lane per row then reads
// its row from LDS (a lane-per-row read of global memory would touch a
// different line per lane for each offset).
__global__ void __launch_bounds__(256)
transposed_masks(const int32_t* __restrict__ in_out_map, int in_capacity, int K, int words, int rows_per_block,
                 int32_t* __restrict__ row_masks) {
    extern __shared__ int32_t map_rows[];
    const int blocks = (in_capacity + rows_per_block - 1) / rows_per_block;
    for (int blk = blockIdx.x; blk < blocks; blk += gridDim.x) {
        const int r0 = blk * rows_per_block;
        const int n = min(rows_per_block, in_capacity - r0);
        const int32_t* src = in_out_map + static_cast<long long>(r0) * K;
        for (int i = threadIdx.x; i < n * K; i += blockDim.x) map_rows[i] = src[i];
        __syncthreads();
        for (int r = threadIdx.x; r < n; r += blockDim.x) {
            const int32_t* m = map_rows + r * K;
            for (int w = 0; w < words; ++w) {
                uint32_t bits = 0;
                for (int k = 32 * w; k < min(K, 32 * w + 32); ++k) bits |= (m[k] >= 0 ? 1u : 0u) << (k & 31);
                row_masks[static_cast<long long>(r0 + r) * words + w] = static_cast<int32_t>(bits);
            }
        }
        __syncthreads();
    }
}

// --------------------------------------- weight gradient (matrix cores) --

template <typename T> struct GradMfma;
template <> struct GradMfma<_Float16> {
    typedef half8_t vec;
    __device__ static float4_t mfma(vec a, vec b, float4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
template <> struct GradMfma<__bf16> {
    typedef bf16x8_t vec;
    __device__ static float4_t mfma(vec a, vec b, float4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

constexpr int kWgEdges = 64;   // edges per staged step (two 32-edge MFMA steps)

// LDS rows of a weight-gradient step: one row per edge, the operand's
// channels in 16-byte pieces (TC / 8 of them).  Piece q of row r sits at
// slot q ^ wg_swizzle(r): the waves' 16-byte stores (two rows of 8 pieces
// per 16 lanes) and the transposing fragment reads (16 rows x 2 pieces per
// instruction) then spread over all the banks.
__device__ inline int wg_swizzle(int r, int pieces) {
    return (2 * (r & 1) + 4 * ((r >> 1) & 1) + 8 * (((r >> 3) ^ r) & 1)) & (pieces - 1);
}

template <int TC>
__device__ inline int wg_piece_slot(int r, int q) { return r * TC + ((q ^ wg_swizzle(r, TC / 8)) << 3); }

typedef short short4_t __attribute__((ext_vector_type(4)));

// One MFMA operand fragment (16 channels x 32 edges) from edge-major LDS
// rows with two transposing reads.  In each 16-lane group, ds_read_b64_tr_b16
// gives lane i element i % 4 of the 8-byte chunks addressed by lanes
// i / 4 + 4j (j = 0..3).  Lane s of group g addresses row
// 32 ks + 8 g + 4 t + s / 4 at channel c0 + 4 (s % 4), so lane i receives
// channel c0 + i of four consecutive edges; the two reads (t = 0, 1) make
// the 8 edges 8 g .. 8 g + 7 the MFMA expects of lane i.
template <typename V, int TC, typename T>
__device__ inline V wg_fragment(const T* lds, int ks, int c0, int lane) {
    const int s = lane & 15;
    const int g = lane >> 4;
    const int q = (c0 >> 3) + ((s & 3) >> 1);
    short4_t h[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int r = 32 * ks + 8 * g + 4 * t + (s >> 2);
        const T* src = lds + wg_piece_slot<TC>(r, q) + 4 * (s & 1);
        h[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) short4_t*)(src));
    }
    typedef short short8_t __attribute__((ext_vector_type(8)));
    const short8_t both = __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(V, both);
}

// Lock-step plan of the weight gradient.  The kernel-grouped edges of each
// offset are in output-row order, so part x (of kXcds equal parts) of every
// offset's edges covers about the same output rows.  The blocks of XCD x
// (launch index = x mod kXcds) all work on part x: S slots per XCD dealt
// to the offsets in proportion to their edge counts (at least one each),
// and the m_k blocks of offset k take its part's 64-edge chunks in turn
// (block j: chunks j, j + m_k, ...).  Every block then sums about the same
// number of edges, and all blocks of an XCD move through their part's
// output rows together, so the cotangent row of an output row, read once
// per offset, stays in that XCD's L2 between the offsets that read it.
constexpr int kXcds = 8;

// Blocks offset k gets on each XCD; first = blocks of the offsets before k.
__device__ inline void wg_share(const int32_t* koff, int K, int slots, int k, int* first, int* count) {
    const long long total = koff[K] - koff[0];
    int nz = 0;
    for (int i = 0; i < K; ++i) nz += koff[i + 1] > koff[i] ? 1 : 0;
    const long long spare = slots - nz;
    int acc = 0;
    *first = 0;
    *count = 0;
    for (int i = 0; i <= k; ++i) {
        const long long n = koff[i + 1] - koff[i];
        const int m = n > 0 ? 1 + static_cast<int>(spare * n / total) : 0;
        if (i == k) {
            *first = acc;
            *count = m;
        }
        acc += m;
    }
}

// Block (launch index): XCD x = index mod 8, then (tile, slot) from
// index / 8; channel tile TCI x TCO, four waves of (TCI/2) x (TCO/2).  Per
// step of 64 edges the block stages both operands into edge-major LDS rows.
template <typename T, int TCI, int TCO>
__global__ void __launch_bounds__(256, 3)
weight_grad_mfma(const T* __restrict__ feats, int n_in, int c_in, const T* __restrict__ cot, int n_out, int c_out,
                 const int32_t* __restrict__ in_rows, const int32_t* __restrict__ out_rows,
                 const int32_t* __restrict__ counts, int edge_capacity, const int32_t* __restrict__ koff,
                 const int32_t* __restrict__ kedges, int K, int tiles, int tiles_co, int slots,
                 float* __restrict__ partial) {
    using V = typename GradMfma<T>::vec;
    constexpr int MB = TCI / 32;  // 16-row blocks per wave
    constexpr int NB = TCO / 32;  // 16-column blocks per wave
    __shared__ __align__(16) T a_t[kWgEdges * TCI];
    __shared__ __align__(16) T b_t[kWgEdges * TCO];
    const int x = static_cast<int>(blockIdx.x) % kXcds;
    const int q = static_cast<int>(blockIdx.x) / kXcds;
    const int tile = q % tiles;
    const int slot = q / tiles;
    // The offset and the turn of this slot.
    int k = -1, turn = 0, turns = 0;
    {
        const long long total = koff[K] - koff[0];
        if (total <= 0) return;
        int nz = 0;
        for (int i = 0; i < K; ++i) nz += koff[i + 1] > koff[i] ? 1 : 0;
        const long long spare = slots - nz;
        int acc = 0;
        for (int i = 0; i < K; ++i) {
            const long long n = koff[i + 1] - koff[i];
            const int m = n > 0 ? 1 + static_cast<int>(spare * n / total) : 0;
            if (slot < acc + m) {
                k = i;
                turn = slot - acc;
                turns = m;
                break;
            }
            acc += m;
        }
    }
    if (k < 0) return;  // a spare slot: no partial tile is read for it
    const int ci0 = (tile / tiles_co) * TCI;
    const int co0 = (tile % tiles_co) * TCO;
    const int E = min(counts[0], edge_capacity);
    const int lo_k = koff[k];
    const long long n_k = koff[k + 1] - lo_k;
    const int lo = lo_k + static_cast<int>(n_k * x / kXcds);
    const int hi = lo_k + static_cast<int>(n_k * (x + 1) / kXcds);
    const int stride = turns * kWgEdges;  // the block's chunks: lo + 64 (turn + t turns)
    const int start = lo + turn * kWgEdges;

    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int wm = wave & 1;
    const int wn = wave >> 1;
    const int lr = lane & 15;
    const int g = lane >> 4;
    float4_t acc[MB][NB];
#pragma unroll
    for (int a = 0; a < MB; ++a)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[a][n] = float4_t{0.f, 0.f, 0.f, 0.f};

    // Thread t stages edges t/8 and t/8 + 32 of the step: 8-channel pieces
    // t%8 + 8i of their feature rows (i < TCI/64) and cotangent rows
    // (i < TCO/64), so a wave's loads cover eight whole 128-byte row lines.
    constexpr int PA = TCI / 64;
    constexpr int PB = TCO / 64;
    const int j = threadIdx.x >> 3;
    const int p = threadIdx.x & 7;
    V av[2][PA], bv[2][PB];
    bool aok[2][PA], bok[2][PB];
    // Three-stage pipeline over the steps: the edge ids of step s+3 and the
    // row indices of step s+2 are loaded while the rows of step s+1 are
    // gathered, so no step waits on a dependent index load.  Edges past the
    // share's end or outside the relation count as zeros.  Every load is
    // issued unconditionally (clamped address, validity kept aside) and the
    // index loads go out before the gathers: gfx950's vector-memory counter
    // retires in issue order, so a wait for an index issued after the
    // gathers would also wait for the gathers.
    const int last_edge = max(hi - 1, 0);
    auto issue_edges = [&](int base, int (&evr)[2], bool (&evv)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int cur = base + j + 32 * h;
            evv[h] = cur < hi;
            evr[h] = kedges[min(cur, last_edge)];
        }
    };
    auto edges_of = [&](const int (&evr)[2], const bool (&evv)[2], int (&ev)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) ev[h] = evv[h] ? evr[h] : -1;
    };
    auto issue_rows = [&](const int (&ev)[2], int (&rin)[2], int (&rout)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int e = ev[h] >= 0 && ev[h] < E ? ev[h] : 0;
            rin[h] = in_rows[e];
            rout[h] = out_rows[e];
        }
    };
    auto rows_of = [&](const int (&ev)[2], const int (&rin)[2], const int (&rout)[2], int (&ri)[2], int (&ro)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool ok = ev[h] >= 0 && ev[h] < E && rin[h] >= 0 && rin[h] < n_in && rout[h] >= 0 &&
                            rout[h] < n_out;
            ri[h] = ok ? rin[h] : -1;
            ro[h] = ok ? rout[h] : -1;
        }
    };
    auto gather = [&](const int (&ri)[2], const int (&ro)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const long long rin = ri[h] >= 0 ? ri[h] : 0, rout = ro[h] >= 0 ? ro[h] : 0;
#pragma unroll
            for (int i = 0; i < PA; ++i) {
                const int c = ci0 + 8 * (p + 8 * i);
                aok[h][i] = ri[h] >= 0 && c < c_in;
                av[h][i] = *reinterpret_cast<const V*>(feats + rin * c_in + (c < c_in ? c : 0));
            }
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                const int c = co0 + 8 * (p + 8 * i);
                bok[h][i] = ro[h] >= 0 && c < c_out;
                bv[h][i] = *reinterpret_cast<const V*>(cot + rout * c_out + (c < c_out ? c : 0));
            }
        }
    };
    int ev[2], evr[2], ri[2], ro[2], rin[2], rout[2];
    bool evv[2];
    issue_edges(start, evr, evv);
    edges_of(evr, evv, ev);
    issue_rows(ev, rin, rout);
    rows_of(ev, rin, rout, ri, ro);
    gather(ri, ro);
    issue_edges(start + stride, evr, evv);
    edges_of(evr, evv, ev);
    issue_rows(ev, rin, rout);
    rows_of(ev, rin, rout, ri, ro);
    issue_edges(start + 2 * stride, evr, evv);
    edges_of(evr, evv, ev);
    for (int base = start; base < hi; base += stride) {
        // The thread's two edges take rows j and j + 32 (the order of edges
        // inside a step is free: the sum over them is in fp32).
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < PA; ++i)
                *reinterpret_cast<V*>(a_t + wg_piece_slot<TCI>(j + 32 * h, p + 8 * i)) = aok[h][i] ? av[h][i] : V{};
#pragma unroll
            for (int i = 0; i < PB; ++i)
                *reinterpret_cast<V*>(b_t + wg_piece_slot<TCO>(j + 32 * h, p + 8 * i)) = bok[h][i] ? bv[h][i] : V{};
        }
        __syncthreads();
        issue_rows(ev, rin, rout);                   // row indices of step s+2
        int ev_next[2];
        {
            int evr_n[2];
            bool evv_n[2];
            issue_edges(base + 3 * stride, evr_n, evv_n);  // edge ids of step s+3
            // Keep the index loads ahead of the gathers in issue order.
            __builtin_amdgcn_sched_barrier(0);
            gather(ri, ro);  // rows of step s+1
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                V af[MB], bf[NB];
#pragma unroll
                for (int m = 0; m < MB; ++m)
                    af[m] = wg_fragment<V, TCI>(a_t, ks, (TCI / 2) * wm + 16 * m, lane);
#pragma unroll
                for (int n = 0; n < NB; ++n)
                    bf[n] = wg_fragment<V, TCO>(b_t, ks, (TCO / 2) * wn + 16 * n, lane);
#pragma unroll
                for (int m = 0; m < MB; ++m)
#pragma unroll
                    for (int n = 0; n < NB; ++n) acc[m][n] = GradMfma<T>::mfma(af[m], bf[n], acc[m][n]);
            }
            edges_of(evr_n, evv_n, ev_next);
        }
        rows_of(ev, rin, rout, ri, ro);
        ev[0] = ev_next[0];
        ev[1] = ev_next[1];
        __syncthreads();
    }
    // D[m][n]: lane holds rows 4*(lane/16) + q, column lane%16 of each block.
    // The partial tile is stored as the lanes hold it (fragment order, one
    // 16-byte store per lane and block: whole 1 KB runs per wave); the
    // reduction maps each 4-float piece back to its (ci, co).
    float4_t* out = reinterpret_cast<float4_t*>(partial) +
                    (static_cast<long long>(x * slots + slot) * tiles + tile) * (TCI * TCO / 4);
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int n = 0; n < NB; ++n) out[((wave * MB + m) * NB + n) * 64 + lane] = acc[m][n];
}

// dW[k] = sum of the partial tiles of offset k's blocks (XCD by XCD, then
// turn by turn), one rounding, written in the weight's layout.  Blocks
// (x, k): offset k's share is worked out once per thread, then the block
// strides over the offset's C_in x C_out entries four at a time (16-byte
// loads of the partials; each entry keeps its own summation order).
constexpr int kReduceBatch = 16;  // partial loads in flight per thread

// dW[k] = sum of the partial tiles of offset k's blocks (XCD by XCD, then
// turn by turn), one rounding, written in the weight's layout.  Blocks
// (x, k): offset k's share is worked out once per thread, then the block
// strides over the partial matrix's 4-float pieces (fragment order of
// weight_grad_mfma: piece (tile, wave, m, n, lane) holds ci = ci0 +
// (TCI/2)*(wave&1) + 16m + 4(lane/16) + q, q < 4, and co = co0 +
// (TCO/2)*(wave>>1) + 16n + lane%16); each entry keeps its own summation
// order.
template <typename T>
__global__ void __launch_bounds__(256)
weight_grad_reduce(const float* __restrict__ partial, const int32_t* __restrict__ koff, int slots,
                   GradWeightIndex widx, int tci, int tco, int tiles, int tiles_co, T* __restrict__ grad) {
    const long long pieces = static_cast<long long>(tiles) * tci * tco / 4;  // per partial matrix
    const int mb = tci / 32, nb = tco / 32;
    const int k = blockIdx.y;
    int first = 0, count = 0;
    if (koff[widx.K] > koff[0]) wg_share(koff, widx.K, slots, k, &first, &count);
    const float4* p4 = reinterpret_cast<const float4*>(partial);
    for (long long w4 = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; w4 < pieces;
         w4 += static_cast<long long>(gridDim.x) * blockDim.x) {
        // partial i of the (x, j) order: x = i / count, j = i % count;
        // kReduceBatch loads are issued before their adds, which run in that
        // order
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const int n = kXcds * count;
        for (int i0 = 0; i0 < n; i0 += kReduceBatch) {
            float4 v[kReduceBatch];
#pragma unroll
            for (int u = 0; u < kReduceBatch; ++u) {
                const int i = i0 + u;
                const int x = count > 0 ? i / count : 0;
                const int j = i - x * count;
                v[u] = i < n ? p4[(x * slots + first + j) * pieces + w4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < kReduceBatch; ++u) {
                if (i0 + u < n) {
                    acc.x += v[u].x;
                    acc.y += v[u].y;
                    acc.z += v[u].z;
                    acc.w += v[u].w;
                }
            }
        }
        const long long per_tile = static_cast<long long>(tci) * tco / 4;
        const int tile = static_cast<int>(w4 / per_tile);
        long long r = w4 - tile * per_tile;
        const int lane = static_cast<int>(r % 64);
        r /= 64;
        const int nn = static_cast<int>(r % nb);
        r /= nb;
        const int mm = static_cast<int>(r % mb);
        const int wave = static_cast<int>(r / mb);
        const int ci = (tile / tiles_co) * tci + (tci / 2) * (wave & 1) + 16 * mm + 4 * (lane >> 4);
        const int co = (tile % tiles_co) * tco + (tco / 2) * (wave >> 1) + 16 * nn + (lane & 15);
        const float a[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (ci + q < widx.c_in && co < widx.c_out) grad[widx(k, ci + q, co)] = static_cast<T>(a[q]);
        }
    }
}

// One lane per weight entry (k, ci, co), co fastest: the kernel-grouped
// edges of k in order with an fp32 accumulator (eval_weight_grad_typed's
// loop).  Used for fp32 and for channel counts the matrix-core kernel does
// not take.
template <typename T>
__global__ void __launch_bounds__(256)
weight_grad_simple(const T* __restrict__ feats, int n_in, const T* __restrict__ cot, int n_out,
                   const int32_t* __restrict__ in_rows, const int32_t* __restrict__ out_rows,
                   const int32_t* __restrict__ counts, int edge_capacity, const int32_t* __restrict__ koff,
                   const int32_t* __restrict__ kedges, GradWeightIndex widx, T* __restrict__ grad) {
    const int c_in = widx.c_in;
    const int c_out = widx.c_out;
    const int E = min(counts[0], edge_capacity);
    const long long total = static_cast<long long>(widx.K) * c_in * c_out;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        const int co = static_cast<int>(i % c_out);
        const int ci = static_cast<int>((i / c_out) % c_in);
        const int k = static_cast<int>(i / (static_cast<long long>(c_in) * c_out));
        float acc = 0.0f;
        for (int cur = koff[k]; cur < koff[k + 1]; ++cur) {
            const int e = kedges[cur];
            if (e < 0 || e >= E) continue;
            const int in = in_rows[e];
            const int o = out_rows[e];
            if (in < 0 || in >= n_in || o < 0 || o >= n_out) continue;
            acc += to_f(feats[static_cast<long long>(in) * c_in + ci]) * to_f(cot[static_cast<long long>(o) * c_out + co]);
        }
        grad[widx(k, ci, co)] = static_cast<T>(acc);
    }
}

int check_grad_dtype(int dtype) {
    LATTICE_REQUIRE(dtype == LATTICE_F32 || dtype == LATTICE_F16 || dtype == LATTICE_BF16,
                    "convolution gradients support float32, float16 and bfloat16.");
    return LATTICE_OK;
}

// Slots per XCD (blocks per channel tile = 8 x slots) of the matrix-core
// weight gradient: about 2,048 edge slots of the relation's capacity per
// block, at least one per offset, at most 96 (three blocks on each of an
// XCD's 32 CUs: one round, so the blocks of an XCD move together).
constexpr int kWgEdgesPerBlock = 2048;
constexpr int kWgMaxSlots = 96;
int weight_grad_slots(int edge_capacity, int kernel_count) {
    const long long want =
        (static_cast<long long>(edge_capacity) + kXcds * kWgEdgesPerBlock - 1) / (kXcds * kWgEdgesPerBlock);
    return static_cast<int>(std::max<long long>(kernel_count, std::min<long long>(kWgMaxSlots, want)));
}

// Channel tiles of the matrix-core weight gradient: 128-channel tiles where
// the channels fill them, so one gather of an edge's rows serves every
// channel pair of the tile.
struct WgTiles {
    int tci, tco, tiles_ci, tiles_co;
    int tiles() const { return tiles_ci * tiles_co; }
};
WgTiles wg_tiles(int c_in, int c_out) {
    WgTiles t;
    t.tci = c_in > 64 ? 128 : 64;
    t.tco = c_out > 64 ? 128 : 64;
    t.tiles_ci = (c_in + t.tci - 1) / t.tci;
    t.tiles_co = (c_out + t.tco - 1) / t.tco;
    return t;
}

// One fp32 partial matrix (every channel tile, in fragment order) per block
// slot.
size_t weight_grad_partial_bytes(int edge_capacity, int kernel_count, int c_in, int c_out) {
    const WgTiles t = wg_tiles(c_in, c_out);
    return static_cast<size_t>(kXcds) * weight_grad_slots(edge_capacity, kernel_count) * t.tiles() * t.tci * t.tco *
           sizeof(float);
}

bool weight_grad_mfma_ok(int dtype, int c_in, int c_out) {
    return (dtype == LATTICE_F16 || dtype == LATTICE_BF16) && c_in % 8 == 0 && c_out % 8 == 0;
}

template <typename T>
void launch_input_grad(const void* cot, int out_capacity, const void* weights, GradWeightIndex widx,
                       const int32_t* out_rows, const int32_t* kernel_ids, const int32_t* counts, int edge_capacity,
                       const int32_t* in_row_offsets, const int32_t* in_edge_ids, int in_capacity, void* grad,
                       hipStream_t stream) {
    const long long nw = static_cast<long long>(widx.K) * widx.c_in * widx.c_out;
    const bool staged = nw <= kGradLdsFloats;
    const unsigned grid = grid_for(static_cast<long long>(in_capacity) * widx.c_in, 256,
                                   staged ? kGradStagedBlocks : 1u << 16);
    input_grad_csr<T><<<grid, 256, staged ? nw * sizeof(float) : 0, stream>>>(
        static_cast<const T*>(cot), out_capacity, static_cast<const T*>(weights), widx, out_rows, kernel_ids, counts,
        edge_capacity, in_row_offsets, in_edge_ids, in_capacity, static_cast<T*>(grad), staged);
}

template <typename T>
int launch_weight_grad(int dtype, const void* feats, int n_in, const void* cot, int n_out, GradWeightIndex widx,
                       const int32_t* in_rows, const int32_t* out_rows, const int32_t* counts, int edge_capacity,
                       const int32_t* koff, const int32_t* kedges, void* grad, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
    if (weight_grad_mfma_ok(dtype, widx.c_in, widx.c_out) && workspace != nullptr) {
        if constexpr (!std::is_same<T, float>::value) {
            const int slots = weight_grad_slots(edge_capacity, widx.K);
            const size_t need = weight_grad_partial_bytes(edge_capacity, widx.K, widx.c_in, widx.c_out);
            LATTICE_REQUIRE(workspace_bytes >= need, "weight gradient workspace too small.");
            float* partial = static_cast<float*>(workspace);
            const WgTiles wt = wg_tiles(widx.c_in, widx.c_out);
            const int tci = wt.tci, tco = wt.tco, tiles_co = wt.tiles_co, tiles = wt.tiles();
            const unsigned grid = static_cast<unsigned>(kXcds) * slots * tiles;
#define LATTICE_WG_LAUNCH(A, B)                                                                                 \
    weight_grad_mfma<T, A, B><<<grid, 256, 0, stream>>>(static_cast<const T*>(feats), n_in, widx.c_in,          \
                                                        static_cast<const T*>(cot), n_out, widx.c_out, in_rows,  \
                                                        out_rows, counts, edge_capacity, koff, kedges, widx.K,   \
                                                        tiles, tiles_co, slots, partial)
            if (tci == 128 && tco == 128) LATTICE_WG_LAUNCH(128, 128);
            else if (tci == 128) LATTICE_WG_LAUNCH(128, 64);
            else if (tco == 128) LATTICE_WG_LAUNCH(64, 128);
            else LATTICE_WG_LAUNCH(64, 64);
#undef LATTICE_WG_LAUNCH
            LATTICE_LAUNCH_CHECK();
            const long long pieces = static_cast<long long>(tiles) * tci * tco / 4;
            const dim3 rgrid(grid_for(pieces, 256, 256), static_cast<unsigned>(widx.K));
            weight_grad_reduce<T><<<rgrid, 256, 0, stream>>>(partial, koff, slots, widx, tci, tco, tiles, tiles_co,
                                                             static_cast<T*>(grad));
            LATTICE_LAUNCH_CHECK();
            return LATTICE_OK;
        }
    }
    const long long total = static_cast<long long>(widx.K) * widx.c_in * widx.c_out;
    weight_grad_simple<T><<<grid_for(total, 256, 1u << 16), 256, 0, stream>>>(
        static_cast<const T*>(feats), n_in, static_cast<const T*>(cot), n_out, in_rows, out_rows, counts,
        edge_capacity, koff, kedges, widx, static_cast<T*>(grad));
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

}  // namespace
}  // namespace lattice

using namespace lattice;

extern "C" int lattice_hip_sparse_conv_input_grad(int dtype, const void* cot, int out_capacity, int c_out,
                                                  const void* weights, int weight_layout, int kernel_count, int c_in,
                                                  const int32_t* out_rows, const int32_t* kernel_ids,
                                                  const int32_t* counts, int edge_capacity,
                                                  const int32_t* in_row_offsets, const int32_t* in_edge_ids,
                                                  int in_capacity, void* grad, void* stream_ptr) {
    int rc = check_grad_dtype(dtype);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(out_capacity >= 0 && in_capacity >= 0 && c_in > 0 && c_out > 0 && kernel_count > 0,
                    "gradient shapes must be positive.");
    LATTICE_REQUIRE(weight_layout == LATTICE_WEIGHT_KERNEL_MAJOR || weight_layout == LATTICE_WEIGHT_DENSE_5D,
                    "weights must have shape (K, C_in, C_out) or (C_out, Kx, Ky, Kz, C_in).");
    if (in_capacity == 0) return LATTICE_OK;
    LATTICE_REQUIRE(weights && out_rows && kernel_ids && counts && in_row_offsets && in_edge_ids && grad &&
                        (cot || out_capacity == 0),
                    "gradient pointers must be non-null.");
    hipStream_t stream = as_stream(stream_ptr);
    GradWeightIndex widx{weight_layout, kernel_count, c_in, c_out};
    if (dtype == LATTICE_F32) {
        launch_input_grad<float>(cot, out_capacity, weights, widx, out_rows, kernel_ids, counts, edge_capacity,
                                 in_row_offsets, in_edge_ids, in_capacity, grad, stream);
    } else if (dtype == LATTICE_F16) {
        launch_input_grad<_Float16>(cot, out_capacity, weights, widx, out_rows, kernel_ids, counts, edge_capacity,
                                    in_row_offsets, in_edge_ids, in_capacity, grad, stream);
    } else {
        launch_input_grad<__bf16>(cot, out_capacity, weights, widx, out_rows, kernel_ids, counts, edge_capacity,
                                  in_row_offsets, in_edge_ids, in_capacity, grad, stream);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_build_transposed_implicit_gemm_map(const int32_t* in_rows, const int32_t* out_rows,
                                                             const int32_t* kernel_ids, const int32_t* counts,
                                                             int edge_capacity, int in_capacity, int kernel_count,
                                                             int32_t* in_out_map, int32_t* row_masks,
                                                             int32_t* status, void* stream_ptr) {
    LATTICE_REQUIRE(edge_capacity >= 0 && in_capacity >= 0 && kernel_count > 0,
                    "transposed map shapes must be nonnegative with a positive kernel count.");
    if (status != nullptr) {
        const int rc = fill_i32(status, 1, 0, as_stream(stream_ptr));
        if (rc != LATTICE_OK) return rc;
    }
    if (in_capacity == 0) return LATTICE_OK;
    LATTICE_REQUIRE(in_out_map && row_masks && counts && (edge_capacity == 0 || (in_rows && out_rows && kernel_ids)),
                    "transposed map pointers must be non-null.");
    hipStream_t stream = as_stream(stream_ptr);
    const int words = (kernel_count + 31) / 32;
    int rc = fill_i32(in_out_map, static_cast<long long>(in_capacity) * kernel_count, -1, stream);
    if (rc != LATTICE_OK) return rc;
    if (edge_capacity > 0) {
        transposed_map<<<grid_for(edge_capacity, 256, 1u << 16), 256, 0, stream>>>(
            in_rows, out_rows, kernel_ids, counts, edge_capacity, in_capacity, kernel_count, in_out_map, status);
        LATTICE_LAUNCH_CHECK();
    }
    // At most 64 KB of map rows per block, and at most one row per lane.
    const int rows_per_block = std::max(1, std::min(256, 16384 / kernel_count));
    const size_t lds = static_cast<size_t>(rows_per_block) * kernel_count * sizeof(int32_t);
    LATTICE_REQUIRE(lds <= 65536, "kernel count too large for the transposed masks.");
    transposed_masks<<<grid_for(in_capacity, rows_per_block, 1u << 16), 256, lds, stream>>>(
        in_out_map, in_capacity, kernel_count, words, rows_per_block, row_masks);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" size_t lattice_hip_conv_weight_grad_workspace_bytes(int dtype, int kernel_count, int c_in, int c_out,
                                                                int edge_capacity) {
    if (!weight_grad_mfma_ok(dtype, c_in, c_out) || kernel_count <= 0) return 0;
    return weight_grad_partial_bytes(edge_capacity, kernel_count, c_in, c_out);
}

extern "C" int lattice_hip_sparse_conv_weight_grad(int dtype, const void* feats, int n_in, int c_in, const void* cot,
                                                   int out_capacity, int c_out, int weight_layout, int kernel_count,
                                                   const int32_t* in_rows, const int32_t* out_rows,
                                                   const int32_t* counts, int edge_capacity,
                                                   const int32_t* kernel_row_offsets,
                                                   const int32_t* kernel_edge_ids, void* grad, void* workspace,
                                                   size_t workspace_bytes, void* stream_ptr) {
    int rc = check_grad_dtype(dtype);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(n_in >= 0 && out_capacity >= 0 && c_in > 0 && c_out > 0 && kernel_count > 0,
                    "gradient shapes must be positive.");
    LATTICE_REQUIRE(weight_layout == LATTICE_WEIGHT_KERNEL_MAJOR || weight_layout == LATTICE_WEIGHT_DENSE_5D,
                    "weights must have shape (K, C_in, C_out) or (C_out, Kx, Ky, Kz, C_in).");
    LATTICE_REQUIRE(grad && counts && kernel_row_offsets && (edge_capacity == 0 || (in_rows && out_rows && kernel_edge_ids)),
                    "gradient pointers must be non-null.");
    hipStream_t stream = as_stream(stream_ptr);
    GradWeightIndex widx{weight_layout, kernel_count, c_in, c_out};
    if (dtype == LATTICE_F32) {
        return launch_weight_grad<float>(dtype, feats, n_in, cot, out_capacity, widx, in_rows, out_rows, counts,
                                         edge_capacity, kernel_row_offsets, kernel_edge_ids, grad, workspace,
                                         workspace_bytes, stream);
    }
    if (dtype == LATTICE_F16) {
        return launch_weight_grad<_Float16>(dtype, feats, n_in, cot, out_capacity, widx, in_rows, out_rows, counts,
                                            edge_capacity, kernel_row_offsets, kernel_edge_ids, grad, workspace,
                                            workspace_bytes, stream);
    }
    return launch_weight_grad<__bf16>(dtype, feats, n_in, cot, out_capacity, widx, in_rows, out_rows, counts,
                                      edge_capacity, kernel_row_offsets, kernel_edge_ids, grad, workspace,
                                      workspace_bytes, stream);
}
