// CPU oracle for the sparse-convolution hot path.
//
// TEST INFRASTRUCTURE ONLY.  This file is a plain-C++ (MLX-free) restatement
// of the reference CPU route of utakotoba/mlx-lattice.  Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, as the
// checker or as the timed CPU baseline; the product path never calls it.
//
// Each function names the reference lines it follows.  Coordinates are read
// as int64 exactly as the reference does (common_detail.h:78-107), so
// candidate coordinates never wrap.
//
// Build: see oracle/Makefile (g++ -O3 -mf16c -shared -fPIC).
//
// How each function is pinned (tests/test_oracle.py):
//   oracle_kernel_offsets          reference known answers (golden JSON).
//   oracle_kernel_relation         reference known answers (forward, strided,
//                                  first-seen downsample, negative duplicates),
//                                  brute force over small seeded clouds, E = N
//                                  for k2s2, a self edge per submanifold row.
//   oracle_target_kernel_relation  reference known answers, brute force.
//   oracle_generative_relation     reference known answers (test_coordinate_
//   oracle_transposed_kernel_      primitives.py:387-423, test_conv.py:674-700),
//     relation                     brute force over seeded clouds, edge sets
//                                  equal to the forward relation from the
//                                  transposed output back to the input, and
//                                  conv over them == torch conv_transpose3d
//                                  on a fully occupied box.
//   oracle_grouped_view            reference known answers (the 10-tuple's
//                                  grouped CSR entries).
//   oracle_implicit_gemm_view      reference known answers (forward, target,
//                                  K = 33 two-word masks).
//   oracle_conv_features           reference known answers, dense box ==
//                                  torch conv3d(padding=1), k2s2 == strided
//                                  dense conv3d, fp16 rounding of the two CPU
//                                  routes checked against a float64 sum.
//   oracle_conv_input_grad         reference known answers (gradients of
//   oracle_conv_weight_grad        tests/ops/test_conv.py:401-487), torch
//                                  autograd of the dense conv3d on a fully
//                                  occupied box, adjointness with
//                                  oracle_conv_features on seeded clouds.
//   oracle_pool_features           reference known answers (tests/ops/
//   oracle_pool_grad               test_pool.py:32-117), a numpy brute force,
//                                  sum pooling == conv with all-ones weights.
//   oracle_sparse_quantize,        reference known answers (tests/ops/
//   oracle_voxelize_features(_grad), test_quantization.py:39-335), brute
//   oracle_point_voxel_map,        force with numpy (np.unique first-seen
//   oracle_point_features(_grad)   order, bincount), trilinear weights
//                                  reproduce affine fields exactly and sum
//                                  to one, gradients adjoint to the forward.
//   oracle_quantized_conv_features unpack formula on hand-built words, equal
//   oracle_dequantize_mapped       to the float route on dequantized weights.
// Not restated here, hence parity unpinned: the reference's quantizer
// (mx.quantize codes and scales; the product defines its own) and the tie
// order of the reference's mask argsort beyond its three-row known answer.

#include <immintrin.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <limits>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

using Coord = std::array<int64_t, 4>;
using Edge = std::array<int32_t, 3>;

// FNV-1a over the four coordinate words, masked to 31 bits.  Follows
// native/features/coordinates/cpu/common_detail.h:68-77.  The hash only
// affects bucket placement; results do not depend on it.
struct CoordHash {
    size_t operator()(const Coord& c) const {
        uint32_t h = 2166136261u;
        for (int i = 0; i < 4; ++i) {
            h = (h ^ static_cast<uint32_t>(c[i])) * 16777619u;
        }
        return static_cast<size_t>(h & 0x7fffffffu);
    }
};

using RowMap = std::unordered_map<Coord, int32_t, CoordHash>;

std::vector<Coord> read_coords(const int32_t* coords, int rows) {
    std::vector<Coord> out(static_cast<size_t>(rows));
    for (int r = 0; r < rows; ++r) {
        for (int a = 0; a < 4; ++a) {
            out[r][a] = coords[static_cast<size_t>(r) * 4 + a];
        }
    }
    return out;
}

// first_row_map: quantization_detail.h:395-402 (emplace keeps the first row).
RowMap first_row_map(const std::vector<Coord>& values) {
    RowMap rows;
    rows.reserve(values.size());
    for (int r = 0; r < static_cast<int>(values.size()); ++r) {
        rows.emplace(values[r], r);
    }
    return rows;
}

// floor_div: quantization_detail.h:3-10.
int64_t floor_div(int64_t v, int64_t d) {
    int64_t q = v / d;
    int64_t r = v % d;
    if (r != 0 && ((r < 0) != (d < 0))) {
        --q;
    }
    return q;
}

// downsample_values: quantization_detail.h:12-31 (first-seen order).
std::vector<Coord> downsample_values(const std::vector<Coord>& values,
                                     const int* stride) {
    std::vector<Coord> out;
    std::unordered_set<Coord, CoordHash> seen;
    seen.reserve(values.size());
    for (const auto& c : values) {
        Coord q = {c[0], floor_div(c[1], stride[0]), floor_div(c[2], stride[1]),
                   floor_div(c[3], stride[2])};
        if (seen.insert(q).second) {
            out.push_back(q);
        }
    }
    return out;
}

// kernel_input_coord: relation_views_detail.h:1-13.
Coord kernel_input_coord(const Coord& o, const int* off, const int* stride,
                         const int* pad) {
    return {o[0], o[1] * stride[0] + off[0] - pad[0],
            o[2] * stride[1] + off[1] - pad[1],
            o[3] * stride[2] + off[2] - pad[2]};
}

// write_map_rows: relation_views_detail.h:15-50.  Tails are zero-filled as
// write_i32 does (common_detail.h:121-125).
void write_map_rows(const std::vector<Edge>& edges, int out_capacity,
                    int edge_capacity, int32_t* in_rows, int32_t* out_rows,
                    int32_t* kernel_ids, int32_t* row_offsets) {
    std::fill(in_rows, in_rows + edge_capacity, 0);
    std::fill(out_rows, out_rows + edge_capacity, 0);
    std::fill(kernel_ids, kernel_ids + edge_capacity, 0);
    int current = 0;
    int n = 0;
    for (const auto& e : edges) {
        while (current <= e[1] && current < out_capacity) {
            row_offsets[current++] = n;
        }
        in_rows[n] = e[0];
        out_rows[n] = e[1];
        kernel_ids[n] = e[2];
        ++n;
    }
    while (current <= out_capacity) {
        row_offsets[current++] = n;
    }
}

void write_coords(const std::vector<Coord>& values, int capacity,
                  int32_t* out) {
    std::fill(out, out + static_cast<size_t>(capacity) * 4, 0);
    for (size_t r = 0; r < values.size(); ++r) {
        for (int a = 0; a < 4; ++a) {
            out[r * 4 + a] = static_cast<int32_t>(values[r][a]);
        }
    }
}

inline float half_to_float(uint16_t h) { return _cvtsh_ss(h); }
inline uint16_t float_to_half(float f) {
    return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
}

int hardware_threads(int requested) {
    if (requested > 0) {
        return requested;
    }
    auto hw = std::thread::hardware_concurrency();
    return hw == 0 ? 1 : static_cast<int>(hw);
}

// parallel_for with the reference grain: cpu/algorithms.cpp:30-67.
template <typename Fn>
void parallel_for(int begin, int end, int threads, Fn fn) {
    constexpr int kGrain = 4096;
    int count = end - begin;
    if (count <= kGrain || threads <= 1) {
        for (int i = begin; i < end; ++i) fn(i);
        return;
    }
    int workers = std::min(threads, std::max(1, (count + kGrain - 1) / kGrain));
    int block = (count + workers - 1) / workers;
    std::vector<std::thread> pool;
    for (int w = 1; w < workers; ++w) {
        int first = begin + w * block;
        int last = std::min(end, first + block);
        if (first >= last) continue;
        pool.emplace_back([first, last, &fn]() {
            for (int i = first; i < last; ++i) fn(i);
        });
    }
    int first_last = std::min(end, begin + block);
    for (int i = begin; i < first_last; ++i) fn(i);
    for (auto& t : pool) t.join();
}

// parallel_rows: cpu/quantized.cpp:15-44.
template <typename Fn>
void parallel_rows(int rows, int threads, Fn fn) {
    int workers = std::min(rows, threads);
    if (workers <= 1 || rows < 1024) {
        for (int r = 0; r < rows; ++r) fn(r);
        return;
    }
    int block = (rows + workers - 1) / workers;
    std::vector<std::thread> pool;
    for (int w = 1; w < workers; ++w) {
        int b = w * block;
        int e = std::min(rows, b + block);
        if (b < e) {
            pool.emplace_back([b, e, &fn]() {
                for (int r = b; r < e; ++r) fn(r);
            });
        }
    }
    for (int r = 0; r < std::min(rows, block); ++r) fn(r);
    for (auto& t : pool) t.join();
}

}  // namespace

extern "C" {

// kernel_offsets: native/features/coordinates/offsets.cpp:11-45.
// Writes K*3 ints; returns K.
int oracle_kernel_offsets(const int* size, const int* dilation, int32_t* out) {
    std::vector<int> axes[3];
    for (int a = 0; a < 3; ++a) {
        if (size[a] % 2 == 1) {
            for (int v = -(size[a] / 2); v <= size[a] / 2; ++v) axes[a].push_back(v);
        } else {
            for (int v = 0; v < size[a]; ++v) axes[a].push_back(v);
        }
    }
    int k = 0;
    for (int x : axes[0])
        for (int y : axes[1])
            for (int z : axes[2]) {
                if (out) {
                    out[k * 3 + 0] = x * dilation[0];
                    out[k * 3 + 1] = y * dilation[1];
                    out[k * 3 + 2] = z * dilation[2];
                }
                ++k;
            }
    return k;
}

// write_kernel_relation: relation_build_detail.h:3-41.  Output capacities as
// make_kernel_relation sizes them (relations.cpp:540-553): out rows = rows,
// edges = rows*K.  counts = [E, N_out].
void oracle_kernel_relation(const int32_t* coords, int rows, int active_rows,
                            const int32_t* offsets, int K, const int* stride,
                            const int* padding, int32_t* in_rows,
                            int32_t* out_rows, int32_t* kernel_ids,
                            int32_t* row_offsets, int32_t* out_coords,
                            int32_t* counts) {
    auto values = read_coords(coords, rows);
    values.resize(std::min(active_rows, rows));
    auto map = first_row_map(values);
    bool identity = stride[0] == 1 && stride[1] == 1 && stride[2] == 1 &&
                    padding[0] == 0 && padding[1] == 0 && padding[2] == 0;
    auto out_values = identity ? values : downsample_values(values, stride);
    std::vector<Edge> edges;
    edges.reserve(out_values.size() * K);
    for (int o = 0; o < static_cast<int>(out_values.size()); ++o) {
        for (int k = 0; k < K; ++k) {
            auto cand = kernel_input_coord(out_values[o], offsets + 3 * k,
                                           stride, padding);
            auto it = map.find(cand);
            if (it != map.end()) edges.push_back({it->second, o, k});
        }
    }
    write_map_rows(edges, rows, rows * K, in_rows, out_rows, kernel_ids,
                   row_offsets);
    write_coords(out_values, rows, out_coords);
    counts[0] = static_cast<int32_t>(edges.size());
    counts[1] = static_cast<int32_t>(out_values.size());
}

// write_target_kernel_relation: relation_build_detail.h:43-80.  Out
// capacity = target_rows, edges = target_rows*K.
void oracle_target_kernel_relation(
    const int32_t* coords, int rows, int active_rows,
    const int32_t* target_coords, int target_rows, int target_active_rows,
    const int32_t* offsets, int K, const int* stride, const int* padding,
    int32_t* in_rows, int32_t* out_rows, int32_t* kernel_ids,
    int32_t* row_offsets, int32_t* counts) {
    auto values = read_coords(coords, rows);
    values.resize(std::min(active_rows, rows));
    auto targets = read_coords(target_coords, target_rows);
    int t_active = std::min(target_active_rows, target_rows);
    auto map = first_row_map(values);
    std::vector<Edge> edges;
    for (int o = 0; o < t_active; ++o) {
        for (int k = 0; k < K; ++k) {
            auto cand = kernel_input_coord(targets[o], offsets + 3 * k, stride,
                                           padding);
            auto it = map.find(cand);
            if (it != map.end()) edges.push_back({it->second, o, k});
        }
    }
    write_map_rows(edges, target_rows, target_rows * K, in_rows, out_rows,
                   kernel_ids, row_offsets);
    counts[0] = static_cast<int32_t>(edges.size());
    counts[1] = t_active;
}

// write_generative_relation: relation_build_detail.h:82-117.  Output row
// in*K + k is coord*stride + offset[k] (no padding, no deduplication); one
// edge per output row.  Capacities rows*K (relations.cpp:599-629).
void oracle_generative_relation(const int32_t* coords, int rows,
                                int active_rows, const int32_t* offsets, int K,
                                const int* stride, int32_t* in_rows,
                                int32_t* out_rows, int32_t* kernel_ids,
                                int32_t* row_offsets, int32_t* out_coords,
                                int32_t* counts) {
    auto values = read_coords(coords, rows);
    values.resize(std::min(active_rows, rows));
    std::vector<Edge> edges;
    std::vector<Coord> out_values;
    for (int in = 0; in < static_cast<int>(values.size()); ++in) {
        for (int k = 0; k < K; ++k) {
            const int o = static_cast<int>(out_values.size());
            out_values.push_back({values[in][0],
                                  values[in][1] * stride[0] + offsets[3 * k],
                                  values[in][2] * stride[1] + offsets[3 * k + 1],
                                  values[in][3] * stride[2] + offsets[3 * k + 2]});
            edges.push_back({in, o, k});
        }
    }
    write_map_rows(edges, rows * K, rows * K, in_rows, out_rows, kernel_ids,
                   row_offsets);
    write_coords(out_values, rows * K, out_coords);
    counts[0] = static_cast<int32_t>(edges.size());
    counts[1] = static_cast<int32_t>(out_values.size());
}

// can_use_direct_transposed_relation: relations.cpp:107-127.  The stride
// exceeds the offsets' extent on every axis, so no two (row, offset)
// candidates of distinct input coordinates coincide.
int oracle_direct_transposed(const int32_t* offsets, int K, const int* stride) {
    if (K <= 0) return 0;
    for (int a = 0; a < 3; ++a) {
        int lo = offsets[a], hi = offsets[a];
        for (int k = 0; k < K; ++k) {
            lo = std::min(lo, offsets[3 * k + a]);
            hi = std::max(hi, offsets[3 * k + a]);
        }
        if (stride[a] <= hi - lo) return 0;
    }
    return 1;
}

// write_transposed_kernel_relation: relation_build_detail.h:119-196.
// Candidates coord*stride + offset[k] - padding, enumerated input-row major.
//   direct: output row in*K + k per candidate (as the generative relation);
//   otherwise: first-seen deduplicated output rows, edges stably sorted by
//   (out_row, kernel_id, in_row) (write_map, relation_views_detail.h:52-82).
// Capacities rows*K (relations.cpp:631-670).
void oracle_transposed_kernel_relation(
    const int32_t* coords, int rows, int active_rows, const int32_t* offsets,
    int K, const int* stride, const int* padding, int32_t* in_rows,
    int32_t* out_rows, int32_t* kernel_ids, int32_t* row_offsets,
    int32_t* out_coords, int32_t* counts) {
    auto values = read_coords(coords, rows);
    values.resize(std::min(active_rows, rows));
    const bool direct = oracle_direct_transposed(offsets, K, stride) != 0;
    std::vector<Edge> edges;
    std::vector<Coord> out_values;
    RowMap seen;
    for (int in = 0; in < static_cast<int>(values.size()); ++in) {
        for (int k = 0; k < K; ++k) {
            Coord cand = {values[in][0],
                          values[in][1] * stride[0] + offsets[3 * k] - padding[0],
                          values[in][2] * stride[1] + offsets[3 * k + 1] - padding[1],
                          values[in][3] * stride[2] + offsets[3 * k + 2] - padding[2]};
            int o;
            if (direct) {
                o = in * K + k;
                out_values.push_back(cand);
            } else {
                auto [it, inserted] =
                    seen.emplace(cand, static_cast<int32_t>(out_values.size()));
                if (inserted) out_values.push_back(cand);
                o = it->second;
            }
            edges.push_back({in, o, k});
        }
    }
    if (!direct) {
        std::stable_sort(edges.begin(), edges.end(),
                         [](const Edge& a, const Edge& b) {
                             if (a[1] != b[1]) return a[1] < b[1];
                             if (a[2] != b[2]) return a[2] < b[2];
                             return a[0] < b[0];
                         });
    }
    write_map_rows(edges, rows * K, rows * K, in_rows, out_rows, kernel_ids,
                   row_offsets);
    write_coords(out_values, rows * K, out_coords);
    counts[0] = static_cast<int32_t>(edges.size());
    counts[1] = static_cast<int32_t>(out_values.size());
}

// write_relation_grouped_view: relation_views_detail.h:84-120.  Stable
// counting sort of edge ids by group; edge_ids tail = -1.
void oracle_grouped_view(const int32_t* group_ids, int edge_capacity,
                         int edge_count, int group_count, int32_t* offsets,
                         int32_t* edge_ids) {
    int n = std::max(0, std::min(edge_count, edge_capacity));
    std::fill(offsets, offsets + group_count + 1, 0);
    for (int e = 0; e < n; ++e) {
        int g = group_ids[e];
        if (g >= 0 && g < group_count) ++offsets[g + 1];
    }
    for (int g = 0; g < group_count; ++g) offsets[g + 1] += offsets[g];
    std::vector<int32_t> cursor(offsets, offsets + group_count);
    std::fill(edge_ids, edge_ids + edge_capacity, -1);
    for (int e = 0; e < n; ++e) {
        int g = group_ids[e];
        if (g >= 0 && g < group_count) edge_ids[cursor[g]++] = e;
    }
}

// write_relation_implicit_gemm_view: relation_views_detail.h:122-169.
void oracle_implicit_gemm_view(const int32_t* source_coords, int source_rows,
                               int source_active, const int32_t* output_coords,
                               int output_rows, int output_active,
                               const int32_t* offsets, int K,
                               const int* stride, const int* padding,
                               int32_t* out_in_map, int32_t* row_masks) {
    auto src = read_coords(source_coords, source_rows);
    auto outs = read_coords(output_coords, output_rows);
    int s_active = std::max(0, std::min(source_active, source_rows));
    int o_active = std::max(0, std::min(output_active, output_rows));
    auto map = first_row_map(src);
    int words = (K + 31) / 32;
    std::fill(out_in_map, out_in_map + static_cast<size_t>(output_rows) * K, -1);
    std::fill(row_masks, row_masks + static_cast<size_t>(output_rows) * words, 0);
    for (int o = 0; o < o_active; ++o) {
        for (int k = 0; k < K; ++k) {
            auto cand = kernel_input_coord(outs[o], offsets + 3 * k, stride,
                                           padding);
            auto it = map.find(cand);
            if (it == map.end() || it->second >= s_active) continue;
            out_in_map[static_cast<size_t>(o) * K + k] = it->second;
            row_masks[static_cast<size_t>(o) * words + k / 32] |=
                static_cast<int32_t>(1u << (k % 32));
        }
    }
}

// Float sparse conv, cpu/algorithms.cpp:180-302 + eval_route :484-508.
// weights: layout 0 = mapped (K, C_in, C_out) contiguous, layout 1 = dense
// 5d (C_out, Kx, Ky, Kz, C_in) contiguous.  dtype: 0 = fp32, 1 = fp16 (raw
// uint16 bits).  Square C in {16,32,64} uses the fp32 accumulator with one
// final rounding (eval_dense_channels_typed); all other channel pairs round
// the running sum to the feature dtype after every multiply-add (eval_typed).
// threads <= 0 means std::thread::hardware_concurrency().
void oracle_conv_features(int dtype, const void* feats, const void* weights,
                          int weight_layout, int n_in, int c_in, int c_out,
                          int K, const int32_t* in_rows,
                          const int32_t* kernel_ids, const int32_t* counts,
                          int edge_capacity, const int32_t* row_offsets,
                          int out_capacity, void* out, int threads) {
    int edge_total = std::min(counts[0], edge_capacity);
    int active_out = std::min(counts[1], out_capacity);
    int nthreads = hardware_threads(threads);
    bool dense_route = c_in == c_out && (c_in == 16 || c_in == 32 || c_in == 64);
    (void)n_in;
    auto widx = [&](int k, int ci, int co) -> size_t {
        if (weight_layout == 0) {
            return (static_cast<size_t>(k) * c_in + ci) * c_out + co;
        }
        return (static_cast<size_t>(co) * K + k) * c_in + ci;
    };
    auto body = [&](auto load, auto store, auto round) {
        parallel_for(0, out_capacity, nthreads, [&](int o) {
            std::vector<float> acc(static_cast<size_t>(c_out), 0.0f);
            if (o < active_out) {
                for (int e = row_offsets[o]; e < row_offsets[o + 1]; ++e) {
                    if (e < 0 || e >= edge_total) continue;
                    int in = in_rows[e];
                    int k = kernel_ids[e];
                    if (in < 0 || k < 0) continue;
                    for (int ci = 0; ci < c_in; ++ci) {
                        float v = load(feats, static_cast<size_t>(in) * c_in + ci);
                        for (int co = 0; co < c_out; ++co) {
                            float w = load(weights, widx(k, ci, co));
                            if (dense_route) {
                                acc[co] += v * w;
                            } else {
                                acc[co] = round(acc[co] + v * w);
                            }
                        }
                    }
                }
            }
            for (int co = 0; co < c_out; ++co) {
                store(out, static_cast<size_t>(o) * c_out + co, acc[co]);
            }
        });
    };
    if (dtype == 0) {
        body([](const void* p, size_t i) { return static_cast<const float*>(p)[i]; },
             [](void* p, size_t i, float v) { static_cast<float*>(p)[i] = v; },
             [](float v) { return v; });
    } else {
        body([](const void* p, size_t i) {
                 return half_to_float(static_cast<const uint16_t*>(p)[i]);
             },
             [](void* p, size_t i, float v) {
                 static_cast<uint16_t*>(p)[i] = float_to_half(v);
             },
             [](float v) { return half_to_float(float_to_half(v)); });
    }
}

// Input gradient, eval_input_grad_typed (cpu/algorithms.cpp:355-410): for
// every input row and input channel, one fp32 accumulator over the row's
// edges in the input-grouped CSR (in_row_offsets / in_edge_ids) and every
// output channel, cot[out][co] * W[k, ci, co]; one rounding to the feature
// dtype.  Edges past counts[0] and out rows past out_capacity are skipped.
void oracle_conv_input_grad(int dtype, const void* cot, const void* weights,
                            int weight_layout, int in_capacity, int c_in,
                            int c_out, int K, const int32_t* out_rows,
                            const int32_t* kernel_ids, const int32_t* counts,
                            int edge_capacity, const int32_t* in_row_offsets,
                            const int32_t* in_edge_ids, int out_capacity,
                            void* grad, int threads) {
    int edge_total = std::min(counts[0], edge_capacity);
    int nthreads = hardware_threads(threads);
    auto widx = [&](int k, int ci, int co) -> size_t {
        if (weight_layout == 0) {
            return (static_cast<size_t>(k) * c_in + ci) * c_out + co;
        }
        return (static_cast<size_t>(co) * K + k) * c_in + ci;
    };
    auto body = [&](auto load, auto store) {
        parallel_for(0, in_capacity, nthreads, [&](int in_row) {
            for (int ci = 0; ci < c_in; ++ci) {
                float acc = 0.0f;
                for (int cur = in_row_offsets[in_row]; cur < in_row_offsets[in_row + 1]; ++cur) {
                    int e = in_edge_ids[cur];
                    if (e < 0 || e >= edge_total) continue;
                    int o = out_rows[e];
                    int k = kernel_ids[e];
                    if (o < 0 || k < 0 || o >= out_capacity) continue;
                    for (int co = 0; co < c_out; ++co) {
                        acc += load(cot, static_cast<size_t>(o) * c_out + co) *
                               load(weights, widx(k, ci, co));
                    }
                }
                store(grad, static_cast<size_t>(in_row) * c_in + ci, acc);
            }
        });
    };
    if (dtype == 0) {
        body([](const void* p, size_t i) { return static_cast<const float*>(p)[i]; },
             [](void* p, size_t i, float v) { static_cast<float*>(p)[i] = v; });
    } else {
        body([](const void* p, size_t i) {
                 return half_to_float(static_cast<const uint16_t*>(p)[i]);
             },
             [](void* p, size_t i, float v) {
                 static_cast<uint16_t*>(p)[i] = float_to_half(v);
             });
    }
}

// Weight gradient, eval_weight_grad_typed (cpu/algorithms.cpp:413-481): for
// every (k, ci, co), one fp32 accumulator over the edges of kernel k in the
// kernel-grouped CSR (kernel_row_offsets / kernel_edge_ids) of
// feats[in][ci] * cot[out][co]; one rounding, written in the weight's
// layout.
void oracle_conv_weight_grad(int dtype, const void* feats, const void* cot,
                             int weight_layout, int c_in, int c_out, int K,
                             const int32_t* in_rows, const int32_t* out_rows,
                             const int32_t* counts, int edge_capacity,
                             const int32_t* kernel_row_offsets,
                             const int32_t* kernel_edge_ids, int out_capacity,
                             void* grad, int threads) {
    int edge_total = std::min(counts[0], edge_capacity);
    int nthreads = hardware_threads(threads);
    auto widx = [&](int k, int ci, int co) -> size_t {
        if (weight_layout == 0) {
            return (static_cast<size_t>(k) * c_in + ci) * c_out + co;
        }
        return (static_cast<size_t>(co) * K + k) * c_in + ci;
    };
    auto body = [&](auto load, auto store) {
        parallel_for(0, K * c_in * c_out, nthreads, [&](int index) {
            int co = index % c_out;
            int ci = (index / c_out) % c_in;
            int k = index / (c_in * c_out);
            float acc = 0.0f;
            for (int cur = kernel_row_offsets[k]; cur < kernel_row_offsets[k + 1]; ++cur) {
                int e = kernel_edge_ids[cur];
                if (e < 0 || e >= edge_total) continue;
                int in = in_rows[e];
                int o = out_rows[e];
                if (in < 0 || o < 0 || o >= out_capacity) continue;
                acc += load(feats, static_cast<size_t>(in) * c_in + ci) *
                       load(cot, static_cast<size_t>(o) * c_out + co);
            }
            store(grad, widx(k, ci, co), acc);
        });
    };
    if (dtype == 0) {
        body([](const void* p, size_t i) { return static_cast<const float*>(p)[i]; },
             [](void* p, size_t i, float v) { static_cast<float*>(p)[i] = v; });
    } else {
        body([](const void* p, size_t i) {
                 return half_to_float(static_cast<const uint16_t*>(p)[i]);
             },
             [](void* p, size_t i, float v) {
                 static_cast<uint16_t*>(p)[i] = float_to_half(v);
             });
    }
}

// Sparse pooling, native/features/pooling/cpu/algorithms.cpp:180-242 (eval):
// every output row starts at the reduction identity (-inf for max, 0
// otherwise); rows below counts[1] reduce feats[in_rows[e]] over their CSR
// edges; avg divides by max(degree, 1).  mode: 0 sum, 1 max, 2 avg; fp32.
void oracle_pool_features(int mode, const float* feats, int channels,
                          const int32_t* in_rows, const int32_t* row_offsets,
                          const int32_t* counts, int out_capacity,
                          float* out) {
    int out_count = std::min(counts[1], out_capacity);
    float identity = mode == 1 ? -std::numeric_limits<float>::infinity() : 0.0f;
    std::fill(out, out + static_cast<size_t>(out_capacity) * channels, identity);
    for (int o = 0; o < out_count; ++o) {
        float* row = out + static_cast<size_t>(o) * channels;
        for (int e = row_offsets[o]; e < row_offsets[o + 1]; ++e) {
            const float* f = feats + static_cast<size_t>(in_rows[e]) * channels;
            for (int c = 0; c < channels; ++c) {
                row[c] = mode == 1 ? std::max(row[c], f[c]) : row[c] + f[c];
            }
        }
    }
    if (mode != 2) return;
    for (int o = 0; o < out_count; ++o) {
        float scale = 1.0f / static_cast<float>(std::max(row_offsets[o + 1] - row_offsets[o], 1));
        float* row = out + static_cast<size_t>(o) * channels;
        for (int c = 0; c < channels; ++c) row[c] *= scale;
    }
}

// Pooling gradient, pooling/cpu/algorithms.cpp:245-331 (eval_grad) over the
// input-grouped CSR (the exclusive layout's direct edge is the same single
// edge): grad[in][c] = sum over the row's edges whose out row is below
// counts[1] of cot[out][c] * scale; scale 1 (sum), 1/max(degree(out), 1)
// (avg), and for max 1/(number of the out row's edges whose feature equals
// the pooled value) when feats[in][c] equals it, else 0.
void oracle_pool_grad(int mode, const float* cot, const float* feats,
                      const float* pooled, int channels,
                      const int32_t* in_rows, const int32_t* out_rows,
                      const int32_t* row_offsets, const int32_t* counts,
                      const int32_t* in_row_offsets,
                      const int32_t* in_edge_ids, int in_capacity,
                      int out_capacity, float* grad) {
    int out_count = std::min(counts[1], out_capacity);
    for (int in = 0; in < in_capacity; ++in) {
        for (int c = 0; c < channels; ++c) {
            float value = 0.0f;
            for (int cur = in_row_offsets[in]; cur < in_row_offsets[in + 1]; ++cur) {
                int e = in_edge_ids[cur];
                if (e < 0) continue;
                int o = out_rows[e];
                if (o < 0 || o >= out_count) continue;
                float scale = 1.0f;
                if (mode == 1) {
                    float fv = feats[static_cast<size_t>(in) * channels + c];
                    float pv = pooled[static_cast<size_t>(o) * channels + c];
                    if (fv != pv) continue;
                    int ties = 0;
                    for (int e2 = row_offsets[o]; e2 < row_offsets[o + 1]; ++e2) {
                        if (feats[static_cast<size_t>(in_rows[e2]) * channels + c] == pv) ++ties;
                    }
                    if (ties == 0) continue;
                    scale = 1.0f / static_cast<float>(ties);
                } else if (mode == 2) {
                    scale = 1.0f / static_cast<float>(std::max(row_offsets[o + 1] - row_offsets[o], 1));
                }
                value += cot[static_cast<size_t>(o) * channels + c] * scale;
            }
            grad[static_cast<size_t>(in) * channels + c] = value;
        }
    }
}

// Quantized sparse conv, cpu/quantized.cpp:54-141.  weights uint32
// (K, storage_c_in*bits/32, C_out); scales/biases (K, storage_c_in/g, C_out)
// in the feature dtype; fp32 accumulator, one rounding.
void oracle_quantized_conv_features(
    int dtype, const void* feats, const uint32_t* weights, const void* scales,
    const void* biases, int c_in, int c_out, int storage_c_in, int group_size,
    int bits, int K, const int32_t* in_rows, const int32_t* kernel_ids,
    const int32_t* counts, int edge_capacity, const int32_t* row_offsets,
    int out_capacity, void* out, int threads) {
    int out_count = std::min(counts[1], out_capacity);
    int edge_count = std::min(counts[0], edge_capacity);
    int packed_words = storage_c_in * bits / 32;
    int groups = storage_c_in / group_size;
    uint32_t mask = (bits == 32) ? 0xffffffffu : ((1u << bits) - 1u);
    auto ld = [dtype](const void* p, size_t i) -> float {
        return dtype == 0 ? static_cast<const float*>(p)[i]
                          : half_to_float(static_cast<const uint16_t*>(p)[i]);
    };
    auto st = [dtype](void* p, size_t i, float v) {
        if (dtype == 0) static_cast<float*>(p)[i] = v;
        else static_cast<uint16_t*>(p)[i] = float_to_half(v);
    };
    parallel_rows(out_capacity, hardware_threads(threads), [&](int o) {
        size_t base = static_cast<size_t>(o) * c_out;
        if (o >= out_count) {
            for (int co = 0; co < c_out; ++co) st(out, base + co, 0.0f);
            return;
        }
        for (int co = 0; co < c_out; ++co) {
            float acc = 0.0f;
            for (int e = row_offsets[o]; e < row_offsets[o + 1]; ++e) {
                if (e < 0 || e >= edge_count) continue;
                int in = in_rows[e];
                int k = kernel_ids[e];
                if (in < 0 || k < 0 || k >= K) continue;
                int wrow = k * packed_words;
                int qrow = k * groups;
                for (int ci = 0; ci < c_in; ++ci) {
                    int g = ci / group_size;
                    int bit = ci * bits;
                    uint32_t word = weights[static_cast<size_t>(wrow) * c_out +
                                            static_cast<size_t>(bit >> 5) * c_out + co];
                    uint32_t q = (word >> (bit & 31)) & mask;
                    size_t sidx = static_cast<size_t>(qrow + g) * c_out + co;
                    float w = static_cast<float>(q) * ld(scales, sidx) + ld(biases, sidx);
                    acc += ld(feats, static_cast<size_t>(in) * c_in + ci) * w;
                }
            }
            st(out, base + co, acc);
        }
    });
}

// Affine dequantization of the spatial packed layout (core/quantized.py:
// 191-223 with the unpack rule of cpu/quantized.cpp:54-62).  Writes the
// mapped (K, C_in, C_out) fp32 weight for logical channels c_in.
void oracle_dequantize_mapped(const uint32_t* weights, const float* scales,
                              const float* biases, int K, int c_in, int c_out,
                              int storage_c_in, int group_size, int bits,
                              float* out) {
    int packed_words = storage_c_in * bits / 32;
    int groups = storage_c_in / group_size;
    uint32_t mask = (1u << bits) - 1u;
    for (int k = 0; k < K; ++k)
        for (int ci = 0; ci < c_in; ++ci)
            for (int co = 0; co < c_out; ++co) {
                int bit = ci * bits;
                uint32_t word = weights[(static_cast<size_t>(k) * packed_words + (bit >> 5)) * c_out + co];
                uint32_t q = (word >> (bit & 31)) & mask;
                size_t s = (static_cast<size_t>(k) * groups + ci / group_size) * c_out + co;
                out[(static_cast<size_t>(k) * c_in + ci) * c_out + co] =
                    static_cast<float>(q) * scales[s] + biases[s];
            }
}

// Round trip through IEEE binary16 with round-to-nearest-even.
void oracle_round_half(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = float_to_half(in[i]);
}

// ------------------------------------------------- point quantization --
// Float arithmetic below is plain IEEE binary32 with one rounding per
// operation (the Makefile builds with -ffp-contract=off).

// voxel_coord_for_point: quantization_detail.h:66-89.
static Coord voxel_of(const float* points, const int32_t* batches, int row,
                      const float* size, const float* origin) {
    const float* p = points + static_cast<size_t>(row) * 3;
    return {batches[row],
            static_cast<int64_t>(std::floor((p[0] - origin[0]) / size[0])),
            static_cast<int64_t>(std::floor((p[1] - origin[1]) / size[1])),
            static_cast<int64_t>(std::floor((p[2] - origin[2]) / size[2]))};
}

// write_sparse_quantization: quantization_detail.h:91-128.  Voxels in
// first-seen point order; inverse_rows -1 for inactive points; counts per
// voxel, zero tail; coords zero tail.  Returns the voxel count.
int oracle_sparse_quantize(const float* points, const int32_t* batches,
                           int rows, int active_rows, const float* size,
                           const float* origin, int32_t* coords,
                           int32_t* inverse_rows, int32_t* counts) {
    const int n = std::min(active_rows, rows);
    RowMap seen;
    std::vector<Coord> out;
    std::fill(inverse_rows, inverse_rows + rows, -1);
    std::fill(counts, counts + rows, 0);
    for (int p = 0; p < n; ++p) {
        Coord c = voxel_of(points, batches, p, size, origin);
        auto [it, inserted] = seen.emplace(c, static_cast<int32_t>(out.size()));
        if (inserted) out.push_back(c);
        inverse_rows[p] = it->second;
        counts[it->second] += 1;
    }
    write_coords(out, rows, coords);
    return static_cast<int>(out.size());
}

// write_voxel_features (quantization_detail.h:141-170) and
// write_voxel_feature_grad (:172-200).  mode 0 = sum, 1 = mean.
void oracle_voxelize_features(int mode, const float* feats, int point_rows,
                              int active_rows, int channels,
                              const int32_t* inverse_rows,
                              const int32_t* counts, int voxel_rows,
                              float* out) {
    const int n = std::min(active_rows, point_rows);
    std::fill(out, out + static_cast<size_t>(voxel_rows) * channels, 0.0f);
    for (int p = 0; p < n; ++p) {
        const int v = inverse_rows[p];
        if (v < 0 || v >= voxel_rows) continue;
        const float scale =
            mode == 1 ? 1.0f / static_cast<float>(std::max(counts[v], 1)) : 1.0f;
        for (int c = 0; c < channels; ++c) {
            out[static_cast<size_t>(v) * channels + c] +=
                feats[static_cast<size_t>(p) * channels + c] * scale;
        }
    }
}

void oracle_voxelize_features_grad(int mode, const float* cot, int point_rows,
                                   int active_rows, int channels,
                                   const int32_t* inverse_rows,
                                   const int32_t* counts, int voxel_rows,
                                   float* grad) {
    const int n = std::min(active_rows, point_rows);
    std::fill(grad, grad + static_cast<size_t>(point_rows) * channels, 0.0f);
    for (int p = 0; p < n; ++p) {
        const int v = inverse_rows[p];
        if (v < 0 || v >= voxel_rows) continue;
        const float scale =
            mode == 1 ? 1.0f / static_cast<float>(std::max(counts[v], 1)) : 1.0f;
        for (int c = 0; c < channels; ++c) {
            grad[static_cast<size_t>(p) * channels + c] =
                cot[static_cast<size_t>(v) * channels + c] * scale;
        }
    }
}

// write_nearest_point_voxel_map (quantization_detail.h:213-257) and
// write_linear_point_voxel_map (:259-318).  mode 0 = nearest, 1 = linear.
// rows/weights are (point_rows, 8): -1 / 0 where no voxel is found.
void oracle_point_voxel_map(const float* points, const int32_t* batches,
                            int point_rows, int point_active,
                            const int32_t* voxel_coords, int voxel_rows,
                            int voxel_active, const float* size,
                            const float* origin, int mode, int32_t* rows,
                            float* weights) {
    const int n = std::min(point_active, point_rows);
    std::fill(rows, rows + static_cast<size_t>(point_rows) * 8, -1);
    std::fill(weights, weights + static_cast<size_t>(point_rows) * 8, 0.0f);
    auto voxels = read_coords(voxel_coords, voxel_rows);
    voxels.resize(std::min(voxel_active, voxel_rows));
    auto map = first_row_map(voxels);
    for (int p = 0; p < n; ++p) {
        float pos[3];
        for (int a = 0; a < 3; ++a) {
            pos[a] = (points[static_cast<size_t>(p) * 3 + a] - origin[a]) / size[a];
        }
        const size_t base = static_cast<size_t>(p) * 8;
        if (mode == 0) {
            Coord q = {batches[p], static_cast<int64_t>(std::floor(pos[0] + 0.5f)),
                       static_cast<int64_t>(std::floor(pos[1] + 0.5f)),
                       static_cast<int64_t>(std::floor(pos[2] + 0.5f))};
            auto it = map.find(q);
            if (it == map.end()) continue;
            rows[base] = it->second;
            weights[base] = 1.0f;
            continue;
        }
        int64_t lo[3];
        float frac[3];
        for (int a = 0; a < 3; ++a) {
            lo[a] = static_cast<int64_t>(std::floor(pos[a]));
            frac[a] = pos[a] - static_cast<float>(lo[a]);
        }
        for (int corner = 0; corner < 8; ++corner) {
            const int dx = corner & 1, dy = (corner >> 1) & 1, dz = (corner >> 2) & 1;
            Coord q = {batches[p], lo[0] + dx, lo[1] + dy, lo[2] + dz};
            auto it = map.find(q);
            if (it == map.end()) continue;
            const float wx = dx == 0 ? 1.0f - frac[0] : frac[0];
            const float wy = dy == 0 ? 1.0f - frac[1] : frac[1];
            const float wz = dz == 0 ? 1.0f - frac[2] : frac[2];
            rows[base + corner] = it->second;
            weights[base + corner] = wx * wy * wz;
        }
    }
}

// write_point_features (quantization_detail.h:333-361) and
// write_point_feature_grad (:363-391).
void oracle_point_features(const float* values, int voxel_rows, int channels,
                           const int32_t* rows, const float* weights,
                           int point_rows, float* out) {
    std::fill(out, out + static_cast<size_t>(point_rows) * channels, 0.0f);
    for (int p = 0; p < point_rows; ++p)
        for (int corner = 0; corner < 8; ++corner) {
            const int v = rows[static_cast<size_t>(p) * 8 + corner];
            if (v < 0 || v >= voxel_rows) continue;
            const float w = weights[static_cast<size_t>(p) * 8 + corner];
            for (int c = 0; c < channels; ++c) {
                out[static_cast<size_t>(p) * channels + c] +=
                    values[static_cast<size_t>(v) * channels + c] * w;
            }
        }
}

void oracle_point_features_grad(const float* point_grad, int voxel_rows,
                                int channels, const int32_t* rows,
                                const float* weights, int point_rows,
                                float* out) {
    std::fill(out, out + static_cast<size_t>(voxel_rows) * channels, 0.0f);
    for (int p = 0; p < point_rows; ++p)
        for (int corner = 0; corner < 8; ++corner) {
            const int v = rows[static_cast<size_t>(p) * 8 + corner];
            if (v < 0 || v >= voxel_rows) continue;
            const float w = weights[static_cast<size_t>(p) * 8 + corner];
            for (int c = 0; c < channels; ++c) {
                out[static_cast<size_t>(v) * channels + c] +=
                    point_grad[static_cast<size_t>(p) * channels + c] * w;
            }
        }
}

int oracle_hardware_concurrency(void) { return hardware_threads(0); }

}  // extern "C"
