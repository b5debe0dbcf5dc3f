// Coordinate hash, kernel-map (relation) construction and relation views
// for gfx950.
//
// Pipeline of a forward relation (write_kernel_relation,
// native/features/coordinates/cpu/relation_build_detail.h:3-41):
//   1. table clear + insert of the active input rows (packed 64-bit keys,
//      value = minimum row, i.e. the first occurrence: first_row_map,
//      cpu/quantization_detail.h:395-402);
//   2. strided/padded relations only: a second table over floor-divided
//      cells, a representative flag per input row (row == cell's first row),
//      a scan and a scatter that emit the output cells in first-seen order
//      (downsample_values, quantization_detail.h:12-31);
//   3. the map query: a lane per (output row, kernel offset) probes the
//      table, writes the dense out_in_map / row_masks view
//      (relation_views_detail.h:122-169) and a per-row degree from a ballot;
//   4. an exclusive scan of the degrees -> row_offsets and counts[0];
//   5. edge emission in (out_row, kernel_id) order: the same lane layout
//      re-reads out_in_map and places each hit at row_offset + ballot rank;
//   6. grouped CSR views (write_relation_grouped_view,
//      relation_views_detail.h:84-120): a stable partition of edge ids by
//      kernel id and by input row.
// Nothing in this file reads device memory back to the host.

#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <climits>

#include "lattice_common.h"
#include "scan.h"

namespace lattice {
namespace {

constexpr int kThreads = 256;

// ------------------------------------------------------------ offsets ----

struct KernelGeometry {
    Int3 size;
    Int3 dilation;
    Int3 stride;
    Int3 padding;
    int volume;
};

// Offset k in the reference order (offsets.cpp:11-45): x outer, z inner;
// odd extents centred, even extents 0..k-1; times dilation.
__device__ inline Int3 offset_of(int k, const KernelGeometry& g) {
    const int yz = g.size.y * g.size.z;
    int ix = k / yz;
    int rem = k - ix * yz;
    int iy = rem / g.size.z;
    int iz = rem - iy * g.size.z;
    if (g.size.x & 1) ix -= g.size.x / 2;
    if (g.size.y & 1) iy -= g.size.y / 2;
    if (g.size.z & 1) iz -= g.size.z / 2;
    return {ix * g.dilation.x, iy * g.dilation.y, iz * g.dilation.z};
}

__device__ inline int4 load_coord(const int32_t* coords, long long row) {
    return reinterpret_cast<const int4*>(coords)[row];
}

// ------------------------------------------------------------- tables ----

__global__ void __launch_bounds__(kThreads)
clear_table(uint64_t* keys, int32_t* rows, int capacity) {
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < capacity; i += gridDim.x * kThreads) {
        keys[i] = kEmptyKey;
        rows[i] = INT_MAX;
    }
}

// Inserts active rows keyed by their coordinate (cell_stride == 1) or by the
// floor-divided cell (cell_stride > 1 on an axis).
__global__ void __launch_bounds__(kThreads)
insert_rows(CoordTable table, const int32_t* __restrict__ coords, int rows,
            const int32_t* __restrict__ active_rows, Int3 cell, int32_t* status) {
    const int active = min(max(*active_rows, 0), rows);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < active; i += gridDim.x * kThreads) {
        int4 c = load_coord(coords, i);
        int64_t x = c.y, y = c.z, z = c.w;
        if (cell.x != 1 || cell.y != 1 || cell.z != 1) {
            x = floor_div_pos(x, cell.x);
            y = floor_div_pos(y, cell.y);
            z = floor_div_pos(z, cell.z);
        }
        uint64_t key;
        if (!pack_key(c.x, x, y, z, &key)) {
            status[0] = LATTICE_STATUS_COORD_RANGE;
            continue;
        }
        table.insert(key, i);
    }
}

// ---------------------------------------------- strided output planning --

// flags[i] = 1 when input row i is the first row of its floor-divided cell.
__global__ void __launch_bounds__(kThreads)
flag_cell_representatives(CoordTable cells, const int32_t* __restrict__ coords, int rows,
                          const int32_t* __restrict__ active_rows, Int3 cell,
                          int32_t* __restrict__ flags) {
    const int active = min(max(*active_rows, 0), rows);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        int flag = 0;
        if (i < active) {
            int4 c = load_coord(coords, i);
            uint64_t key;
            if (pack_key(c.x, floor_div_pos(c.y, cell.x), floor_div_pos(c.z, cell.y),
                         floor_div_pos(c.w, cell.z), &key)) {
                flag = cells.find(key) == i ? 1 : 0;
            }
        }
        flags[i] = flag;
    }
}

// Scatters representative cells to their first-seen position; zero tail.
__global__ void __launch_bounds__(kThreads)
scatter_cells(const int32_t* __restrict__ coords, int rows, const int32_t* __restrict__ flags,
              const int32_t* __restrict__ positions, const int32_t* __restrict__ counts,
              Int3 cell, int32_t* __restrict__ out_coords) {
    const int n_out = counts[1];
    int4* out = reinterpret_cast<int4*>(out_coords);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        if (flags[i]) {
            int4 c = load_coord(coords, i);
            int4 q;
            q.x = c.x;
            q.y = static_cast<int>(floor_div_pos(c.y, cell.x));
            q.z = static_cast<int>(floor_div_pos(c.z, cell.y));
            q.w = static_cast<int>(floor_div_pos(c.w, cell.z));
            out[positions[i]] = q;
        }
        if (i >= n_out) out[i] = make_int4(0, 0, 0, 0);
    }
}

// Identity output support: out_coords = active prefix of coords, zero tail.
__global__ void __launch_bounds__(kThreads)
copy_active_coords(const int32_t* __restrict__ coords, int rows,
                   const int32_t* __restrict__ active_rows, int32_t* __restrict__ out_coords) {
    const int active = min(max(*active_rows, 0), rows);
    int4* out = reinterpret_cast<int4*>(out_coords);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        out[i] = i < active ? load_coord(coords, i) : make_int4(0, 0, 0, 0);
    }
}

__global__ void set_out_count(const int32_t* __restrict__ src, int limit, int32_t* counts) {
    if (threadIdx.x == 0 && blockIdx.x == 0) counts[1] = min(max(*src, 0), limit);
}

// ------------------------------------------------------------ map query --
//
// Lanes per output row: 32 when K <= 32 (two rows per wave), else 64 with a
// loop over 64-offset chunks.  Each lane probes one offset; the ballot of
// hits gives the row mask words and the degree.

struct QueryArgs {
    const int32_t* out_coords;   // coordinates of the output rows
    int out_capacity;
    const int32_t* out_active;   // device count of active output rows
    const int32_t* offsets;      // device [K,3] or null (closed form)
    KernelGeometry geom;
    int words;
    CoordTable table;
    int32_t* out_in_map;         // [out_capacity, K]
    int32_t* row_masks;          // [out_capacity, words]
    int32_t* degrees;            // [out_capacity] or null
};

template <int kLanes>
__global__ void __launch_bounds__(kThreads) query_map(QueryArgs a) {
    constexpr int kRowsPerWave = kWave / kLanes;
    const int lane = lane_id();
    const int sub = lane / kLanes;          // row slot within the wave
    const int k_lane = lane % kLanes;
    const int K = a.geom.volume;
    const int n_active = min(max(*a.out_active, 0), a.out_capacity);
    const long long waves = static_cast<long long>(gridDim.x) * (kThreads / kWave);
    const long long wave_id = static_cast<long long>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
    for (long long base = wave_id * kRowsPerWave; base < a.out_capacity; base += waves * kRowsPerWave) {
        const long long row = base + sub;
        const bool row_ok = row < a.out_capacity;
        const bool row_active = row < n_active;
        int4 oc = make_int4(0, 0, 0, 0);
        if (row_active) oc = load_coord(a.out_coords, row);
        int degree = 0;
        for (int k0 = 0; k0 < K; k0 += kLanes) {
            const int k = k0 + k_lane;
            int found = -1;
            if (row_active && k < K) {
                Int3 off;
                if (a.offsets != nullptr) {
                    off = {a.offsets[3 * k], a.offsets[3 * k + 1], a.offsets[3 * k + 2]};
                } else {
                    off = offset_of(k, a.geom);
                }
                int64_t x = static_cast<int64_t>(oc.y) * a.geom.stride.x + off.x - a.geom.padding.x;
                int64_t y = static_cast<int64_t>(oc.z) * a.geom.stride.y + off.y - a.geom.padding.y;
                int64_t z = static_cast<int64_t>(oc.w) * a.geom.stride.z + off.z - a.geom.padding.z;
                uint64_t key;
                if (pack_key(oc.x, x, y, z, &key)) found = a.table.find(key);
            }
            if (row_ok && k < K) a.out_in_map[row * K + k] = found;
            const uint64_t hits = ballot(found >= 0);
            const uint64_t mine = kLanes == 64 ? hits : ((hits >> (sub * kLanes)) & 0xffffffffull);
            degree += __popcll(mine);
            if (row_ok && k_lane == 0) {
                const int w0 = k0 / 32;
                a.row_masks[row * a.words + w0] = static_cast<int32_t>(static_cast<uint32_t>(mine));
                if (kLanes == 64 && w0 + 1 < a.words) {
                    a.row_masks[row * a.words + w0 + 1] = static_cast<int32_t>(static_cast<uint32_t>(mine >> 32));
                }
            }
        }
        if (row_ok && k_lane == 0 && a.degrees != nullptr) a.degrees[row] = degree;
    }
}

// Edge emission in (out_row, kernel) order from out_in_map and row_offsets.
template <int kLanes>
__global__ void __launch_bounds__(kThreads)
emit_edges(const int32_t* __restrict__ out_in_map, int out_capacity, int K,
           const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ counts,
           int32_t* __restrict__ in_rows, int32_t* __restrict__ out_rows,
           int32_t* __restrict__ kernel_ids) {
    constexpr int kRowsPerWave = kWave / kLanes;
    const int lane = lane_id();
    const int sub = lane / kLanes;
    const int k_lane = lane % kLanes;
    const int n_out = min(counts[1], out_capacity);
    const long long waves = static_cast<long long>(gridDim.x) * (kThreads / kWave);
    const long long wave_id = static_cast<long long>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
    for (long long base = wave_id * kRowsPerWave; base < n_out; base += waves * kRowsPerWave) {
        const long long row = base + sub;
        const bool row_ok = row < n_out;
        int cursor = row_ok ? row_offsets[row] : 0;
        for (int k0 = 0; k0 < K; k0 += kLanes) {
            const int k = k0 + k_lane;
            const int in = (row_ok && k < K) ? out_in_map[row * K + k] : -1;
            const uint64_t hits = ballot(in >= 0);
            const uint64_t mine = kLanes == 64 ? hits : ((hits >> (sub * kLanes)) & 0xffffffffull);
            if (in >= 0) {
                const int rank = __popcll(mine & ((1ull << k_lane) - 1ull));
                const int e = cursor + rank;
                in_rows[e] = in;
                out_rows[e] = static_cast<int32_t>(row);
                kernel_ids[e] = k;
            }
            cursor += __popcll(mine);
        }
    }
}

// ------------------------------------------------- kernel-id CSR view ----
//
// Edge ids are partitioned by kernel id, stable in edge order.  The edge
// array is cut into 1024-edge segments, one wave each: pass 1 counts per
// (kernel, segment); the counts are scanned kernel-major; pass 2 replays the
// segment in order and places every edge at its kernel's running cursor.

constexpr int kSegment = 1024;

__global__ void __launch_bounds__(kWave)
kernel_group_count(const int32_t* __restrict__ kernel_ids, const int32_t* __restrict__ counts,
                   int edge_capacity, int K, int segments, int32_t* __restrict__ seg_counts) {
    extern __shared__ int lds_counts[];
    const int seg = blockIdx.x;
    for (int k = threadIdx.x; k < K; k += kWave) lds_counts[k] = 0;
    __syncthreads();
    const int E = min(counts[0], edge_capacity);
    const int begin = seg * kSegment;
    for (int i = threadIdx.x; i < kSegment; i += kWave) {
        const int e = begin + i;
        if (e < E) {
            const int k = kernel_ids[e];
            if (k >= 0 && k < K) atomicAdd(&lds_counts[k], 1);
        }
    }
    __syncthreads();
    for (int k = threadIdx.x; k < K; k += kWave) seg_counts[static_cast<long long>(k) * segments + seg] = lds_counts[k];
}

__global__ void __launch_bounds__(kWave)
kernel_group_scatter(const int32_t* __restrict__ kernel_ids, const int32_t* __restrict__ counts,
                     int edge_capacity, int K, int segments,
                     const int32_t* __restrict__ seg_offsets, int32_t* __restrict__ edge_ids) {
    extern __shared__ int lds_cursor[];
    const int seg = blockIdx.x;
    for (int k = threadIdx.x; k < K; k += kWave) lds_cursor[k] = seg_offsets[static_cast<long long>(k) * segments + seg];
    __syncthreads();
    const int E = min(counts[0], edge_capacity);
    const int begin = seg * kSegment;
    const int lane = lane_id();
    for (int c = 0; c < kSegment; c += kWave) {
        const int e = begin + c + lane;
        int k = (e < E) ? kernel_ids[e] : -1;
        if (k >= K) k = -1;
        bool pending = k >= 0;
        // Peel one kernel id per iteration: all lanes holding it get their
        // rank among themselves, then the cursor advances.
        while (true) {
            const uint64_t todo = ballot(pending);
            if (todo == 0) break;
            const int leader = __ffsll(static_cast<long long>(todo)) - 1;
            const int k0 = __shfl(k, leader, kWave);
            const uint64_t same = ballot(pending && k == k0);
            const int base = lds_cursor[k0];
            if (pending && k == k0) {
                edge_ids[base + lanes_below(same)] = e;
                pending = false;
            }
            __syncthreads();
            if (lane == leader) lds_cursor[k0] = base + __popcll(same);
            __syncthreads();
        }
    }
}

__global__ void kernel_group_offsets(const int32_t* __restrict__ seg_offsets, int K, int segments,
                                     const int32_t* __restrict__ counts, int edge_capacity,
                                     int32_t* __restrict__ row_offsets) {
    const int E = min(counts[0], edge_capacity);
    for (int k = threadIdx.x; k <= K; k += blockDim.x) {
        row_offsets[k] = k < K ? seg_offsets[static_cast<long long>(k) * segments] : E;
    }
}

// --------------------------------------------------- input-row CSR view --
//
// Group sizes are bounded by the kernel volume (an input row feeds an output
// row at most once per offset), so edges are placed with atomics and each
// group is then sorted by edge id, which restores the stable order.

__global__ void __launch_bounds__(kThreads)
count_groups(const int32_t* __restrict__ group_ids, const int32_t* __restrict__ counts,
             int edge_capacity, int groups, int32_t* __restrict__ group_counts) {
    const int E = min(counts[0], edge_capacity);
    for (int e = blockIdx.x * kThreads + threadIdx.x; e < E; e += gridDim.x * kThreads) {
        const int g = group_ids[e];
        if (g >= 0 && g < groups) atomicAdd(group_counts + g, 1);
    }
}

__global__ void __launch_bounds__(kThreads)
place_groups(const int32_t* __restrict__ group_ids, const int32_t* __restrict__ counts,
             int edge_capacity, int groups, int32_t* __restrict__ cursors,
             int32_t* __restrict__ edge_ids) {
    const int E = min(counts[0], edge_capacity);
    for (int e = blockIdx.x * kThreads + threadIdx.x; e < E; e += gridDim.x * kThreads) {
        const int g = group_ids[e];
        if (g >= 0 && g < groups) edge_ids[atomicAdd(cursors + g, 1)] = e;
    }
}

__global__ void __launch_bounds__(kThreads)
sort_groups(const int32_t* __restrict__ offsets, int groups, int32_t* __restrict__ edge_ids) {
    for (int g = blockIdx.x * kThreads + threadIdx.x; g < groups; g += gridDim.x * kThreads) {
        const int b = offsets[g];
        const int e = offsets[g + 1];
        for (int i = b + 1; i < e; ++i) {
            const int v = edge_ids[i];
            int j = i - 1;
            while (j >= b && edge_ids[j] > v) {
                edge_ids[j + 1] = edge_ids[j];
                --j;
            }
            edge_ids[j + 1] = v;
        }
    }
}

__global__ void copy_i32(const int32_t* __restrict__ src, int32_t* __restrict__ dst, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) dst[i] = src[i];
}

// ------------------------------------------------------------- helpers ----

int table_capacity(int rows) {
    int cap = 1;
    int want = std::max(rows * 2, 1);
    while (cap < want) cap <<= 1;
    return cap;
}

size_t table_bytes(int rows) {
    const size_t cap = static_cast<size_t>(table_capacity(rows));
    return aligned_bytes(cap * sizeof(uint64_t)) + aligned_bytes(cap * sizeof(int32_t));
}

int make_table(int rows, Workspace& ws, CoordTable* table) {
    const int cap = table_capacity(rows);
    table->keys = ws.take<uint64_t>(cap);
    table->rows = ws.take<int32_t>(cap);
    table->mask = static_cast<uint32_t>(cap - 1);
    if (table->keys == nullptr || table->rows == nullptr) {
        set_error("relation workspace too small for the coordinate table");
        return LATTICE_ERROR_INVALID_ARGUMENT;
    }
    return LATTICE_OK;
}

int build_table(const int32_t* coords, int rows, const int32_t* active_rows, Int3 cell,
                int32_t* status, Workspace& ws, hipStream_t stream, CoordTable* table) {
    int rc = make_table(rows, ws, table);
    if (rc != LATTICE_OK) return rc;
    const int cap = static_cast<int>(table->mask) + 1;
    clear_table<<<grid_for(cap, kThreads, 4096), kThreads, 0, stream>>>(table->keys, table->rows, cap);
    LATTICE_LAUNCH_CHECK();
    if (rows > 0) {
        insert_rows<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
            *table, coords, rows, active_rows, cell, status);
        LATTICE_LAUNCH_CHECK();
    }
    return LATTICE_OK;
}

size_t group_view_bytes(int edge_capacity, int in_capacity, int K) {
    const long long segments = std::max(1, (edge_capacity + kSegment - 1) / kSegment);
    size_t bytes = aligned_bytes(static_cast<size_t>(segments) * K * sizeof(int32_t));
    bytes += scan_workspace_bytes(segments * K);
    bytes += aligned_bytes(static_cast<size_t>(in_capacity + 1) * sizeof(int32_t));
    bytes += scan_workspace_bytes(in_capacity + 1);
    return bytes;
}

int build_group_views(const lattice_relation_outputs* out, int edge_capacity, int in_capacity,
                      int K, Workspace& ws, hipStream_t stream) {
    // kernel-id CSR
    const int segments = std::max(1, (edge_capacity + kSegment - 1) / kSegment);
    int32_t* seg = ws.take<int32_t>(static_cast<size_t>(segments) * K);
    LATTICE_REQUIRE(seg != nullptr, "relation workspace too small for the kernel view");
    const size_t lds = static_cast<size_t>(K) * sizeof(int);
    kernel_group_count<<<segments, kWave, lds, stream>>>(out->kernel_ids, out->counts, edge_capacity, K,
                                                         segments, seg);
    LATTICE_LAUNCH_CHECK();
    int rc = exclusive_scan(seg, seg, static_cast<long long>(segments) * K, nullptr, ws, stream);
    if (rc != LATTICE_OK) return rc;
    kernel_group_scatter<<<segments, kWave, lds, stream>>>(out->kernel_ids, out->counts, edge_capacity, K,
                                                           segments, seg, out->kernel_edge_ids);
    LATTICE_LAUNCH_CHECK();
    kernel_group_offsets<<<1, 256, 0, stream>>>(seg, K, segments, out->counts, edge_capacity,
                                               out->kernel_row_offsets);
    LATTICE_LAUNCH_CHECK();

    // input-row CSR
    rc = fill_i32(out->in_row_offsets, in_capacity + 1, 0, stream);
    if (rc != LATTICE_OK) return rc;
    const unsigned eg = grid_for(edge_capacity, kThreads, 8192);
    count_groups<<<eg, kThreads, 0, stream>>>(out->in_rows, out->counts, edge_capacity, in_capacity,
                                              out->in_row_offsets);
    LATTICE_LAUNCH_CHECK();
    rc = exclusive_scan(out->in_row_offsets, out->in_row_offsets, in_capacity + 1, nullptr, ws, stream);
    if (rc != LATTICE_OK) return rc;
    int32_t* cursors = ws.take<int32_t>(static_cast<size_t>(in_capacity) + 1);
    LATTICE_REQUIRE(cursors != nullptr, "relation workspace too small for the input view");
    copy_i32<<<grid_for(in_capacity + 1, kThreads, 4096), kThreads, 0, stream>>>(out->in_row_offsets, cursors,
                                                                                 in_capacity + 1);
    LATTICE_LAUNCH_CHECK();
    place_groups<<<eg, kThreads, 0, stream>>>(out->in_rows, out->counts, edge_capacity, in_capacity, cursors,
                                              out->in_edge_ids);
    LATTICE_LAUNCH_CHECK();
    sort_groups<<<grid_for(in_capacity, kThreads, 4096), kThreads, 0, stream>>>(out->in_row_offsets,
                                                                                 in_capacity, out->in_edge_ids);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

int validate_geometry(const int* size, const int* stride, const int* padding, const int* dilation) {
    for (int a = 0; a < 3; ++a) {
        LATTICE_REQUIRE(size[a] > 0, "kernel_size values must be positive.");
        LATTICE_REQUIRE(stride[a] > 0, "stride values must be positive.");
        LATTICE_REQUIRE(padding[a] >= 0, "padding values must be non-negative.");
        LATTICE_REQUIRE(dilation[a] > 0, "dilation values must be positive.");
    }
    return LATTICE_OK;
}

KernelGeometry make_geometry(const int* size, const int* stride, const int* padding, const int* dilation) {
    KernelGeometry g;
    g.size = {size[0], size[1], size[2]};
    g.stride = {stride[0], stride[1], stride[2]};
    g.padding = {padding[0], padding[1], padding[2]};
    g.dilation = {dilation[0], dilation[1], dilation[2]};
    g.volume = size[0] * size[1] * size[2];
    return g;
}

int launch_query(const QueryArgs& a, hipStream_t stream) {
    if (a.out_capacity <= 0) return LATTICE_OK;
    if (a.geom.volume <= 32) {
        const long long waves = (a.out_capacity + 1) / 2;
        query_map<32><<<grid_for(waves, kThreads / kWave, 1u << 16), kThreads, 0, stream>>>(a);
    } else {
        query_map<64><<<grid_for(a.out_capacity, kThreads / kWave, 1u << 16), kThreads, 0, stream>>>(a);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

int launch_emit(const int32_t* map, int out_capacity, int K, const lattice_relation_outputs* out,
                hipStream_t stream) {
    if (out_capacity <= 0) return LATTICE_OK;
    if (K <= 32) {
        const long long waves = (out_capacity + 1) / 2;
        emit_edges<32><<<grid_for(waves, kThreads / kWave, 1u << 16), kThreads, 0, stream>>>(
            map, out_capacity, K, out->row_offsets, out->counts, out->in_rows, out->out_rows, out->kernel_ids);
    } else {
        emit_edges<64><<<grid_for(out_capacity, kThreads / kWave, 1u << 16), kThreads, 0, stream>>>(
            map, out_capacity, K, out->row_offsets, out->counts, out->in_rows, out->out_rows, out->kernel_ids);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

// Common tail: query -> degrees -> scan -> emit -> views.
int finish_relation(QueryArgs q, int in_capacity, const lattice_relation_outputs* out, Workspace& ws,
                    hipStream_t stream) {
    const int K = q.geom.volume;
    const int out_capacity = q.out_capacity;
    q.degrees = out->row_offsets;  // degrees land in row_offsets, then scan in place
    int rc = launch_query(q, stream);
    if (rc != LATTICE_OK) return rc;
    rc = fill_i32(out->row_offsets + out_capacity, 1, 0, stream);
    if (rc != LATTICE_OK) return rc;
    rc = exclusive_scan(out->row_offsets, out->row_offsets, static_cast<long long>(out_capacity) + 1,
                        out->counts, ws, stream);
    if (rc != LATTICE_OK) return rc;
    rc = launch_emit(q.out_in_map, out_capacity, K, out, stream);
    if (rc != LATTICE_OK) return rc;
    return build_group_views(out, out_capacity * K, in_capacity, K, ws, stream);
}

int check_outputs(const lattice_relation_outputs* out, bool need_coords, long long out_capacity, int K) {
    LATTICE_REQUIRE(out != nullptr, "relation outputs are required.");
    LATTICE_REQUIRE(out->row_offsets && out->counts && out->in_row_offsets && out->kernel_row_offsets && out->status,
                    "relation output pointers must be non-null.");
    if (out_capacity > 0) {
        LATTICE_REQUIRE(out->in_rows && out->out_rows && out->kernel_ids && out->in_edge_ids &&
                            out->kernel_edge_ids && out->out_in_map && out->row_masks,
                        "relation output pointers must be non-null.");
        LATTICE_REQUIRE(!need_coords || out->out_coords != nullptr, "out_coords must be non-null.");
    }
    (void)K;
    return LATTICE_OK;
}

}  // namespace

size_t forward_relation_bytes(int rows, int K) {
    size_t bytes = 2 * table_bytes(rows);                                  // coords + cells
    bytes += 2 * aligned_bytes(static_cast<size_t>(rows) * sizeof(int32_t)); // flags + positions
    bytes += scan_workspace_bytes(rows);
    bytes += scan_workspace_bytes(static_cast<long long>(rows) + 1);
    bytes += group_view_bytes(rows * K, rows, K);
    return bytes + 4096;
}

}  // namespace lattice

using namespace lattice;

extern "C" int lattice_hip_coord_hash_capacity(int rows) { return table_capacity(rows); }

extern "C" int lattice_hip_kernel_offsets(const int kernel_size[3], const int dilation[3], int32_t* out) {
    for (int a = 0; a < 3; ++a) {
        if (kernel_size[a] <= 0 || dilation[a] <= 0) return -1;
    }
    int k = 0;
    for (int x = 0; x < kernel_size[0]; ++x)
        for (int y = 0; y < kernel_size[1]; ++y)
            for (int z = 0; z < kernel_size[2]; ++z) {
                if (out != nullptr) {
                    int v[3] = {x, y, z};
                    for (int a = 0; a < 3; ++a) {
                        if (kernel_size[a] & 1) v[a] -= kernel_size[a] / 2;
                        out[3 * k + a] = v[a] * dilation[a];
                    }
                }
                ++k;
            }
    return k;
}

extern "C" size_t lattice_hip_kernel_relation_workspace_bytes(int rows, int kernel_count) {
    return forward_relation_bytes(std::max(rows, 0), std::max(kernel_count, 1));
}

extern "C" size_t lattice_hip_target_relation_workspace_bytes(int rows, int target_rows, int kernel_count) {
    size_t bytes = table_bytes(std::max(rows, 0));
    bytes += scan_workspace_bytes(static_cast<long long>(std::max(target_rows, 0)) + 1);
    bytes += group_view_bytes(std::max(target_rows, 0) * std::max(kernel_count, 1), std::max(rows, 0),
                              std::max(kernel_count, 1));
    return bytes + 4096;
}

extern "C" int lattice_hip_build_kernel_relation(const int32_t* coords, int rows, const int32_t* active_rows,
                                                 const int kernel_size[3], const int stride[3],
                                                 const int padding[3], const int dilation[3],
                                                 const lattice_relation_outputs* out, void* workspace,
                                                 size_t workspace_bytes, void* stream_ptr) {
    int rc = validate_geometry(kernel_size, stride, padding, dilation);
    if (rc != LATTICE_OK) return rc;
    rc = check_outputs(out, true, rows, kernel_size[0] * kernel_size[1] * kernel_size[2]);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(rows >= 0, "coords must have shape (N, 4).");
    LATTICE_REQUIRE(rows == 0 || coords != nullptr, "coords must be non-null.");
    LATTICE_REQUIRE(active_rows != nullptr, "active_rows must be non-null.");
    const KernelGeometry geom = make_geometry(kernel_size, stride, padding, dilation);
    const int K = geom.volume;
    LATTICE_REQUIRE(static_cast<long long>(rows) * K < INT_MAX, "relation edge capacity exceeds int32.");
    LATTICE_REQUIRE(workspace_bytes >= forward_relation_bytes(rows, K), "relation workspace too small.");
    hipStream_t stream = as_stream(stream_ptr);
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};

    rc = fill_i32(out->status, 1, 0, stream);
    if (rc != LATTICE_OK) return rc;
    CoordTable table;
    rc = build_table(coords, rows, active_rows, Int3{1, 1, 1}, out->status, ws, stream, &table);
    if (rc != LATTICE_OK) return rc;

    const bool identity = stride[0] == 1 && stride[1] == 1 && stride[2] == 1 && padding[0] == 0 &&
                          padding[1] == 0 && padding[2] == 0;
    QueryArgs q{};
    q.out_capacity = rows;
    q.offsets = nullptr;
    q.geom = geom;
    q.words = (K + 31) / 32;
    q.table = table;
    q.out_in_map = out->out_in_map;
    q.row_masks = out->row_masks;
    if (identity) {
        if (rows > 0) {
            copy_active_coords<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(coords, rows, active_rows,
                                                                                       out->out_coords);
            LATTICE_LAUNCH_CHECK();
        }
        set_out_count<<<1, 64, 0, stream>>>(active_rows, rows, out->counts);
        LATTICE_LAUNCH_CHECK();
        q.out_coords = coords;
        q.out_active = out->counts + 1;
    } else {
        const Int3 cell{stride[0], stride[1], stride[2]};
        CoordTable cells;
        rc = build_table(coords, rows, active_rows, cell, out->status, ws, stream, &cells);
        if (rc != LATTICE_OK) return rc;
        int32_t* flags = ws.take<int32_t>(std::max(rows, 1));
        int32_t* positions = ws.take<int32_t>(std::max(rows, 1));
        LATTICE_REQUIRE(flags != nullptr && positions != nullptr, "relation workspace too small.");
        if (rows > 0) {
            flag_cell_representatives<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
                cells, coords, rows, active_rows, cell, flags);
            LATTICE_LAUNCH_CHECK();
        }
        rc = exclusive_scan(flags, positions, rows, out->counts + 1, ws, stream);
        if (rc != LATTICE_OK) return rc;
        if (rows > 0) {
            scatter_cells<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
                coords, rows, flags, positions, out->counts, cell, out->out_coords);
            LATTICE_LAUNCH_CHECK();
        }
        q.out_coords = out->out_coords;
        q.out_active = out->counts + 1;
    }
    return finish_relation(q, rows, out, ws, stream);
}

extern "C" int lattice_hip_build_target_kernel_relation(
    const int32_t* coords, int rows, const int32_t* active_rows, const int32_t* target_coords, int target_rows,
    const int32_t* target_active_rows, const int kernel_size[3], const int stride[3], const int padding[3],
    const int dilation[3], const lattice_relation_outputs* out, void* workspace, size_t workspace_bytes,
    void* stream_ptr) {
    int rc = validate_geometry(kernel_size, stride, padding, dilation);
    if (rc != LATTICE_OK) return rc;
    rc = check_outputs(out, false, target_rows, kernel_size[0] * kernel_size[1] * kernel_size[2]);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(rows >= 0 && target_rows >= 0, "coords must have shape (N, 4).");
    LATTICE_REQUIRE(active_rows != nullptr && target_active_rows != nullptr, "active_rows must be non-null.");
    const KernelGeometry geom = make_geometry(kernel_size, stride, padding, dilation);
    const int K = geom.volume;
    LATTICE_REQUIRE(static_cast<long long>(target_rows) * K < INT_MAX, "relation edge capacity exceeds int32.");
    LATTICE_REQUIRE(workspace_bytes >= lattice_hip_target_relation_workspace_bytes(rows, target_rows, K),
                    "relation workspace too small.");
    hipStream_t stream = as_stream(stream_ptr);
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    rc = fill_i32(out->status, 1, 0, stream);
    if (rc != LATTICE_OK) return rc;
    CoordTable table;
    rc = build_table(coords, rows, active_rows, Int3{1, 1, 1}, out->status, ws, stream, &table);
    if (rc != LATTICE_OK) return rc;
    set_out_count<<<1, 64, 0, stream>>>(target_active_rows, target_rows, out->counts);
    LATTICE_LAUNCH_CHECK();
    QueryArgs q{};
    q.out_coords = target_coords;
    q.out_capacity = target_rows;
    q.out_active = out->counts + 1;
    q.offsets = nullptr;
    q.geom = geom;
    q.words = (K + 31) / 32;
    q.table = table;
    q.out_in_map = out->out_in_map;
    q.row_masks = out->row_masks;
    return finish_relation(q, rows, out, ws, stream);
}

extern "C" size_t lattice_hip_implicit_gemm_view_workspace_bytes(int source_rows) {
    return table_bytes(std::max(source_rows, 0)) + 4096;
}

extern "C" int lattice_hip_build_relation_implicit_gemm_view(
    const int32_t* source_coords, int source_rows, const int32_t* source_active_rows,
    const int32_t* output_coords, int output_rows, const int32_t* output_active_rows, const int32_t* offsets,
    int kernel_count, const int stride[3], const int padding[3], int32_t* out_in_map, int32_t* row_masks,
    int32_t* status, void* workspace, size_t workspace_bytes, void* stream_ptr) {
    LATTICE_REQUIRE(kernel_count > 0, "offsets must have shape (K, 3) with K > 0.");
    LATTICE_REQUIRE(source_rows >= 0 && output_rows >= 0, "coords must have shape (N, 4).");
    LATTICE_REQUIRE(offsets && out_in_map && row_masks && status && source_active_rows && output_active_rows,
                    "implicit GEMM view pointers must be non-null.");
    for (int a = 0; a < 3; ++a) {
        LATTICE_REQUIRE(stride[a] > 0, "stride values must be positive.");
        LATTICE_REQUIRE(padding[a] >= 0, "padding values must be non-negative.");
    }
    LATTICE_REQUIRE(workspace_bytes >= lattice_hip_implicit_gemm_view_workspace_bytes(source_rows),
                    "implicit GEMM view workspace too small.");
    hipStream_t stream = as_stream(stream_ptr);
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    int rc = fill_i32(status, 1, 0, stream);
    if (rc != LATTICE_OK) return rc;
    CoordTable table;
    rc = build_table(source_coords, source_rows, source_active_rows, Int3{1, 1, 1}, status, ws, stream, &table);
    if (rc != LATTICE_OK) return rc;
    QueryArgs q{};
    q.out_coords = output_coords;
    q.out_capacity = output_rows;
    q.out_active = output_active_rows;
    q.offsets = offsets;
    q.geom.volume = kernel_count;
    q.geom.stride = {stride[0], stride[1], stride[2]};
    q.geom.padding = {padding[0], padding[1], padding[2]};
    q.geom.size = {kernel_count, 1, 1};
    q.geom.dilation = {1, 1, 1};
    q.words = (kernel_count + 31) / 32;
    q.table = table;
    q.out_in_map = out_in_map;
    q.row_masks = row_masks;
    q.degrees = nullptr;
    return launch_query(q, stream);
}

// ------------------------------------------------------------ sorted view --

namespace lattice {
namespace {

__global__ void __launch_bounds__(kThreads)
first_word_and_iota(const int32_t* __restrict__ row_masks, int rows, int words, int32_t* __restrict__ keys,
                    int32_t* __restrict__ ids) {
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        keys[i] = row_masks[static_cast<long long>(i) * words];
        ids[i] = i;
    }
}

__global__ void __launch_bounds__(kThreads)
gather_sorted(const int32_t* __restrict__ out_in_map, int rows, int K, const int32_t* __restrict__ order,
              int32_t* __restrict__ sorted_map, int32_t* __restrict__ kv_map) {
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        const long long src = static_cast<long long>(order[i]) * K;
        for (int k = 0; k < K; ++k) {
            const int v = out_in_map[src + k];
            sorted_map[static_cast<long long>(i) * K + k] = v;
            kv_map[static_cast<long long>(k) * rows + i] = v;
        }
    }
}

__global__ void __launch_bounds__(kThreads)
tile_quarter_masks(const int32_t* __restrict__ sorted_keys, int rows, int tiles, int32_t* __restrict__ tile_masks) {
    for (int w = blockIdx.x * kThreads + threadIdx.x; w < tiles * 4; w += gridDim.x * kThreads) {
        int acc = 0;
        const int start = w * 16;
        for (int r = start; r < start + 16 && r < rows; ++r) acc |= sorted_keys[r];
        tile_masks[w] = acc;
    }
}

size_t radix_temp_bytes(int rows) {
    size_t temp = 0;
    (void)hipcub::DeviceRadixSort::SortPairs(nullptr, temp, static_cast<const int32_t*>(nullptr),
                                       static_cast<int32_t*>(nullptr), static_cast<const int32_t*>(nullptr),
                                       static_cast<int32_t*>(nullptr), std::max(rows, 1));
    return temp;
}

}  // namespace
}  // namespace lattice

extern "C" size_t lattice_hip_sorted_view_workspace_bytes(int rows) {
    const size_t n = static_cast<size_t>(std::max(rows, 1));
    return 3 * aligned_bytes(n * sizeof(int32_t)) + aligned_bytes(radix_temp_bytes(rows)) + 4096;
}

extern "C" int lattice_hip_build_sorted_implicit_gemm_view(const int32_t* out_in_map, const int32_t* row_masks,
                                                           int rows, int kernel_count, int32_t* reorder_rows,
                                                           int32_t* sorted_out_in_map,
                                                           int32_t* sorted_kv_out_in_map, int32_t* tile_masks,
                                                           void* workspace, size_t workspace_bytes,
                                                           void* stream_ptr) {
    LATTICE_REQUIRE(kernel_count > 0 && kernel_count <= 32, "sorted implicit GEMM view currently supports K <= 32.");
    LATTICE_REQUIRE(rows >= 0, "out_in_map must have shape (N_out, K).");
    LATTICE_REQUIRE(workspace_bytes >= lattice_hip_sorted_view_workspace_bytes(rows),
                    "sorted view workspace too small.");
    hipStream_t stream = as_stream(stream_ptr);
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    const int tiles = (rows + 63) / 64;
    if (rows == 0) return LATTICE_OK;
    int32_t* keys = ws.take<int32_t>(rows);
    int32_t* sorted_keys = ws.take<int32_t>(rows);
    int32_t* ids = ws.take<int32_t>(rows);
    size_t temp_bytes = radix_temp_bytes(rows);
    void* temp = ws.take<char>(temp_bytes);
    LATTICE_REQUIRE(keys && sorted_keys && ids && temp, "sorted view workspace too small.");
    const int words = 1;
    first_word_and_iota<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(row_masks, rows, words, keys, ids);
    LATTICE_LAUNCH_CHECK();
    LATTICE_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys, sorted_keys, ids, reorder_rows,
                                                       rows, 0, 32, stream));
    gather_sorted<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(out_in_map, rows, kernel_count,
                                                                          reorder_rows, sorted_out_in_map,
                                                                          sorted_kv_out_in_map);
    LATTICE_LAUNCH_CHECK();
    tile_quarter_masks<<<grid_for(tiles * 4, kThreads, 4096), kThreads, 0, stream>>>(sorted_keys, rows, tiles,
                                                                                    tile_masks);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}
