// Point -> voxel quantization and the point <-> voxel feature maps for gfx950
// (mlx_lattice/core/coords/quantization.py; CPU routines
// native/features/coordinates/cpu/quantization_detail.h:66-391).
//
//  * sparse_quantize: voxel = (batch, floor((p - origin) / voxel_size)) per
//    point in binary32 with one rounding per operation.  The voxels are
//    deduplicated in first-seen point order exactly as the forward
//    relation's downsample is: a coordinate table keeps the minimum point
//    row per voxel, a flag + scan places the representatives, every active
//    point looks its voxel row up (inverse_rows) and counts it.
//  * voxelize_features: one lane per (voxel, channel) sums its points in
//    point order over a voxel -> points CSR (a stable grouping of the
//    inverse rows), so the sum is deterministic and adds in the CPU
//    routine's order.  Its gradient is a gather, one lane per (point,
//    channel).
//  * point_voxel_map: a coordinate table over the voxel coordinates (first
//    row per coordinate); each point probes its nearest voxel or the eight
//    corners of its cell, with trilinear weights (wx * wy) * wz.
//  * interpolate_point_features: one lane per (point, channel) adds its
//    eight corners in order; the gradient sums, per (voxel, channel), the
//    (point, corner) entries that hit the voxel, in (point, corner) order,
//    over a second stable grouping.
// Floating-point contraction is off for this file: every product and sum
// rounds once, in the CPU routine's order, so no multiply-add is fused.

#include <algorithm>
#include <climits>

#include "lattice_common.h"
#include "scan.h"

#pragma clang fp contract(off)

namespace lattice {
namespace {

constexpr int kThreads = 256;

struct VoxelGrid {
    float size[3];
    float origin[3];
};

__device__ inline float grid_position(float p, int axis, const VoxelGrid& g) {
    return ((p - g.origin[axis]) / g.size[axis]);
}

// floor of a float as int64; false outside +-2^40 (and for NaN), where no
// int32 voxel coordinate can match.
__device__ inline bool floor_int(float v, int64_t* out) {
    const float f = floorf(v);
    if (!(fabsf(f) < 1099511627776.0f)) return false;
    *out = static_cast<int64_t>(f);
    return true;
}

// floor of a float as int64 (static_cast<int64_t>(std::floor(v)), exact
// below 2^63 in magnitude).  The reference's conversion is undefined beyond
// that and for NaN; here they saturate, NaN to INT64_MIN.
__device__ inline int64_t floor_i64(float v) {
    const float f = floorf(v);
    if (!(f >= -9223372036854775808.0f)) return INT64_MIN;
    if (f >= 9223372036854775808.0f) return INT64_MAX;
    return static_cast<int64_t>(f);
}

// The voxel of a point (batch, floor((p - origin) / voxel_size)): the key
// source of the voxel table.
struct PointSource {
    const float* points;
    const int32_t* batches;
    VoxelGrid g;
    __device__ inline FullKey key_of(int32_t p) const {
        const float* q = points + 3ll * p;
        return {batches[p], floor_i64(grid_position(q[0], 0, g)), floor_i64(grid_position(q[1], 1, g)),
                floor_i64(grid_position(q[2], 2, g))};
    }
};

int table_capacity_for(int rows) {
    int cap = 1;
    const long long want = std::max(2ll * rows, 1ll);
    while (cap < want) cap <<= 1;
    return cap;
}

size_t table_bytes_for(int rows) {
    const size_t cap = static_cast<size_t>(table_capacity_for(rows));
    return aligned_bytes(cap * sizeof(CoordSlot));
}

// Clears the table, zeroes `zero[0..zero_n)` and the status word.
__global__ void __launch_bounds__(kThreads)
clear_quant(CoordSlot* slots, int capacity, int32_t* zero, int zero_n, int32_t* status) {
    const int n = max(capacity, zero_n);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
        if (i < capacity) reinterpret_cast<int4*>(slots)[i] = empty_coord_slot();
        if (i < zero_n) zero[i] = 0;
        if (i == 0 && status != nullptr) status[0] = 0;
    }
}

// ------------------------------------------------------ sparse_quantize --

// Inserts the voxel of every active point with the point row; slots[p] =
// the voxel's table slot (-1 for inactive points).
__global__ void __launch_bounds__(kThreads)
insert_points(CoordTable table, PointSource src, int rows, const int32_t* __restrict__ active_rows,
              int32_t* __restrict__ slots) {
    const int active = min(max(*active_rows, 0), rows);
    for (int p = blockIdx.x * kThreads + threadIdx.x; p < rows; p += gridDim.x * kThreads) {
        int32_t slot = -1;
        if (p < active) {
            const FullKey v = src.key_of(p);
            slot = static_cast<int32_t>(table.insert(table_key(v.b, v.x, v.y, v.z), p, src));
        }
        slots[p] = slot;
    }
}

__global__ void __launch_bounds__(kThreads)
flag_points(CoordTable table, const int32_t* __restrict__ slots, int rows, int32_t* __restrict__ flags) {
    for (int p = blockIdx.x * kThreads + threadIdx.x; p < rows; p += gridDim.x * kThreads) {
        const int32_t s = slots[p];
        flags[p] = (s >= 0 && table.slots[s].row == p) ? 1 : 0;
    }
}

// Output voxel coordinates are written as int32 (write_coords); an axis
// value outside int32 keeps its low 32 bits.
__global__ void __launch_bounds__(kThreads)
place_points(CoordTable table, PointSource src, const int32_t* __restrict__ slots, int rows,
             const int32_t* __restrict__ flags, const int32_t* __restrict__ positions,
             const int32_t* __restrict__ voxel_count, int32_t* __restrict__ coords,
             int32_t* __restrict__ inverse_rows, int32_t* __restrict__ counts) {
    const int n_vox = *voxel_count;
    int4* out = reinterpret_cast<int4*>(coords);
    for (int p = blockIdx.x * kThreads + threadIdx.x; p < rows; p += gridDim.x * kThreads) {
        const int32_t s = slots[p];
        int inv = -1;
        if (s >= 0) {
            inv = positions[table.slots[s].row];
            atomicAdd(counts + inv, 1);
            if (flags[p]) {
                const FullKey v = src.key_of(p);
                out[positions[p]] = make_int4(static_cast<int32_t>(v.b), static_cast<int32_t>(v.x),
                                              static_cast<int32_t>(v.y), static_cast<int32_t>(v.z));
            }
        }
        if (p >= n_vox) out[p] = make_int4(0, 0, 0, 0);
        inverse_rows[p] = inv;
    }
}

// ---------------------------------------------------- voxel features --

__device__ inline float mean_scale(int mode, const int32_t* counts, int v) {
    return mode == 1 ? (1.0f / static_cast<float>(max(counts[v], 1))) : 1.0f;
}

// Feature kernels run one lane per (row, V-channel chunk): V = 4 (16-byte
// loads and stores) when the channel count allows, else 1.  Each channel is
// still accumulated in the same order with the same roundings.
template <int V> struct Vec;
typedef float f32x4v_t __attribute__((ext_vector_type(4)));
// Outputs (voxel and point features, gradients) are written with
// non-temporal stores: streamed past the caches, as no later load of the
// same kernel reads them (voxelize mean over 1M points: 136 -> 94 us).
template <> struct Vec<1> {
    float v[1];
    __device__ static Vec load(const float* p) { return {{p[0]}}; }
    __device__ void store(float* p) const { __builtin_nontemporal_store(v[0], p); }
};
template <> struct Vec<4> {
    float v[4];
    __device__ static Vec load(const float* p) {
        const float4 f = *reinterpret_cast<const float4*>(p);
        return {{f.x, f.y, f.z, f.w}};
    }
    __device__ void store(float* p) const {
        __builtin_nontemporal_store(f32x4v_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4v_t*>(p));
    }
};

template <int V>
__device__ inline void add_scaled(Vec<V>& acc, const Vec<V>& x, float s) {
#pragma unroll
    for (int j = 0; j < V; ++j) acc.v[j] = acc.v[j] + x.v[j] * s;
}

template <int V>
__global__ void __launch_bounds__(kThreads)
voxelize_csr(int mode, const float* __restrict__ feats, int channels, const int32_t* __restrict__ counts,
             int voxel_rows, const int32_t* __restrict__ offsets, const int32_t* __restrict__ point_ids,
             float* __restrict__ out) {
    const int chunks = channels / V;
    const long long total = static_cast<long long>(voxel_rows) * chunks;
    for (long long t = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * kThreads) {
        const int v = static_cast<int>(t / chunks);
        const int c = static_cast<int>(t - static_cast<long long>(v) * chunks) * V;
        const float scale = mean_scale(mode, counts, v);
        Vec<V> acc{};
        const int lo = offsets[v];
        const int hi = offsets[v + 1];
        int i = lo;
        for (; i + 1 < hi; i += 2) {  // two gathers in flight
            const Vec<V> a = Vec<V>::load(feats + static_cast<long long>(point_ids[i]) * channels + c);
            const Vec<V> b = Vec<V>::load(feats + static_cast<long long>(point_ids[i + 1]) * channels + c);
            add_scaled(acc, a, scale);
            add_scaled(acc, b, scale);
        }
        if (i < hi) add_scaled(acc, Vec<V>::load(feats + static_cast<long long>(point_ids[i]) * channels + c), scale);
        acc.store(out + static_cast<long long>(v) * channels + c);
    }
}

template <int V>
__global__ void __launch_bounds__(kThreads)
voxelize_grad(int mode, const float* __restrict__ cot, int voxel_rows, int channels,
              const int32_t* __restrict__ inverse_rows, const int32_t* __restrict__ counts, int point_rows,
              const int32_t* __restrict__ point_active, float* __restrict__ grad) {
    const int active = min(max(*point_active, 0), point_rows);
    const int chunks = channels / V;
    const long long total = static_cast<long long>(point_rows) * chunks;
    for (long long t = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * kThreads) {
        const int p = static_cast<int>(t / chunks);
        const int c = static_cast<int>(t - static_cast<long long>(p) * chunks) * V;
        Vec<V> value{};
        if (p < active) {
            const int v = inverse_rows[p];
            if (v >= 0 && v < voxel_rows) {
                const float s = mean_scale(mode, counts, v);
                const Vec<V> x = Vec<V>::load(cot + static_cast<long long>(v) * channels + c);
#pragma unroll
                for (int j = 0; j < V; ++j) value.v[j] = x.v[j] * s;
            }
        }
        value.store(grad + static_cast<long long>(p) * channels + c);
    }
}

// ---------------------------------------------------- point-voxel map --

// Block-bucketed table of the voxel rows for the point-voxel map: a 2x2x2
// block of voxels per 64-byte bucket, so a point's 8 trilinear corners
// touch at most 8 lines (one when the corners share a block) and each probe
// reads its key and row from one line.
int block_capacity_for(int rows) {
    int cap = 1;
    const long long want = std::max(static_cast<long long>(rows) + rows / 2 + 1, 1ll);
    while (cap < want) cap <<= 1;
    return cap;
}

// Clears the block table (one thread per 16-byte quarter of a bucket) and
// the status word.
__global__ void __launch_bounds__(kThreads)
clear_voxel_blocks(BlockBucket* buckets, long long quarters, int32_t* status) {
    int4* q = reinterpret_cast<int4*>(buckets);
    for (long long i = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; i < quarters;
         i += static_cast<long long>(gridDim.x) * kThreads) {
        q[i] = (i & 3) == 0 ? make_int4(-1, -1, 0, 0) : make_int4(0, 0, 0, 0);
        if (i == 0) status[0] = 0;
    }
}

__global__ void __launch_bounds__(kThreads)
insert_voxel_blocks(BlockTable table, const int32_t* __restrict__ coords, int rows,
                    const int32_t* __restrict__ active_rows) {
    const int active = min(max(*active_rows, 0), rows);
    for (int v = blockIdx.x * kThreads + threadIdx.x; v < active; v += gridDim.x * kThreads) {
        const int4 c = reinterpret_cast<const int4*>(coords)[v];
        TableKey block_key;
        int octant;
        block_of(c.x, c.y, c.z, c.w, &block_key, &octant);
        table.insert(block_key, octant, v);
    }
}

__device__ inline int probe(const BlockTable& table, int b, int64_t x, int64_t y, int64_t z) {
    TableKey block_key;
    int octant;
    if (!block_of(b, x, y, z, &block_key, &octant)) return -1;
    return table.find(block_key, octant);
}

__global__ void __launch_bounds__(kThreads)
map_points(BlockTable table, const float* __restrict__ points, const int32_t* __restrict__ batches, int point_rows,
           const int32_t* __restrict__ point_active, VoxelGrid g, int linear, int32_t* __restrict__ rows_out,
           float* __restrict__ weights_out) {
    const int active = min(max(*point_active, 0), point_rows);
    for (int p = blockIdx.x * kThreads + threadIdx.x; p < point_rows; p += gridDim.x * kThreads) {
        int r[8];
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            r[i] = -1;
            w[i] = 0.0f;
        }
        if (p < active) {
            const float* q = points + 3ll * p;
            const int b = batches[p];
            float pos[3];
            for (int a = 0; a < 3; ++a) pos[a] = grid_position(q[a], a, g);
            if (!linear) {
                int64_t n[3];
                bool ok = true;
                for (int a = 0; a < 3; ++a) ok = floor_int((pos[a] + 0.5f), &n[a]) && ok;
                const int row = ok ? probe(table, b, n[0], n[1], n[2]) : -1;
                if (row >= 0) {
                    r[0] = row;
                    w[0] = 1.0f;
                }
            } else {
                int64_t lo[3];
                float frac[3];
                bool ok = true;
                for (int a = 0; a < 3; ++a) {
                    ok = floor_int(pos[a], &lo[a]) && ok;
                    frac[a] = (pos[a] - static_cast<float>(lo[a]));
                }
                const auto weight = [&](int dx, int dy, int dz) {
                    const float wx = dx == 0 ? (1.0f - frac[0]) : frac[0];
                    const float wy = dy == 0 ? (1.0f - frac[1]) : frac[1];
                    const float wz = dz == 0 ? (1.0f - frac[2]) : frac[2];
                    return ((wx * wy) * wz);
                };
                // When the cell's blocks have packed keys (batch in [0, 1022],
                // lo in [-2^18, 2^18 - 2] per axis) every corner's home bucket
                // (key word and the corner's row word) is read before any is
                // resolved, so the eight lookups overlap; a corner whose home
                // bucket holds another key continues by linear probing.
                const auto packs = [](int64_t v) { return v >= -(1 << 18) && v <= (1 << 18) - 2; };
                if (ok && b >= 0 && b <= LATTICE_MAX_BATCH && packs(lo[0]) && packs(lo[1]) && packs(lo[2])) {
                    const int x0 = static_cast<int>(lo[0]), y0 = static_cast<int>(lo[1]), z0 = static_cast<int>(lo[2]);
                    uint64_t want[8];
                    uint32_t slot[8];
                    unsigned long long seen[8];
                    int32_t raw[8];
#pragma unroll
                    for (int corner = 0; corner < 8; ++corner) {
                        const int x = x0 + (corner & 1), y = y0 + ((corner >> 1) & 1), z = z0 + ((corner >> 2) & 1);
                        pack_key(b, x >> 1, y >> 1, z >> 1, &want[corner]);
                        slot[corner] = static_cast<uint32_t>(mix64(want[corner])) & table.mask;
                        seen[corner] = table.buckets[slot[corner]].key;
                        raw[corner] = table.buckets[slot[corner]].rows[((x & 1) << 2) | ((y & 1) << 1) | (z & 1)];
                    }
#pragma unroll
                    for (int corner = 0; corner < 8; ++corner) {
                        const int dx = corner & 1, dy = (corner >> 1) & 1, dz = (corner >> 2) & 1;
                        const int oct = (((x0 + dx) & 1) << 2) | (((y0 + dy) & 1) << 1) | ((z0 + dz) & 1);
                        while (seen[corner] != want[corner] && seen[corner] != kEmptyKey) {
                            slot[corner] = (slot[corner] + 1) & table.mask;
                            seen[corner] = table.buckets[slot[corner]].key;
                            raw[corner] = table.buckets[slot[corner]].rows[oct];
                        }
                        if (seen[corner] == want[corner] && raw[corner] != 0) {
                            r[corner] = kRowBias - raw[corner];
                            w[corner] = weight(dx, dy, dz);
                        }
                    }
                } else if (ok) {
                    // Wide block keys: the table's full lookup per corner,
                    // written straight out.
#pragma unroll 1
                    for (int corner = 0; corner < 8; ++corner) {
                        const int dx = corner & 1, dy = (corner >> 1) & 1, dz = (corner >> 2) & 1;
                        const int row = probe(table, b, lo[0] + dx, lo[1] + dy, lo[2] + dz);
                        rows_out[8ll * p + corner] = row < 0 ? -1 : row;
                        weights_out[8ll * p + corner] = row < 0 ? 0.0f : weight(dx, dy, dz);
                    }
                    continue;
                }
            }
        }
        int4* ro = reinterpret_cast<int4*>(rows_out + 8ll * p);
        float4* wo = reinterpret_cast<float4*>(weights_out + 8ll * p);
        ro[0] = make_int4(r[0], r[1], r[2], r[3]);
        ro[1] = make_int4(r[4], r[5], r[6], r[7]);
        wo[0] = make_float4(w[0], w[1], w[2], w[3]);
        wo[1] = make_float4(w[4], w[5], w[6], w[7]);
    }
}

template <int V>
__global__ void __launch_bounds__(kThreads)
interpolate(const float* __restrict__ values, int voxel_rows, int channels, const int32_t* __restrict__ rows,
            const float* __restrict__ weights, int point_rows, float* __restrict__ out) {
    const int chunks = channels / V;
    const long long total = static_cast<long long>(point_rows) * chunks;
    for (long long t = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * kThreads) {
        const int p = static_cast<int>(t / chunks);
        const int c = static_cast<int>(t - static_cast<long long>(p) * chunks) * V;
        const int4* r4 = reinterpret_cast<const int4*>(rows + 8ll * p);
        const float4* w4 = reinterpret_cast<const float4*>(weights + 8ll * p);
        const int4 ra = r4[0], rb = r4[1];
        const float4 wa = w4[0], wb = w4[1];
        const int r[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
        const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
        Vec<V> x[8];
#pragma unroll
        for (int corner = 0; corner < 8; ++corner) {  // all gathers in flight
            x[corner] = (r[corner] >= 0 && r[corner] < voxel_rows)
                            ? Vec<V>::load(values + static_cast<long long>(r[corner]) * channels + c)
                            : Vec<V>{};
        }
        Vec<V> acc{};
#pragma unroll
        for (int corner = 0; corner < 8; ++corner) {
            if (r[corner] >= 0 && r[corner] < voxel_rows) add_scaled(acc, x[corner], w[corner]);
        }
        acc.store(out + static_cast<long long>(p) * channels + c);
    }
}

template <int V>
__global__ void __launch_bounds__(kThreads)
interpolate_grad(const float* __restrict__ point_grad, int channels, const float* __restrict__ weights,
                 const int32_t* __restrict__ offsets, const int32_t* __restrict__ entries, int voxel_rows,
                 float* __restrict__ out) {
    const int chunks = channels / V;
    const long long total = static_cast<long long>(voxel_rows) * chunks;
    for (long long t = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * kThreads) {
        const int v = static_cast<int>(t / chunks);
        const int c = static_cast<int>(t - static_cast<long long>(v) * chunks) * V;
        Vec<V> acc{};
        for (int i = offsets[v]; i < offsets[v + 1]; ++i) {
            const int e = entries[i];
            add_scaled(acc, Vec<V>::load(point_grad + static_cast<long long>(e >> 3) * channels + c), weights[e]);
        }
        acc.store(out + static_cast<long long>(v) * channels + c);
    }
}

// Launches kernel<4> when the channels split into 16-byte chunks, else <1>.
#define LATTICE_LAUNCH_VEC(kernel, channels, rows, stream, ...)                                             \
    do {                                                                                                    \
        if ((channels) % 4 == 0) {                                                                          \
            const long long work_ = static_cast<long long>(rows) * ((channels) / 4);                        \
            kernel<4><<<grid_for(work_, kThreads, 1u << 16), kThreads, 0, stream>>>(__VA_ARGS__);           \
        } else {                                                                                            \
            const long long work_ = static_cast<long long>(rows) * (channels);                              \
            kernel<1><<<grid_for(work_, kThreads, 1u << 16), kThreads, 0, stream>>>(__VA_ARGS__);           \
        }                                                                                                   \
    } while (0)

int check_grid(const float* size, const float* origin) {
    LATTICE_REQUIRE(size != nullptr && origin != nullptr, "voxel_size and origin must be non-null.");
    for (int a = 0; a < 3; ++a) LATTICE_REQUIRE(size[a] > 0.0f, "voxel_size values must be positive.");
    return LATTICE_OK;
}

VoxelGrid make_grid(const float* size, const float* origin) {
    VoxelGrid g;
    for (int a = 0; a < 3; ++a) {
        g.size[a] = size[a];
        g.origin[a] = origin[a];
    }
    return g;
}

}  // namespace
}  // namespace lattice

using namespace lattice;

extern "C" size_t lattice_hip_sparse_quantize_workspace_bytes(int rows) {
    const size_t n = static_cast<size_t>(std::max(rows, 1));
    return table_bytes_for(std::max(rows, 0)) + aligned_bytes(n * sizeof(int32_t)) +
           2 * aligned_bytes(n * sizeof(int32_t)) + scan_workspace_bytes(std::max(rows, 0)) + 1024;
}

extern "C" int lattice_hip_sparse_quantize(const float* points, const int32_t* batch_indices, int rows,
                                           const int32_t* active_rows, const float voxel_size[3],
                                           const float origin[3], int32_t* coords, int32_t* voxel_count,
                                           int32_t* inverse_rows, int32_t* counts, int32_t* status,
                                           void* workspace, size_t workspace_bytes, void* stream_ptr) {
    int rc = check_grid(voxel_size, origin);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(rows >= 0, "points must have shape (N, 3).");
    LATTICE_REQUIRE(active_rows && voxel_count && status && (rows == 0 || (points && batch_indices && coords &&
                                                                           inverse_rows && counts)),
                    "sparse_quantize pointers must be non-null.");
    LATTICE_REQUIRE(workspace_bytes >= lattice_hip_sparse_quantize_workspace_bytes(rows),
                    "sparse_quantize workspace too small.");
    hipStream_t stream = as_stream(stream_ptr);
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    const int cap = table_capacity_for(rows);
    CoordTable table;
    table.slots = ws.take<CoordSlot>(cap);
    table.mask = static_cast<uint32_t>(cap - 1);
    int32_t* slots = ws.take<int32_t>(std::max(rows, 1));
    int32_t* flags = ws.take<int32_t>(std::max(rows, 1));
    int32_t* positions = ws.take<int32_t>(std::max(rows, 1));
    LATTICE_REQUIRE(table.slots && slots && flags && positions, "sparse_quantize workspace too small.");
    clear_quant<<<grid_for(std::max(cap, rows), kThreads, 8192), kThreads, 0, stream>>>(table.slots, cap,
                                                                                      counts, rows, status);
    LATTICE_LAUNCH_CHECK();
    if (rows == 0) return fill_i32(voxel_count, 1, 0, stream);
    const PointSource src{points, batch_indices, make_grid(voxel_size, origin)};
    const unsigned grid = grid_for(rows, kThreads, 1u << 14);
    insert_points<<<grid, kThreads, 0, stream>>>(table, src, rows, active_rows, slots);
    LATTICE_LAUNCH_CHECK();
    flag_points<<<grid, kThreads, 0, stream>>>(table, slots, rows, flags);
    LATTICE_LAUNCH_CHECK();
    rc = exclusive_scan(flags, positions, rows, voxel_count, ws, stream);
    if (rc != LATTICE_OK) return rc;
    place_points<<<grid, kThreads, 0, stream>>>(table, src, slots, rows, flags, positions, voxel_count, coords,
                                               inverse_rows, counts);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_voxelize_features(int mode, const float* feats, int channels, const int32_t* counts,
                                             int voxel_rows, const int32_t* voxel_offsets,
                                             const int32_t* point_ids, float* out, void* stream_ptr) {
    LATTICE_REQUIRE(mode == 0 || mode == 1, "reduction must be 'sum' or 'mean'.");
    LATTICE_REQUIRE(channels > 0 && voxel_rows >= 0, "voxelize shapes must be positive.");
    if (voxel_rows == 0) return LATTICE_OK;
    LATTICE_REQUIRE(feats && counts && voxel_offsets && point_ids && out, "voxelize pointers must be non-null.");
    LATTICE_LAUNCH_VEC(voxelize_csr, channels, voxel_rows, as_stream(stream_ptr), mode, feats, channels, counts,
                       voxel_rows, voxel_offsets, point_ids, out);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_voxelize_features_grad(int mode, const float* cot, int voxel_rows, int channels,
                                                  const int32_t* inverse_rows, const int32_t* counts,
                                                  int point_rows, const int32_t* point_active, float* grad,
                                                  void* stream_ptr) {
    LATTICE_REQUIRE(mode == 0 || mode == 1, "reduction must be 'sum' or 'mean'.");
    LATTICE_REQUIRE(channels > 0 && voxel_rows >= 0 && point_rows >= 0, "voxelize shapes must be positive.");
    if (point_rows == 0) return LATTICE_OK;
    LATTICE_REQUIRE(grad && inverse_rows && point_active && (voxel_rows == 0 || (cot && counts)),
                    "voxelize gradient pointers must be non-null.");
    LATTICE_LAUNCH_VEC(voxelize_grad, channels, point_rows, as_stream(stream_ptr), mode, cot, voxel_rows, channels,
                       inverse_rows, counts, point_rows, point_active, grad);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" size_t lattice_hip_point_voxel_map_workspace_bytes(int voxel_rows) {
    return aligned_bytes(static_cast<size_t>(block_capacity_for(std::max(voxel_rows, 0))) * sizeof(BlockBucket)) +
           1024;
}

extern "C" int lattice_hip_build_point_voxel_map(const float* points, const int32_t* batch_indices, int point_rows,
                                                 const int32_t* point_active, const int32_t* voxel_coords,
                                                 int voxel_rows, const int32_t* voxel_active,
                                                 const float voxel_size[3], const float origin[3],
                                                 int interpolation, int32_t* rows_out, float* weights_out,
                                                 int32_t* status, void* workspace, size_t workspace_bytes,
                                                 void* stream_ptr) {
    int rc = check_grid(voxel_size, origin);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(interpolation == 0 || interpolation == 1, "interpolation must be 'nearest' or 'linear'.");
    LATTICE_REQUIRE(point_rows >= 0 && voxel_rows >= 0, "point and voxel rows must be non-negative.");
    LATTICE_REQUIRE(point_active && voxel_active && status &&
                        (point_rows == 0 || (points && batch_indices && rows_out && weights_out)) &&
                        (voxel_rows == 0 || voxel_coords),
                    "point-voxel map pointers must be non-null.");
    LATTICE_REQUIRE(workspace_bytes >= lattice_hip_point_voxel_map_workspace_bytes(voxel_rows),
                    "point-voxel map workspace too small.");
    hipStream_t stream = as_stream(stream_ptr);
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    const int cap = block_capacity_for(voxel_rows);
    BlockTable table;
    table.buckets = ws.take<BlockBucket>(cap);
    table.mask = static_cast<uint32_t>(cap - 1);
    table.src = BlockSource{voxel_coords};
    LATTICE_REQUIRE(table.buckets, "point-voxel map workspace too small.");
    clear_voxel_blocks<<<grid_for(4ll * cap, kThreads, 8192), kThreads, 0, stream>>>(table.buckets, 4ll * cap,
                                                                                   status);
    LATTICE_LAUNCH_CHECK();
    if (voxel_rows > 0) {
        insert_voxel_blocks<<<grid_for(voxel_rows, kThreads, 1u << 14), kThreads, 0, stream>>>(
            table, voxel_coords, voxel_rows, voxel_active);
        LATTICE_LAUNCH_CHECK();
    }
    if (point_rows == 0) return LATTICE_OK;
    map_points<<<grid_for(point_rows, kThreads, 1u << 14), kThreads, 0, stream>>>(
        table, points, batch_indices, point_rows, point_active, make_grid(voxel_size, origin), interpolation,
        rows_out, weights_out);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_interpolate_point_features(const float* values, int voxel_rows, int channels,
                                                      const int32_t* rows, const float* weights, int point_rows,
                                                      float* out, void* stream_ptr) {
    LATTICE_REQUIRE(channels > 0 && voxel_rows >= 0 && point_rows >= 0, "interpolation shapes must be positive.");
    if (point_rows == 0) return LATTICE_OK;
    LATTICE_REQUIRE(rows && weights && out && (voxel_rows == 0 || values),
                    "interpolation pointers must be non-null.");
    LATTICE_LAUNCH_VEC(interpolate, channels, point_rows, as_stream(stream_ptr), values, voxel_rows, channels, rows,
                       weights, point_rows, out);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

extern "C" int lattice_hip_interpolate_point_features_grad(const float* point_grad, int channels,
                                                           const float* weights, const int32_t* voxel_offsets,
                                                           const int32_t* entry_ids, int voxel_rows, float* out,
                                                           void* stream_ptr) {
    LATTICE_REQUIRE(channels > 0 && voxel_rows >= 0, "interpolation shapes must be positive.");
    if (voxel_rows == 0) return LATTICE_OK;
    LATTICE_REQUIRE(point_grad && weights && voxel_offsets && entry_ids && out,
                    "interpolation gradient pointers must be non-null.");
    LATTICE_LAUNCH_VEC(interpolate_grad, channels, voxel_rows, as_stream(stream_ptr), point_grad, channels, weights,
                       voxel_offsets, entry_ids, voxel_rows, out);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}
