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

#include <cstring>


#include <algorithm>
#include <climits>

#include "lattice_common.h"

#include "scan.h"
#include "sort.h"

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
clear_table(CoordSlot* slots, int capacity) {
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < capacity; i += gridDim.x * kThreads) {
        reinterpret_cast<int4*>(slots)[i] = empty_coord_slot();
    }
}

// Small writes a relation build needs before its first query, folded into
// the table clear so they cost no launch of their own: zero the status
// word, set counts[1] (the active output rows), copy the active input
// coordinates to out_coords (zero tail).  Each part is skipped when its
// pointer is null.
struct Prologue {
    int32_t* status;
    const int32_t* count_src;  // counts[1] = clamp(*count_src, 0, count_limit)
    int count_limit;
    int32_t* counts;
    const int32_t* copy_src;   // out_coords rows [0, copy_rows)
    const int32_t* copy_active;
    int copy_rows;
    int32_t* copy_dst;
};

// Clears a block table (key = empty, all eight rows absent: one thread per
// 16-byte quarter of a bucket) and runs the prologue.
__global__ void __launch_bounds__(kThreads)
clear_blocks(BlockBucket* buckets, long long quarters, Prologue p) {
    const long long tid = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x;
    const long long step = static_cast<long long>(gridDim.x) * kThreads;
    int4* q = reinterpret_cast<int4*>(buckets);
    for (long long i = tid; i < quarters; i += step) {
        q[i] = (i & 3) == 0 ? make_int4(-1, -1, 0, 0) : make_int4(0, 0, 0, 0);
    }
    if (tid == 0) {
        if (p.status != nullptr) p.status[0] = 0;
        if (p.count_src != nullptr) p.counts[1] = min(max(*p.count_src, 0), p.count_limit);
    }
    if (p.copy_src != nullptr) {
        const int active = min(max(*p.copy_active, 0), p.copy_rows);
        int4* out = reinterpret_cast<int4*>(p.copy_dst);
        for (long long i = tid; i < p.copy_rows; i += step) {
            out[i] = i < active ? reinterpret_cast<const int4*>(p.copy_src)[i] : make_int4(0, 0, 0, 0);
        }
    }
}

// Inserts the active rows into the block table.  Every int32 coordinate
// has a key: packed when it fits, wide otherwise.  kExact = false stores
// the rows plainly (see BlockTable::insert).
template <bool kExact>
__global__ void __launch_bounds__(kThreads)
insert_blocks(BlockTable table, const int32_t* __restrict__ coords, int rows,
              const int32_t* __restrict__ active_rows) {
    const int active = min(max(*active_rows, 0), rows);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < active; i += gridDim.x * kThreads) {
        const int4 c = load_coord(coords, i);
        TableKey block_key;
        int octant;
        block_of(c.x, c.y, c.z, c.w, &block_key, &octant);
        table.insert<kExact>(block_key, octant, i);
    }
}

// The floor-divided cell of an input row (downsample_values,
// quantization_detail.h:12-31): the key source of the cell table.
struct CellSource {
    const int32_t* coords;
    Int3 cell;
    __device__ inline FullKey key_of(int32_t row) const {
        const int4 c = load_coord(coords, row);
        return {c.x, floor_div_pos(c.y, cell.x), floor_div_pos(c.z, cell.y), floor_div_pos(c.w, cell.z)};
    }
    __device__ inline TableKey table_key_of(int32_t row) const {
        const FullKey k = key_of(row);
        return table_key(k.b, k.x, k.y, k.z);
    }
};

// Inserts active rows keyed by their floor-divided cell.
__global__ void __launch_bounds__(kThreads)
insert_rows(CoordTable table, const int32_t* __restrict__ coords, int rows,
            const int32_t* __restrict__ active_rows, Int3 cell) {
    const int active = min(max(*active_rows, 0), rows);
    const CellSource src{coords, cell};
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < active; i += gridDim.x * kThreads) {
        table.insert(src.table_key_of(i), i, src);
    }
}

// ---------------------------------------------- strided output planning --
//
// First-seen placement of the output cells: a flag per input row (the row
// is its cell's first row), the flag count of every 64-row group (one
// wave: rows 64g .. 64g + 63), one scan of the group counts
// (scan_block_totals, which also writes the cell count), and a scatter in
// which each wave ranks its flags with a ballot.  Grid-stride loops step
// by whole blocks, so a wave always holds one aligned 64-row group.

// Writes the flag count of the calling wave's 64-row group.
__device__ inline void write_group_total(bool flag, long long i, int32_t* group_totals) {
    const uint64_t b = ballot(flag);
    if (lane_id() == 0) group_totals[i >> 6] = __popcll(b);
}

// Output row of a flagged input row: its group's offset plus its rank
// among the group's flags.
__device__ inline int group_position(bool flag, long long i, const int32_t* group_offsets) {
    const uint64_t b = ballot(flag);
    return group_offsets[i >> 6] + lanes_below(b);
}

// flags[i] = 1 when input row i is the first row of its floor-divided cell.
__global__ void __launch_bounds__(kThreads)
flag_cell_representatives(CoordTable cells, const int32_t* __restrict__ coords, int rows,
                          const int32_t* __restrict__ active_rows, Int3 cell,
                          int32_t* __restrict__ flags, int32_t* __restrict__ group_totals) {
    const int active = min(max(*active_rows, 0), rows);
    const CellSource src{coords, cell};
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        const bool flag = i < active && cells.find(src.table_key_of(i), src) == i;
        flags[i] = flag ? 1 : 0;
        write_group_total(flag, i, group_totals);
    }
}

// Scatters representative cells to their first-seen position; zero tail.
__global__ void __launch_bounds__(kThreads)
scatter_cells(const int32_t* __restrict__ coords, int rows, const int32_t* __restrict__ flags,
              const int32_t* __restrict__ group_offsets, const int32_t* __restrict__ counts,
              Int3 cell, int32_t* __restrict__ out_coords) {
    const int n_out = counts[1];
    int4* out = reinterpret_cast<int4*>(out_coords);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        const bool flag = flags[i] != 0;
        const int pos = group_position(flag, i, group_offsets);
        if (flag) {
            int4 c = load_coord(coords, i);
            int4 q;
            q.x = c.x;
            q.y = static_cast<int>(floor_div_pos(c.y, cell.x));
            q.z = static_cast<int>(floor_div_pos(c.z, cell.y));
            q.w = static_cast<int>(floor_div_pos(c.w, cell.z));
            out[pos] = q;
        }
        if (i >= n_out) out[i] = make_int4(0, 0, 0, 0);
    }
}

// ------------------------------------------- 2x2x2 stride-2 downsample --
//
// kernel_size = stride = 2, no padding, unit dilation: the cell of a voxel
// is floor(v / 2) per axis, which is exactly the 2x2x2 block the block
// table buckets by, and offset k = 4 dx + 2 dy + dz of output cell X is the
// voxel 2X + (dx, dy, dz), i.e. octant k of that block.  So the input rows'
// block table alone gives the downsample (no cell table): a cell's first
// row is the minimum of its bucket's eight first rows, and its map row is
// the bucket's eight rows in order.

// Decoded first row of a bucket entry (-1 when absent).
__device__ inline int32_t bucket_row(int32_t raw) { return raw == 0 ? -1 : kRowBias - raw; }

// flags[i] = 1 when input row i is its cell's first row; buckets[i] = its
// cell's bucket.
__global__ void __launch_bounds__(kThreads)
flag_block_representatives(BlockTable table, const int32_t* __restrict__ coords, int rows,
                           const int32_t* __restrict__ active_rows, int32_t* __restrict__ flags,
                           int32_t* __restrict__ buckets, int32_t* __restrict__ group_totals) {
    const int active = min(max(*active_rows, 0), rows);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        int flag = 0, bucket = -1;
        if (i < active) {
            const int4 c = load_coord(coords, i);
            TableKey key;
            int octant;
            block_of(c.x, c.y, c.z, c.w, &key, &octant);
            bucket = table.find_bucket(key);  // present: row i inserted it
            const int4* r = reinterpret_cast<const int4*>(table.buckets + bucket);
            const int4 lo = r[0], mid = r[1];
            const int2 hi = *reinterpret_cast<const int2*>(r + 2);
            // stored rows are kRowBias - row (0 = absent): the first row of
            // the cell is the largest stored value
            const int32_t top = max(max(max(lo.z, lo.w), max(mid.x, mid.y)), max(max(mid.z, mid.w), max(hi.x, hi.y)));
            flag = bucket_row(top) == i ? 1 : 0;
        }
        flags[i] = flag;
        buckets[i] = bucket;
        write_group_total(flag != 0, i, group_totals);
    }
}

// Places each cell at its first-seen position: out_coords (zero tail) and
// the cell's bucket (out_buckets, -1 tail).
__global__ void __launch_bounds__(kThreads)
scatter_block_cells(const int32_t* __restrict__ coords, int rows, const int32_t* __restrict__ flags,
                    const int32_t* __restrict__ group_offsets, const int32_t* __restrict__ buckets,
                    const int32_t* __restrict__ counts, int32_t* __restrict__ out_coords,
                    int32_t* __restrict__ out_buckets) {
    const int n_out = counts[1];
    int4* out = reinterpret_cast<int4*>(out_coords);
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < rows; i += gridDim.x * kThreads) {
        const bool flag = flags[i] != 0;
        const int pos = group_position(flag, i, group_offsets);
        if (flag) {
            const int4 c = load_coord(coords, i);
            out[pos] = make_int4(c.x, c.y >> 1, c.z >> 1, c.w >> 1);
            out_buckets[pos] = buckets[i];
        }
        if (i >= n_out) {
            out[i] = make_int4(0, 0, 0, 0);
            out_buckets[i] = -1;
        }
    }
}

// Map query of the 2x2x2 stride-2 downsample: one lane per output row
// copies its cell's bucket rows to out_in_map (K = 8) and writes the row
// mask and degree; per-block degree totals feed the row-offset scan, as in
// query_map.
__global__ void __launch_bounds__(kWave)
query_map_blocks(BlockTable table, const int32_t* __restrict__ out_buckets, int out_capacity,
                 int32_t* __restrict__ out_in_map, int32_t* __restrict__ row_masks, int32_t* __restrict__ degrees,
                 int32_t* __restrict__ block_totals) {
    const int lane = lane_id();
    const long long row = static_cast<long long>(blockIdx.x) * kWave + lane;  // kQueryRows rows per block
    int degree = 0;
    if (row < out_capacity) {
        const int32_t b = out_buckets[row];
        int v[8];
        if (b >= 0) {
            const int4* r = reinterpret_cast<const int4*>(table.buckets + b);
            const int4 lo = r[0], mid = r[1];
            const int2 hi = *reinterpret_cast<const int2*>(r + 2);
            v[0] = bucket_row(lo.z);
            v[1] = bucket_row(lo.w);
            v[2] = bucket_row(mid.x);
            v[3] = bucket_row(mid.y);
            v[4] = bucket_row(mid.z);
            v[5] = bucket_row(mid.w);
            v[6] = bucket_row(hi.x);
            v[7] = bucket_row(hi.y);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = -1;
        }
        uint32_t mask = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            mask |= v[k] >= 0 ? 1u << k : 0u;
        }
        degree = __popc(mask);
        int4* dst = reinterpret_cast<int4*>(out_in_map + row * 8);
        dst[0] = make_int4(v[0], v[1], v[2], v[3]);
        dst[1] = make_int4(v[4], v[5], v[6], v[7]);
        row_masks[row] = static_cast<int32_t>(mask);
        degrees[row] = degree;
    }
    int sum = degree;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
    if (lane == 0) block_totals[blockIdx.x] = sum;
}

// Identity output support: out_coords = active prefix of coords, zero tail.
// ------------------------------------------------------------ map query --
//
// Lanes per output row: 32 when K <= 32 (two rows per wave), else 64 with a
// loop over 64-offset chunks.  Each lane probes one offset; the ballot of
// hits gives the row mask words and the degree.  A block owns kQueryRows
// consecutive output rows; it writes their degrees and (optionally) their
// sum, from which the row offsets are scanned per block.

constexpr int kQueryRows = 64;

struct QueryArgs {
    const int32_t* out_coords;   // coordinates of the output rows
    int out_capacity;
    const int32_t* out_active;   // device count of active output rows
    const int32_t* offsets;      // device [K,3] or null (closed form)
    KernelGeometry geom;
    int words;
    BlockTable table;
    int32_t* out_in_map;         // [out_capacity, K]
    int32_t* row_masks;          // [out_capacity, words]
    int32_t* degrees;            // [out_capacity] or null
    int32_t* block_totals;       // [ceil(out_capacity / kQueryRows)] or null
    const int32_t* out_buckets;  // 2x2x2 stride-2 downsample: bucket of each output cell, else null
    // Submanifold relations: status word that gets LATTICE_STATUS_REPEATED_COORD
    // when an active row's self lookup (offset index `center`, the zero
    // offset) finds an earlier row with the same coordinate; else null.
    int32_t* repeat_status;
    int center;
    // 3x3x3 submanifold over a table whose voxel slots were stored plainly:
    // an active row whose self lookup finds a larger row (a repeated
    // coordinate whose store came last) puts its own row back with an
    // atomic max, and the repeat flag makes the query run again
    // (rerun_if: the status word; the launch returns at once when its
    // LATTICE_STATUS_REPEATED_COORD bit is clear).
    bool fix_rows;
    const int32_t* rerun_if;
};

// Flags a repeated coordinate seen by any lane of the wave (one atomic).
__device__ inline void flag_repeats(int32_t* status, bool repeated) {
    const uint64_t any = ballot(repeated);
    if (any != 0 && lane_id() == __ffsll(static_cast<long long>(any)) - 1) {
        atomicOr(status, LATTICE_STATUS_REPEATED_COORD);
    }
}

template <int kLanes>
__global__ void __launch_bounds__(kThreads) query_map(QueryArgs a) {
    constexpr int kRowsPerWave = kWave / kLanes;
    constexpr int kRowsPerPass = kRowsPerWave * (kThreads / kWave);
    __shared__ int wave_sum[kThreads / kWave];
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int sub = lane / kLanes;          // row slot within the wave
    const int k_lane = lane % kLanes;
    const int K = a.geom.volume;
    const int n_active = min(max(*a.out_active, 0), a.out_capacity);
    int degree_sum = 0;
    for (int pass = 0; pass < kQueryRows / kRowsPerPass; ++pass) {
        const long long row = static_cast<long long>(blockIdx.x) * kQueryRows + pass * kRowsPerPass +
                              wave * kRowsPerWave + sub;
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
                TableKey block_key;
                int octant;
                if (block_of(oc.x, x, y, z, &block_key, &octant)) found = a.table.find(block_key, octant);
            }
            if (row_ok && k < K) a.out_in_map[row * K + k] = found;
            if (a.repeat_status != nullptr) flag_repeats(a.repeat_status, row_active && k == a.center && found != row);
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
        if (row_ok && k_lane == 0) {
            if (a.degrees != nullptr) a.degrees[row] = degree;
            degree_sum += degree;
        }
    }
    if (a.block_totals == nullptr) return;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) degree_sum += __shfl_xor(degree_sum, off, kWave);
    if (lane == 0) wave_sum[wave] = degree_sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        int total = 0;
        for (int w = 0; w < kThreads / kWave; ++w) total += wave_sum[w];
        a.block_totals[blockIdx.x] = total;
    }
}

// 3x3x3 offsets, unit stride and dilation, no padding (submanifold and
// k=3 target maps): one lane per output row.  The 27 neighbours of a voxel
// lie in the 2x2x2 blocks (v-1)>>1 .. +1 on each axis, 8 blocks in all, so a
// row costs 8 hash probes instead of 27, and all 8 bucket reads are issued
// before any is used.  The buckets' rows form a 4x4x4 window around the
// voxel; the neighbour at offset d sits at window index d + 2 - (v & 1) per
// axis, picked with selects on the coordinate parities.  The wave's 64 map
// rows are staged in LDS and written out contiguously.
constexpr int kK3 = 27;

// Queries the 64 rows row0 .. row0 + 63 (one per lane): stages their map
// rows in `stage`, writes row_masks, returns the lane's degree (0 past the
// active rows).  The caller copies `stage` to out_in_map.
__device__ inline int query_rows_k3(const QueryArgs& a, long long row0, int lane, int32_t* stage) {
    constexpr int K = kK3;
    const long long row = row0 + lane;
    const int n_active = min(max(*a.out_active, 0), a.out_capacity);
    const bool row_ok = row < a.out_capacity;
    const bool active = row < n_active;
    const int4 c = active ? load_coord(a.out_coords, row) : make_int4(0, 0, 0, 0);
    // The window's blocks floor((v - 1) / 2) .. floor((v + 1) / 2) per axis
    // have packed keys when v lies in [-2^18 + 1, 2^18 - 2] and the batch in
    // [0, 1022]; int32 arithmetic is exact there.
    const auto window_packs = [](int v) { return v >= -(1 << 18) + 1 && v <= (1 << 18) - 2; };
    const bool packed = c.x >= 0 && c.x <= LATTICE_MAX_BATCH && window_packs(c.y) && window_packs(c.z) &&
                        window_packs(c.w);
    uint64_t keys[8];
    bool key_ok[8];
    uint32_t slot[8];
    uint4 lo[8], mid[8];
    uint2 hi[8];
    if (packed || !active) {
        const int bx = (c.y - 1) >> 1, by = (c.z - 1) >> 1, bz = (c.w - 1) >> 1;  // floor division
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            pack_key(c.x, bx + (j >> 2), by + ((j >> 1) & 1), bz + (j & 1), &keys[j]);
            key_ok[j] = active;
            slot[j] = static_cast<uint32_t>(mix64(keys[j])) & a.table.mask;
            const uint4* bucket = reinterpret_cast<const uint4*>(a.table.buckets + slot[j]);
            lo[j] = bucket[0];   // key, rows 0..1
            mid[j] = bucket[1];  // rows 2..5
            hi[j] = *reinterpret_cast<const uint2*>(bucket + 2);  // rows 6..7
        }
    } else {
        // Rare: some block key is wide.  Each block is found through the
        // table, which compares wide keys in full (int64: v - 1 leaves int32
        // at INT_MIN); the probe below then stops at once.
        const int64_t bx = (static_cast<int64_t>(c.y) - 1) >> 1;
        const int64_t by = (static_cast<int64_t>(c.z) - 1) >> 1;
        const int64_t bz = (static_cast<int64_t>(c.w) - 1) >> 1;
        for (int j = 0; j < 8; ++j) {
            const int32_t b = a.table.find_bucket(table_key(c.x, bx + (j >> 2), by + ((j >> 1) & 1), bz + (j & 1)));
            slot[j] = b < 0 ? 0u : static_cast<uint32_t>(b);
            const uint4* bucket = reinterpret_cast<const uint4*>(a.table.buckets + slot[j]);
            lo[j] = bucket[0];
            mid[j] = bucket[1];
            hi[j] = *reinterpret_cast<const uint2*>(bucket + 2);
            key_ok[j] = b >= 0;
            keys[j] = (static_cast<uint64_t>(lo[j].y) << 32) | lo[j].x;
        }
    }
    uint32_t rows[8][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint64_t k = (static_cast<uint64_t>(lo[j].y) << 32) | lo[j].x;
        while (key_ok[j] && k != keys[j] && k != kEmptyKey) {  // linear probing, rare
            slot[j] = (slot[j] + 1) & a.table.mask;
            const uint4* bucket = reinterpret_cast<const uint4*>(a.table.buckets + slot[j]);
            lo[j] = bucket[0];
            mid[j] = bucket[1];
            hi[j] = *reinterpret_cast<const uint2*>(bucket + 2);
            k = (static_cast<uint64_t>(lo[j].y) << 32) | lo[j].x;
        }
        const bool found = key_ok[j] && k == keys[j];
        rows[j][0] = found ? lo[j].z : 0u;
        rows[j][1] = found ? lo[j].w : 0u;
        rows[j][2] = found ? mid[j].x : 0u;
        rows[j][3] = found ? mid[j].y : 0u;
        rows[j][4] = found ? mid[j].z : 0u;
        rows[j][5] = found ? mid[j].w : 0u;
        rows[j][6] = found ? hi[j].x : 0u;
        rows[j][7] = found ? hi[j].y : 0u;
    }
    // window[lx][ly][lz], l in 0..3 = 2 * block + octant bit
    const bool px = c.y & 1, py = c.z & 1, pz = c.w & 1;
    uint32_t wx[3][4][4];  // x picked
#pragma unroll
    for (int dx = 0; dx < 3; ++dx)
#pragma unroll
        for (int ly = 0; ly < 4; ++ly)
#pragma unroll
            for (int lz = 0; lz < 4; ++lz) {
                const int l0 = dx + 1, l1 = dx;  // window x for even / odd voxel x
                const uint32_t even = rows[(l0 >> 1) * 4 + (ly >> 1) * 2 + (lz >> 1)][(l0 & 1) * 4 + (ly & 1) * 2 + (lz & 1)];
                const uint32_t odd = rows[(l1 >> 1) * 4 + (ly >> 1) * 2 + (lz >> 1)][(l1 & 1) * 4 + (ly & 1) * 2 + (lz & 1)];
                wx[dx][ly][lz] = px ? odd : even;
            }
    uint32_t mask = 0;
    int degree = 0;
    uint32_t self_raw = 0;
#pragma unroll
    for (int dx = 0; dx < 3; ++dx)
#pragma unroll
        for (int dy = 0; dy < 3; ++dy)
#pragma unroll
            for (int dz = 0; dz < 3; ++dz) {
                const uint32_t y0 = py ? wx[dx][dy][dz] : wx[dx][dy + 1][dz];
                const uint32_t y1 = py ? wx[dx][dy][dz + 1] : wx[dx][dy + 1][dz + 1];
                const uint32_t raw = pz ? y0 : y1;
                const int k = dx * 9 + dy * 3 + dz;
                if (k == kK3 / 2) self_raw = raw;
                const int32_t v = raw == 0 ? -1 : kRowBias - static_cast<int32_t>(raw);
                stage[lane * K + k] = v;
                if (raw != 0) {
                    mask |= 1u << k;
                    ++degree;
                }
            }
    if (a.fix_rows && active && self_raw != 0 && kRowBias - static_cast<int32_t>(self_raw) > row) {
        // the own voxel sits in window block (1 - x&1, 1 - y&1, 1 - z&1), octant (x&1, y&1, z&1)
        const int j_own = (px ? 0 : 4) + (py ? 0 : 2) + (pz ? 0 : 1);
        uint32_t own_slot = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) own_slot = j == j_own ? slot[j] : own_slot;
        atomicMax(&a.table.buckets[own_slot].rows[(px ? 4 : 0) + (py ? 2 : 0) + (pz ? 1 : 0)],
                  kRowBias - static_cast<int32_t>(row));
    }
    if (row_ok) a.row_masks[row] = static_cast<int32_t>(mask);
    return row_ok ? degree : 0;
}

// Copies the staged map rows of row0 .. row0 + 63 to out_in_map.
__device__ inline void store_map_rows_k3(const QueryArgs& a, long long row0, int lane, const int32_t* stage) {
    const int n = static_cast<int>(min(static_cast<long long>(kQueryRows), a.out_capacity - row0)) * kK3;
    int32_t* dst = a.out_in_map + row0 * kK3;
    for (int i = lane; i < n; i += kWave) dst[i] = stage[i];
}

__global__ void __launch_bounds__(kWave) query_map_k3(QueryArgs a) {
    if (a.rerun_if != nullptr && (*a.rerun_if & LATTICE_STATUS_REPEATED_COORD) == 0) return;
    __shared__ int32_t stage[kQueryRows * kK3];
    const int lane = lane_id();
    const long long chunks = (static_cast<long long>(a.out_capacity) + kQueryRows - 1) / kQueryRows;
    // one 64-row chunk per block, or several when the grid is capped (the
    // conditional second pass)
    for (long long chunk = blockIdx.x; chunk < chunks; chunk += gridDim.x) {
        const long long row0 = chunk * kQueryRows;
        const int degree = query_rows_k3(a, row0, lane, stage);
        if (a.degrees != nullptr && row0 + lane < a.out_capacity) a.degrees[row0 + lane] = degree;
        __syncthreads();
        if (a.repeat_status != nullptr) {
            const long long r = row0 + lane;
            const int n_active = min(max(*a.out_active, 0), a.out_capacity);
            flag_repeats(a.repeat_status, r < n_active && stage[lane * kK3 + kK3 / 2] != r);
        }
        store_map_rows_k3(a, row0, lane, stage);
        if (a.block_totals != nullptr) {
            int sum = degree;
#pragma unroll
            for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
            if (lane == 0) a.block_totals[chunk] = sum;
        }
        __syncthreads();
    }
}

bool is_unit_k3(const QueryArgs& a) {
    const KernelGeometry& g = a.geom;
    return a.offsets == nullptr && g.volume == 27 && g.size.x == 3 && g.size.y == 3 && g.size.z == 3 &&
           g.dilation.x == 1 && g.dilation.y == 1 && g.dilation.z == 1 && g.stride.x == 1 && g.stride.y == 1 &&
           g.stride.z == 1 && g.padding.x == 0 && g.padding.y == 0 && g.padding.z == 0 && a.words == 1;
}

// Exclusive prefix of the per-block degree totals (one workgroup); the sum
// of all is the edge count, counts[0].  Each thread owns a contiguous run;
// loads are issued kScanBatch at a time before use.
constexpr int kBlockScanThreads = 1024;
constexpr int kScanBatch = 16;

__global__ void __launch_bounds__(kBlockScanThreads)
scan_block_totals(const int32_t* __restrict__ totals, int blocks, int32_t* __restrict__ offsets,
                  int32_t* __restrict__ counts) {
    __shared__ int wave_sum[kBlockScanThreads / kWave];
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int per = (blocks + kBlockScanThreads - 1) / kBlockScanThreads;
    const int begin = threadIdx.x * per;
    const int end = min(begin + per, blocks);
    // Up to kScanBatch totals per thread (blocks <= 16384) stay in registers
    // between the two passes; larger inputs reload them.
    int first[kScanBatch];
    int sum = 0;
    for (int i0 = begin; i0 < end; i0 += kScanBatch) {
        int v[kScanBatch];
#pragma unroll
        for (int j = 0; j < kScanBatch; ++j) v[j] = i0 + j < end ? totals[i0 + j] : 0;
#pragma unroll
        for (int j = 0; j < kScanBatch; ++j) sum += v[j];
        if (i0 == begin) {
#pragma unroll
            for (int j = 0; j < kScanBatch; ++j) first[j] = v[j];
        }
    }
    int incl = sum;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int u = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += u;
    }
    if (lane == kWave - 1) wave_sum[wave] = incl;
    __syncthreads();
    int run = incl - sum;
    for (int w = 0; w < wave; ++w) run += wave_sum[w];
    if (threadIdx.x == kBlockScanThreads - 1) counts[0] = run + sum;
    for (int i0 = begin; i0 < end; i0 += kScanBatch) {
        int v[kScanBatch];
#pragma unroll
        for (int j = 0; j < kScanBatch; ++j)
            v[j] = i0 == begin ? first[j] : (i0 + j < end ? totals[i0 + j] : 0);
#pragma unroll
        for (int j = 0; j < kScanBatch; ++j) {
            if (i0 + j < end) offsets[i0 + j] = run;
            run += v[j];
        }
    }
}

// Edge emission in (out_row, kernel) order.  A block owns the same
// kQueryRows rows as in the query: it turns their degrees (read from
// row_offsets, where the query left them) into row offsets with its block
// offset, writes them back, and emits each row's edges from out_in_map.
// The block holding the last row also writes row_offsets[out_capacity].
template <int kLanes>
__global__ void __launch_bounds__(kThreads)
emit_edges(const int32_t* __restrict__ out_in_map, int out_capacity, int K,
           const int32_t* __restrict__ block_offsets, const int32_t* __restrict__ counts,
           int32_t* __restrict__ row_offsets, int32_t* __restrict__ in_rows, int32_t* __restrict__ out_rows,
           int32_t* __restrict__ kernel_ids) {
    static_assert(kQueryRows == kWave, "one wave scans a block's row degrees");
    constexpr int kRowsPerWave = kWave / kLanes;
    constexpr int kRowsPerPass = kRowsPerWave * (kThreads / kWave);
    __shared__ int start[kQueryRows];
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int sub = lane / kLanes;
    const int k_lane = lane % kLanes;
    const long long row0 = static_cast<long long>(blockIdx.x) * kQueryRows;
    if (wave == 0) {
        const long long r = row0 + lane;
        const int d = r < out_capacity ? row_offsets[r] : 0;
        int incl = d;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int u = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += u;
        }
        const int s0 = block_offsets[blockIdx.x] + incl - d;
        start[lane] = s0;
        if (r < out_capacity) row_offsets[r] = s0;
        if (r == out_capacity - 1) row_offsets[out_capacity] = counts[0];
    }
    __syncthreads();
    for (int pass = 0; pass < kQueryRows / kRowsPerPass; ++pass) {
        const int local = pass * kRowsPerPass + wave * kRowsPerWave + sub;
        const long long row = row0 + local;
        const bool row_ok = row < out_capacity;
        int cursor = row_ok ? start[local] : 0;
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

// --------------------------------------------------- grouped CSR views ----
//
// write_relation_grouped_view (relation_views_detail.h:84-120) is a stable
// counting sort of edge ids by a group id (input row or kernel offset).
// Here: keys = group of each active edge (inactive slots get the sentinel
// `groups`, which sorts last), a stable radix sort of (key, edge id), and
// the row offsets read off the sorted keys.

// offsets[g] = number of sorted keys below g, for g in [0, groups].  The
// lane at position i writes the groups its key step (prev, cur] skips.  The
// trailing run of empty groups (up to `groups`, past the last real key) can
// be as long as the capacity, so no lane writes it: the lane at its start
// records (first empty group, position) in tail[0..1] and fill_group_tail
// spreads it over the grid.
__global__ void __launch_bounds__(kThreads)
group_offsets(const int32_t* __restrict__ sorted_keys, int capacity, int groups, int32_t* __restrict__ offsets,
              int32_t* __restrict__ tail, const int32_t* run_if) {
    if (run_if != nullptr && *run_if == 0) return;
    for (int i = blockIdx.x * kThreads + threadIdx.x; i <= capacity; i += gridDim.x * kThreads) {
        const int prev = i > 0 ? min(sorted_keys[i - 1], groups) : -1;
        const int cur = i < capacity ? min(sorted_keys[i], groups) : groups;
        if (cur >= groups) {
            if (prev < groups) {
                tail[0] = prev + 1;
                tail[1] = i;
            }
            continue;
        }
        for (int g = prev + 1; g <= cur; ++g) offsets[g] = i;
    }
}

__global__ void __launch_bounds__(kThreads)
fill_group_tail(const int32_t* __restrict__ tail, int groups, int32_t* __restrict__ offsets, const int32_t* run_if) {
    if (run_if != nullptr && *run_if == 0) return;
    const int first = tail[0];
    const int value = tail[1];
    for (int g = blockIdx.x * kThreads + threadIdx.x; g <= groups; g += gridDim.x * kThreads) {
        if (g >= first) offsets[g] = value;
    }
}

constexpr unsigned kConditionalGrid = 1024;

// Row offsets of sorted group keys (sentinel `groups` for inactive slots);
// skipped on the device when run_if is non-null and *run_if == 0.
int launch_group_offsets(const int32_t* sorted_keys, int capacity, int groups, int32_t* offsets,
                         int32_t* tail, hipStream_t stream, const int32_t* run_if = nullptr) {
    // A conditional launch mostly returns at once, and the dispatch of its
    // workgroups is then its whole cost: it gets four blocks per CU, which
    // the grid-stride loops cover any size with.
    const unsigned max_grid = run_if != nullptr ? kConditionalGrid : 8192;
    group_offsets<<<grid_for(static_cast<long long>(capacity) + 1, kThreads, max_grid), kThreads, 0, stream>>>(
        sorted_keys, capacity, groups, offsets, tail, run_if);
    LATTICE_LAUNCH_CHECK();
    fill_group_tail<<<grid_for(static_cast<long long>(groups) + 1, kThreads, max_grid), kThreads, 0, stream>>>(
        tail, groups, offsets, run_if);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

// ------------------------------------------------------------- helpers ----

// Slot count of the coordinate table: a power of two at least twice the
// row count (so at least half the slots stay empty).
int table_capacity(int rows) {
    int cap = 1;
    const long long want = std::max(2ll * rows, 1ll);
    while (cap < want) cap <<= 1;
    return cap;
}

size_t table_bytes(int rows) {
    const size_t cap = static_cast<size_t>(table_capacity(rows));
    return aligned_bytes(cap * sizeof(CoordSlot));
}

int make_table(int rows, Workspace& ws, CoordTable* table) {
    const int cap = table_capacity(rows);
    table->slots = ws.take<CoordSlot>(cap);
    table->mask = static_cast<uint32_t>(cap - 1);
    if (table->slots == nullptr) {
        set_error("relation workspace too small for the coordinate table");
        return LATTICE_ERROR_INVALID_ARGUMENT;
    }
    return LATTICE_OK;
}

int build_table(const int32_t* coords, int rows, const int32_t* active_rows, Int3 cell,
                Workspace& ws, hipStream_t stream, CoordTable* table, int32_t* status = nullptr) {
    int rc = make_table(rows, ws, table);
    if (rc != LATTICE_OK) return rc;
    table->status = status;
    const int cap = static_cast<int>(table->mask) + 1;
    clear_table<<<grid_for(cap, kThreads, 4096), kThreads, 0, stream>>>(table->slots, cap);
    LATTICE_LAUNCH_CHECK();
    if (rows > 0) {
        insert_rows<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
            *table, coords, rows, active_rows, cell);
        LATTICE_LAUNCH_CHECK();
    }
    return LATTICE_OK;
}

// Bucket count of the block table: a power of two above 1.5x the row count,
// so the load factor stays below 2/3 even when every voxel has its own block.
int block_capacity(int rows) {
    int cap = 1;
    const long long want = std::max(static_cast<long long>(rows) + rows / 2 + 1, 1ll);
    while (cap < want) cap <<= 1;
    return cap;
}

size_t block_table_bytes(int rows) {
    return aligned_bytes(static_cast<size_t>(block_capacity(rows)) * sizeof(BlockBucket));
}

// The block table sits at the start of the workspace.  With `ready` the
// workspace already holds the table of these coordinates and active rows
// (an earlier relation build over them): only the prologue runs.
int build_block_table(const int32_t* coords, int rows, const int32_t* active_rows,
                      const Prologue& prologue, Workspace& ws, hipStream_t stream, BlockTable* table,
                      bool ready = false, bool exact_rows = true) {
    const int cap = block_capacity(rows);
    table->buckets = ws.take<BlockBucket>(cap);
    table->mask = static_cast<uint32_t>(cap - 1);
    table->src = BlockSource{coords};
    table->status = prologue.status;
    if (table->buckets == nullptr) {
        set_error("relation workspace too small for the coordinate table");
        return LATTICE_ERROR_INVALID_ARGUMENT;
    }
    const long long quarters = ready ? 0 : 4ll * cap;
    clear_blocks<<<grid_for(std::max<long long>({quarters, prologue.copy_rows, 1}), kThreads, 8192), kThreads, 0,
                   stream>>>(table->buckets, quarters, prologue);
    LATTICE_LAUNCH_CHECK();
    if (rows > 0 && !ready) {
        if (exact_rows) {
            insert_blocks<true><<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(*table, coords, rows,
                                                                                      active_rows);
        } else {
            insert_blocks<false><<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(*table, coords, rows,
                                                                                       active_rows);
        }
        LATTICE_LAUNCH_CHECK();
    }
    return LATTICE_OK;
}

size_t group_view_bytes(int edge_capacity) {
    const size_t n = static_cast<size_t>(std::max(edge_capacity, 1));
    return aligned_bytes(n * sizeof(int32_t)) + aligned_bytes(2 * sizeof(int32_t)) +
           radix_sort_workspace_bytes(edge_capacity, 32) + 1024;
}

int bit_width(int v) {
    int bits = 1;
    while ((1 << bits) <= v) ++bits;
    return bits;
}

// One grouped view: stable sort of edge ids by group; offsets[groups + 1].
int build_group_view(const int32_t* group_ids, const int32_t* counts, int edge_capacity, int groups,
                     int32_t* offsets, int32_t* edge_ids, Workspace ws, hipStream_t stream) {
    if (edge_capacity <= 0) return fill_i32(offsets, groups + 1, 0, stream);
    int32_t* sorted = ws.take<int32_t>(edge_capacity);
    int32_t* tail = ws.take<int32_t>(2);
    LATTICE_REQUIRE(sorted && tail, "grouped view workspace too small.");
    const SortKeys keys{group_ids, 1, counts, groups, false};
    int rc = radix_sort_indices(keys, edge_capacity, bit_width(groups), sorted, edge_ids, ws, stream);
    if (rc != LATTICE_OK) return rc;
    return launch_group_offsets(sorted, edge_capacity, groups, offsets, tail, stream);
}

int build_group_views(const int32_t* in_rows, const int32_t* kernel_ids, const int32_t* counts, int edge_capacity,
                      int in_capacity, int K, int32_t* in_row_offsets, int32_t* in_edge_ids,
                      int32_t* kernel_row_offsets, int32_t* kernel_edge_ids, Workspace& ws, hipStream_t stream) {
    int rc = build_group_view(kernel_ids, counts, edge_capacity, K, kernel_row_offsets, kernel_edge_ids, ws, stream);
    if (rc != LATTICE_OK) return rc;
    return build_group_view(in_rows, counts, edge_capacity, in_capacity, in_row_offsets, in_edge_ids, ws, stream);
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

int query_blocks(int out_capacity) { return (out_capacity + kQueryRows - 1) / kQueryRows; }

int launch_query(const QueryArgs& a, hipStream_t stream) {
    if (a.out_capacity <= 0) return LATTICE_OK;
    const unsigned blocks = static_cast<unsigned>(query_blocks(a.out_capacity));
    if (a.out_buckets != nullptr) {
        query_map_blocks<<<blocks, kWave, 0, stream>>>(a.table, a.out_buckets, a.out_capacity, a.out_in_map,
                                                       a.row_masks, a.degrees, a.block_totals);
    } else if (is_unit_k3(a)) {
        query_map_k3<<<blocks, kWave, 0, stream>>>(a);
    } else if (a.geom.volume <= 32) {
        query_map<32><<<blocks, kThreads, 0, stream>>>(a);
    } else {
        query_map<64><<<blocks, kThreads, 0, stream>>>(a);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

int launch_emit(const int32_t* map, int out_capacity, int K, const int32_t* block_offsets,
                const lattice_relation_outputs* out, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(query_blocks(out_capacity));
    if (K <= 32) {
        emit_edges<32><<<blocks, kThreads, 0, stream>>>(map, out_capacity, K, block_offsets, out->counts,
                                                        out->row_offsets, out->in_rows, out->out_rows,
                                                        out->kernel_ids);
    } else {
        emit_edges<64><<<blocks, kThreads, 0, stream>>>(map, out_capacity, K, block_offsets, out->counts,
                                                        out->row_offsets, out->in_rows, out->out_rows,
                                                        out->kernel_ids);
    }
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

// Exclusive scan of the flag counts of the 64-row groups of `rows` rows;
// *total (device) receives the sum.  rows == 0 writes a zero total.
int scan_groups(const int32_t* group_totals, int rows, int32_t* group_offsets, int32_t* total, hipStream_t stream) {
    if (rows <= 0) return fill_i32(total, 1, 0, stream);
    scan_block_totals<<<1, kBlockScanThreads, 0, stream>>>(group_totals, query_blocks(rows), group_offsets, total);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

// Common tail: query (degrees + per-block totals) -> scan of the block
// totals -> emit (row offsets + edges) -> grouped views when requested.
int finish_relation(QueryArgs q, int in_capacity, const lattice_relation_outputs* out, Workspace& ws,
                    hipStream_t stream) {
    const int K = q.geom.volume;
    const int out_capacity = q.out_capacity;
    if (out_capacity <= 0) {
        int rc = fill_i32(out->row_offsets, 1, 0, stream);
        if (rc != LATTICE_OK) return rc;
        rc = fill_i32(out->counts, 1, 0, stream);
        if (rc != LATTICE_OK) return rc;
    } else {
        const int blocks = query_blocks(out_capacity);
        int32_t* totals = ws.take<int32_t>(blocks);
        int32_t* offsets = ws.take<int32_t>(blocks);
        LATTICE_REQUIRE(totals && offsets, "relation workspace too small.");
        q.degrees = out->row_offsets;  // degrees land in row_offsets; emit turns them into offsets
        q.block_totals = totals;
        int rc = launch_query(q, stream);
        if (rc != LATTICE_OK) return rc;
        if (q.fix_rows) {
            // the same query again once a repeated coordinate has restored its
            // first row; a capped grid that returns at once otherwise
            QueryArgs again = q;
            again.fix_rows = false;
            again.rerun_if = q.repeat_status;
            query_map_k3<<<static_cast<unsigned>(std::min(blocks, 1024)), kWave, 0, stream>>>(again);
            LATTICE_LAUNCH_CHECK();
        }
        scan_block_totals<<<1, kBlockScanThreads, 0, stream>>>(totals, blocks, offsets, out->counts);
        LATTICE_LAUNCH_CHECK();
        rc = launch_emit(q.out_in_map, out_capacity, K, offsets, out, stream);
        if (rc != LATTICE_OK) return rc;
    }
    if (out->in_edge_ids == nullptr && out->kernel_edge_ids == nullptr) return LATTICE_OK;  // views on demand
    return build_group_views(out->in_rows, out->kernel_ids, out->counts, out_capacity * K, in_capacity, K,
                             out->in_row_offsets, out->in_edge_ids, out->kernel_row_offsets, out->kernel_edge_ids,
                             ws, stream);
}

int check_outputs(const lattice_relation_outputs* out, bool need_coords, long long out_capacity, int K) {
    LATTICE_REQUIRE(out != nullptr, "relation outputs are required.");
    LATTICE_REQUIRE(out->row_offsets && out->counts && out->status, "relation output pointers must be non-null.");
    const bool views = out->in_edge_ids != nullptr || out->kernel_edge_ids != nullptr;
    LATTICE_REQUIRE(!views || (out->in_edge_ids && out->kernel_edge_ids && out->in_row_offsets &&
                               out->kernel_row_offsets),
                    "grouped view outputs must be all set or all null.");
    if (out_capacity > 0) {
        LATTICE_REQUIRE(out->in_rows && out->out_rows && out->kernel_ids && out->out_in_map && out->row_masks,
                        "relation output pointers must be non-null.");
        LATTICE_REQUIRE(!need_coords || out->out_coords != nullptr, "out_coords must be non-null.");
    }
    (void)K;
    return LATTICE_OK;
}

}  // namespace

size_t forward_relation_bytes(int rows, int K) {
    size_t bytes = block_table_bytes(rows) + table_bytes(rows);           // coords + cells
    bytes += 2 * aligned_bytes(static_cast<size_t>(rows) * sizeof(int32_t)); // flags + positions
    bytes += scan_workspace_bytes(rows);
    bytes += 2 * aligned_bytes(static_cast<size_t>(query_blocks(rows) + 1) * sizeof(int32_t));  // block sums
    bytes += group_view_bytes(rows * K);
    return bytes + 4096;
}

}  // namespace lattice

using namespace lattice;

extern "C" int lattice_hip_coord_hash_capacity(int rows) { return table_capacity(rows); }

extern "C" int lattice_hip_block_table_capacity(int rows) { return block_capacity(rows); }

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
    size_t bytes = block_table_bytes(std::max(rows, 0));
    bytes += 2 * aligned_bytes(static_cast<size_t>(query_blocks(std::max(target_rows, 0)) + 1) * sizeof(int32_t));
    bytes += group_view_bytes(std::max(target_rows, 0) * std::max(kernel_count, 1));
    return bytes + 4096;
}

extern "C" size_t lattice_hip_block_table_bytes(int rows) { return block_table_bytes(std::max(rows, 0)); }

extern "C" int lattice_hip_build_kernel_relation(const int32_t* coords, int rows, const int32_t* active_rows,
                                                 const int kernel_size[3], const int stride[3],
                                                 const int padding[3], const int dilation[3],
                                                 const lattice_relation_outputs* out, void* workspace,
                                                 size_t workspace_bytes, void* stream_ptr) {
    // The block table sits at the start of the workspace, the rest after it.
    const size_t flags = workspace_bytes & LATTICE_RELATION_TABLE_READY;
    const size_t bytes = workspace_bytes & ~static_cast<size_t>(LATTICE_RELATION_TABLE_READY);
    const size_t tbytes = block_table_bytes(std::max(rows, 0));
    const bool split = workspace != nullptr && bytes >= tbytes;  // else the callee reports what is wrong
    return lattice_hip_build_kernel_relation_with_table(
        coords, rows, active_rows, kernel_size, stride, padding, dilation, out, workspace,
        (split ? tbytes : bytes) | flags, split ? static_cast<char*>(workspace) + tbytes : nullptr,
        split ? bytes - tbytes : 0, stream_ptr);
}

extern "C" int lattice_hip_build_kernel_relation_with_table(
    const int32_t* coords, int rows, const int32_t* active_rows, const int kernel_size[3], const int stride[3],
    const int padding[3], const int dilation[3], const lattice_relation_outputs* out, void* table_mem,
    size_t table_bytes, void* workspace, size_t workspace_bytes, void* stream_ptr) {
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
    const bool table_ready = (table_bytes & LATTICE_RELATION_TABLE_READY) != 0;
    table_bytes &= ~static_cast<size_t>(LATTICE_RELATION_TABLE_READY);
    LATTICE_REQUIRE(table_mem != nullptr && table_bytes >= block_table_bytes(rows), "block table too small.");
    LATTICE_REQUIRE(workspace_bytes >= forward_relation_bytes(rows, K) - block_table_bytes(rows),
                    "relation workspace too small.");
    hipStream_t stream = as_stream(stream_ptr);
    Workspace tws{static_cast<char*>(table_mem), table_bytes};
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};

    const bool identity = stride[0] == 1 && stride[1] == 1 && stride[2] == 1 && padding[0] == 0 &&
                          padding[1] == 0 && padding[2] == 0;
    Prologue prologue{out->status, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr};
    if (identity) {
        // submanifold: out_coords = the active input coords, counts[1] = active rows
        prologue.count_src = active_rows;
        prologue.count_limit = rows;
        prologue.counts = out->counts;
        prologue.copy_src = coords;
        prologue.copy_active = active_rows;
        prologue.copy_rows = rows;
        prologue.copy_dst = out->out_coords;
    }
    // The 3x3x3 submanifold query restores first rows itself, so its table
    // takes plain stores (one device atomic per row instead of two).
    const bool unit_k3_subm = identity && kernel_size[0] == 3 && kernel_size[1] == 3 && kernel_size[2] == 3 &&
                              dilation[0] == 1 && dilation[1] == 1 && dilation[2] == 1;
    BlockTable table;
    rc = build_block_table(coords, rows, active_rows, prologue, tws, stream, &table, table_ready, !unit_k3_subm);
    if (rc != LATTICE_OK) return rc;

    QueryArgs q{};
    q.out_capacity = rows;
    q.offsets = nullptr;
    q.geom = geom;
    q.words = (K + 31) / 32;
    q.table = table;
    q.out_in_map = out->out_in_map;
    q.row_masks = out->row_masks;
    if (identity) {
        q.out_coords = coords;
        q.out_active = out->counts + 1;
        // The self lookup: the zero offset sits at index size/2 of each odd
        // axis and at index 0 of an even one.
        const int cx = kernel_size[0] % 2 ? kernel_size[0] / 2 : 0;
        const int cy = kernel_size[1] % 2 ? kernel_size[1] / 2 : 0;
        const int cz = kernel_size[2] % 2 ? kernel_size[2] / 2 : 0;
        q.repeat_status = out->status;
        q.center = (cx * kernel_size[1] + cy) * kernel_size[2] + cz;
        q.fix_rows = unit_k3_subm && !table_ready;
    } else if (kernel_size[0] == 2 && kernel_size[1] == 2 && kernel_size[2] == 2 && stride[0] == 2 &&
               stride[1] == 2 && stride[2] == 2 && padding[0] == 0 && padding[1] == 0 && padding[2] == 0 &&
               dilation[0] == 1 && dilation[1] == 1 && dilation[2] == 1) {
        // 2x2x2 stride-2 downsample: the cells are the block table's buckets.
        int32_t* flags = ws.take<int32_t>(std::max(rows, 1));
        int32_t* buckets = ws.take<int32_t>(std::max(rows, 1));
        int32_t* out_buckets = ws.take<int32_t>(std::max(rows, 1));
        int32_t* group_totals = ws.take<int32_t>(query_blocks(rows) + 1);
        int32_t* group_offsets = ws.take<int32_t>(query_blocks(rows) + 1);
        LATTICE_REQUIRE(flags && buckets && out_buckets && group_totals && group_offsets,
                        "relation workspace too small.");
        if (rows > 0) {
            flag_block_representatives<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
                table, coords, rows, active_rows, flags, buckets, group_totals);
            LATTICE_LAUNCH_CHECK();
        }
        rc = scan_groups(group_totals, rows, group_offsets, out->counts + 1, stream);
        if (rc != LATTICE_OK) return rc;
        if (rows > 0) {
            scatter_block_cells<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
                coords, rows, flags, group_offsets, buckets, out->counts, out->out_coords, out_buckets);
            LATTICE_LAUNCH_CHECK();
        }
        q.out_coords = out->out_coords;
        q.out_active = out->counts + 1;
        q.out_buckets = out_buckets;
    } else {
        const Int3 cell{stride[0], stride[1], stride[2]};
        CoordTable cells;
        rc = build_table(coords, rows, active_rows, cell, ws, stream, &cells, out->status);
        if (rc != LATTICE_OK) return rc;
        int32_t* flags = ws.take<int32_t>(std::max(rows, 1));
        int32_t* group_totals = ws.take<int32_t>(query_blocks(rows) + 1);
        int32_t* group_offsets = ws.take<int32_t>(query_blocks(rows) + 1);
        LATTICE_REQUIRE(flags && group_totals && group_offsets, "relation workspace too small.");
        if (rows > 0) {
            flag_cell_representatives<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
                cells, coords, rows, active_rows, cell, flags, group_totals);
            LATTICE_LAUNCH_CHECK();
        }
        rc = scan_groups(group_totals, rows, group_offsets, out->counts + 1, stream);
        if (rc != LATTICE_OK) return rc;
        if (rows > 0) {
            scatter_cells<<<grid_for(rows, kThreads, 4096), kThreads, 0, stream>>>(
                coords, rows, flags, group_offsets, out->counts, cell, out->out_coords);
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
    const Prologue prologue{out->status, target_active_rows, target_rows, out->counts, nullptr, nullptr, 0, nullptr};
    BlockTable table;
    rc = build_block_table(coords, rows, active_rows, prologue, ws, stream, &table);
    if (rc != LATTICE_OK) return rc;
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

extern "C" size_t lattice_hip_relation_grouped_views_workspace_bytes(int edge_capacity) {
    return group_view_bytes(std::max(edge_capacity, 0));
}

extern "C" int lattice_hip_build_relation_grouped_views(const int32_t* in_rows, const int32_t* kernel_ids,
                                                        const int32_t* counts, int edge_capacity, int in_capacity,
                                                        int kernel_count, int32_t* in_row_offsets,
                                                        int32_t* in_edge_ids, int32_t* kernel_row_offsets,
                                                        int32_t* kernel_edge_ids, void* workspace,
                                                        size_t workspace_bytes, void* stream_ptr) {
    LATTICE_REQUIRE(edge_capacity >= 0 && in_capacity >= 0 && kernel_count > 0,
                    "grouped views need non-negative capacities and a positive kernel count.");
    LATTICE_REQUIRE(counts && in_row_offsets && kernel_row_offsets, "grouped view pointers must be non-null.");
    LATTICE_REQUIRE(edge_capacity == 0 || (in_rows && kernel_ids && in_edge_ids && kernel_edge_ids),
                    "grouped view pointers must be non-null.");
    LATTICE_REQUIRE(workspace_bytes >= lattice_hip_relation_grouped_views_workspace_bytes(edge_capacity),
                    "grouped view workspace too small.");
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    return build_group_views(in_rows, kernel_ids, counts, edge_capacity, in_capacity, kernel_count, in_row_offsets,
                             in_edge_ids, kernel_row_offsets, kernel_edge_ids, ws, as_stream(stream_ptr));
}

extern "C" size_t lattice_hip_implicit_gemm_view_workspace_bytes(int source_rows) {
    return block_table_bytes(std::max(source_rows, 0)) + 4096;
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
    const Prologue prologue{status, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr};
    BlockTable table;
    int rc = build_block_table(source_coords, source_rows, source_active_rows, prologue, ws, stream, &table);
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

// Gathers 64 sorted rows of out_in_map per block through LDS: rows are
// read as contiguous K-int segments, the K-major view is written as 64-int
// runs per offset and, when requested (non-null), the row-major sorted map
// as one contiguous block.
constexpr int kGatherRows = 64;

__global__ void __launch_bounds__(kThreads)
gather_sorted(const int32_t* __restrict__ out_in_map, const int32_t* __restrict__ row_masks, int rows, int K,
              const int32_t* __restrict__ order, int32_t* __restrict__ sorted_map, int32_t* __restrict__ kv_map,
              int32_t* __restrict__ tile_masks) {
    __shared__ int32_t tile[kGatherRows * 33];
    __shared__ int32_t src_rows[kGatherRows];
    const int row0 = blockIdx.x * kGatherRows;
    const int n = min(kGatherRows, rows - row0);
    if (threadIdx.x < kGatherRows) {
        // the quarter masks of this 64-row tile: OR of 16 sorted row masks
        // (rows past the end count as 0)
        const int src = threadIdx.x < n ? order[row0 + threadIdx.x] : -1;
        if (threadIdx.x < n) src_rows[threadIdx.x] = src;
        int m = src >= 0 ? row_masks[src] : 0;
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) m |= __shfl_xor(m, off, 16);
        if ((threadIdx.x & 15) == 0) tile_masks[blockIdx.x * 4 + threadIdx.x / 16] = m;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n * K; i += kThreads) {
        const int r = i / K;
        const int k = i - r * K;
        const int v = out_in_map[static_cast<long long>(src_rows[r]) * K + k];
        tile[r * 33 + k] = v;
        if (sorted_map != nullptr) sorted_map[static_cast<long long>(row0) * K + i] = v;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n * K; i += kThreads) {
        const int k = i / n;
        const int r = i - k * n;
        // non-temporal: the k-major map is read by the conv launches, not by
        // this kernel (sorted view of 400k rows 90 -> 87 us)
        __builtin_nontemporal_store(tile[r * 33 + k], kv_map + static_cast<long long>(k) * rows + row0 + r);
    }
}

}  // namespace
}  // namespace lattice

extern "C" size_t lattice_hip_sorted_view_workspace_bytes(int rows) {
    const size_t n = static_cast<size_t>(std::max(rows, 1));
    return aligned_bytes(n * sizeof(int32_t)) + radix_sort_workspace_bytes(rows, 32) + 4096;
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
    // Masks of K < 32 offsets are non-negative and fit in K bits; a 32-bit
    // mask sorts as a signed word, like the reference's int32 argsort.
    const SortKeys keys{row_masks, 1, nullptr, -1, kernel_count == 32};
    int rc = radix_sort_indices(keys, rows, kernel_count, nullptr, reorder_rows, ws, stream);
    if (rc != LATTICE_OK) return rc;
    gather_sorted<<<tiles, kThreads, 0, stream>>>(out_in_map, row_masks, rows, kernel_count, reorder_rows,
                                                  sorted_out_in_map, sorted_kv_out_in_map, tile_masks);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

// ---------------------------------------------------- expanded relations --
//
// Generative and transposed relations (relation_build_detail.h:82-196)
// expand every active input row into K candidates
//     cand(j) = (b, coord * stride + offset[k] - padding),  j = in * K + k,
// and give every (row, offset) exactly one edge.  Capacities are rows * K
// for both the output rows and the edges (relations.cpp:599-670).
//   * generative, and transposed when the stride exceeds the offsets' extent
//     on every axis (can_use_direct_transposed_relation, relations.cpp:
//     107-127): output row j is cand(j), edge j = (in, j, k).  One lane per j.
//   * other transposed relations: the output rows are the distinct
//     candidates in first-seen j order, and the
//     edges run in (out_row, kernel_id, in_row) order (write_map,
//     relation_views_detail.h:52-82).  The first j of a candidate is found
//     without a candidate table: cand(in, k) = cand(in', k') exactly when
//     offset[k] - offset[k'] is a multiple of the stride on every axis and
//     coord(in') = coord(in) + (offset[k] - offset[k']) / stride, so its
//     representative is the minimum of first_row(coord') * K + k' over those
//     k' (k itself included), looked up in the input rows' block table.  A
//     flag, a scan and a scatter then place the representatives.  That
//     edge order is a stable sort by
//     out_row of the j's listed kernel-major (t = k * rows + in), which
//     already runs in (kernel_id, in_row) order.  A repeated input coordinate
//     gives a second edge for the same (out_row, kernel_id); the edge pass
//     flags that in the status word, since the dense out_in_map view cannot
//     hold it.

namespace lattice {
namespace {

__device__ inline int4 candidate_of(const int32_t* coords, int in, int k, const KernelGeometry& g,
                                    int64_t* x, int64_t* y, int64_t* z) {
    const int4 c = load_coord(coords, in);
    const Int3 off = offset_of(k, g);
    *x = static_cast<int64_t>(c.y) * g.stride.x + off.x - g.padding.x;
    *y = static_cast<int64_t>(c.z) * g.stride.y + off.y - g.padding.y;
    *z = static_cast<int64_t>(c.w) * g.stride.z + off.z - g.padding.z;
    return make_int4(c.x, static_cast<int>(*x), static_cast<int>(*y), static_cast<int>(*z));
}

__global__ void __launch_bounds__(kThreads)
expand_direct(const int32_t* __restrict__ coords, int rows, const int32_t* __restrict__ active_rows,
              KernelGeometry g, lattice_relation_outputs out) {
    const int K = g.volume;
    const long long cap = static_cast<long long>(rows) * K;
    const int total = min(max(*active_rows, 0), rows) * K;
    int4* oc = reinterpret_cast<int4*>(out.out_coords);
    for (long long j = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; j <= cap;
         j += static_cast<long long>(gridDim.x) * kThreads) {
        if (j == cap) {
            out.row_offsets[cap] = total;
            out.counts[0] = total;
            out.counts[1] = total;
            continue;
        }
        if (j < total) {
            const int in = static_cast<int>(j / K);
            const int k = static_cast<int>(j - static_cast<long long>(in) * K);
            int64_t x, y, z;
            oc[j] = candidate_of(coords, in, k, g, &x, &y, &z);
            out.in_rows[j] = in;
            out.out_rows[j] = static_cast<int32_t>(j);
            out.kernel_ids[j] = k;
            out.row_offsets[j] = static_cast<int32_t>(j);
        } else {
            oc[j] = make_int4(0, 0, 0, 0);
            out.in_rows[j] = 0;
            out.out_rows[j] = 0;
            out.kernel_ids[j] = 0;
            out.row_offsets[j] = total;
        }
    }
}

__device__ inline int axis_offset(int i, int size, int dilation) {
    return (i - ((size & 1) ? size / 2 : 0)) * dilation;
}

// First input row of a coordinate, or -1.
__device__ inline int first_row(const BlockTable& table, int b, int64_t x, int64_t y, int64_t z) {
    TableKey block_key;
    int octant;
    if (!block_of(b, x, y, z, &block_key, &octant)) return -1;
    return table.find(block_key, octant);
}

// reps[j] = first candidate index j' with cand(j') == cand(j) (-1 for
// inactive rows); flags[j] = reps[j]
// == j.  Lanes of one input row share its neighbourhood's bucket lines.
__global__ void __launch_bounds__(kThreads)
resolve_candidates(BlockTable table, const int32_t* __restrict__ coords, int rows,
                   const int32_t* __restrict__ active_rows, KernelGeometry g,
                   int32_t* __restrict__ reps, int32_t* __restrict__ flags) {
    const int K = g.volume;
    const int cap = rows * K;
    const int total = min(max(*active_rows, 0), rows) * K;
    const int yz = g.size.y * g.size.z;
    for (int j = blockIdx.x * kThreads + threadIdx.x; j < cap; j += gridDim.x * kThreads) {
        int rep = -1;
        if (j < total) {
            const int in = j / K;
            const int k = j - in * K;
            {
                const int4 src = load_coord(coords, in);
                const int ix = k / yz;
                const int iy = (k - ix * yz) / g.size.z;
                const int iz = k - ix * yz - iy * g.size.z;
                const int ox = axis_offset(ix, g.size.x, g.dilation.x);
                const int oy = axis_offset(iy, g.size.y, g.dilation.y);
                const int oz = axis_offset(iz, g.size.z, g.dilation.z);
                rep = j;
                for (int ax = 0; ax < g.size.x; ++ax) {
                    const int dx = ox - axis_offset(ax, g.size.x, g.dilation.x);
                    if (dx % g.stride.x != 0) continue;
                    for (int ay = 0; ay < g.size.y; ++ay) {
                        const int dy = oy - axis_offset(ay, g.size.y, g.dilation.y);
                        if (dy % g.stride.y != 0) continue;
                        for (int az = 0; az < g.size.z; ++az) {
                            const int dz = oz - axis_offset(az, g.size.z, g.dilation.z);
                            if (dz % g.stride.z != 0) continue;
                            const int r = first_row(table, src.x, static_cast<int64_t>(src.y) + dx / g.stride.x,
                                                    static_cast<int64_t>(src.z) + dy / g.stride.y,
                                                    static_cast<int64_t>(src.w) + dz / g.stride.z);
                            if (r >= 0) rep = min(rep, r * K + ax * yz + ay * g.size.z + az);
                        }
                    }
                }
            }
        }
        reps[j] = rep;
        flags[j] = rep == j ? 1 : 0;
    }
}

constexpr int kResolveRows = 64;
constexpr int kResolveCells = 64;
constexpr int kMaxRowMembers = 8;  // candidate list slots per representative

// Exclusive scan of an (x, y) pair over the block's threads; the block
// total comes back through `total`.  Every thread of the block calls it.
__device__ inline int2 block_scan_pair(int2 v, int2* total) {
    __shared__ int2 wave_sums[kThreads / kWave];
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    int2 incl = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int ux = __shfl_up(incl.x, d, kWave);
        const int uy = __shfl_up(incl.y, d, kWave);
        if (lane >= d) {
            incl.x += ux;
            incl.y += uy;
        }
    }
    if (lane == kWave - 1) wave_sums[wave] = incl;
    __syncthreads();
    int2 base = make_int2(0, 0), tot = make_int2(0, 0);
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) {
        const int2 ws = wave_sums[w];
        if (w < wave) {
            base.x += ws.x;
            base.y += ws.y;
        }
        tot.x += ws.x;
        tot.y += ws.y;
    }
    __syncthreads();
    *total = tot;
    return make_int2(base.x + incl.x - v.x, base.y + incl.y - v.y);
}

// Exclusive scan of the per-tile (representatives, edges) totals in one
// block; counts[1] receives the number of representatives.
__global__ void __launch_bounds__(kThreads)
scan_tile_pairs(int32_t* __restrict__ tile_firsts, int32_t* __restrict__ tile_edges, int tiles,
                int32_t* __restrict__ counts) {
    int2 carry = make_int2(0, 0);
    for (int c = 0; c < tiles; c += kThreads) {
        const int i = c + threadIdx.x;
        const int2 v = i < tiles ? make_int2(tile_firsts[i], tile_edges[i]) : make_int2(0, 0);
        int2 tot;
        const int2 pre = block_scan_pair(v, &tot);
        if (i < tiles) {
            tile_firsts[i] = carry.x + pre.x;
            tile_edges[i] = carry.y + pre.y;
        }
        carry.x += tot.x;
        carry.y += tot.y;
    }
    if (threadIdx.x == 0) counts[1] = carry.x;
}

// positions[j] (output row of a representative) and edge_offsets[j] (its
// first edge): the tile's scanned base plus the in-tile exclusive prefix
// of flags and sizes, in j order.
__global__ void __launch_bounds__(kThreads)
finalize_tiles(const int32_t* __restrict__ flags, const int32_t* __restrict__ sizes,
               const int32_t* __restrict__ tile_firsts, const int32_t* __restrict__ tile_edges, int rows, int K,
               int32_t* __restrict__ positions, int32_t* __restrict__ edge_offsets) {
    const int tiles = (rows + kResolveRows - 1) / kResolveRows;
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const int j0 = tile * kResolveRows * K;
        const int n = min(kResolveRows, rows - tile * kResolveRows) * K;
        int2 base = make_int2(tile_firsts[tile], tile_edges[tile]);
        for (int c = 0; c < n; c += kThreads) {
            const int i = c + threadIdx.x;
            const int2 v = i < n ? make_int2(flags[j0 + i], sizes[j0 + i]) : make_int2(0, 0);
            int2 tot;
            const int2 pre = block_scan_pair(v, &tot);
            if (i < n) {
                positions[j0 + i] = base.x + pre.x;
                edge_offsets[j0 + i] = base.y + pre.y;
            }
            base.x += tot.x;
            base.y += tot.y;
        }
    }
}


// resolve_candidates for a tile of kResolveRows input rows at a time: the
// block first looks up every input coordinate a candidate of the tile can
// coincide with, coord(in) + d for d in [-R, R] per axis (R = floor(offset
// extent / stride)), into LDS, one lane per (row, d), so a wave's lanes probe
// neighbouring lines; then each (row, k) lane takes the minimum over its
// preimages from LDS.  Used when the neighbourhood has at most
// kResolveCells cells.  kK3S2 is the instance for kernel 3, stride 2,
// dilation 1 on every axis (the decoder's upsampling): its sizes, period,
// step and reach are compile-time constants, so the member walks unroll and
// the divisions by K and the period become shifts and multiplies.
template <bool kK3S2>
__global__ void __launch_bounds__(kThreads)
resolve_candidates_tiled(BlockTable table, const int32_t* __restrict__ coords, int rows,
                         const int32_t* __restrict__ active_rows, KernelGeometry g, Int3 reach, Int3 period,
                         Int3 step, int32_t* status,
                         int32_t* __restrict__ reps, int32_t* __restrict__ flags, int32_t* __restrict__ sizes,
                         int32_t* __restrict__ ranks, int32_t* __restrict__ tile_firsts,
                         int32_t* __restrict__ tile_edges, int32_t* __restrict__ member_ids, int max_members) {
    if constexpr (kK3S2) {
        g.size = Int3{3, 3, 3};
        g.volume = 27;
        reach = Int3{1, 1, 1};
        period = Int3{2, 2, 2};
        step = Int3{1, 1, 1};
        max_members = kMaxRowMembers;
    }
    __shared__ int32_t found[kResolveRows * kResolveCells];
    const int K = g.volume;
    const int active = min(max(*active_rows, 0), rows);
    const int dx_n = 2 * reach.x + 1, dy_n = 2 * reach.y + 1, dz_n = 2 * reach.z + 1;
    const int cells = dx_n * dy_n * dz_n;
    const bool windowed = reach.x == 1 && reach.y == 1 && reach.z == 1;
    const int yz = g.size.y * g.size.z;
    const int tiles = (rows + kResolveRows - 1) / kResolveRows;
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const int r0 = tile * kResolveRows;
        const int tile_rows = min(kResolveRows, rows - r0);
        if (windowed) {
            // Unit reach (3x3x3 cells): the cells of a row lie in the 2x2x2
            // blocks floor((v - 1) / 2) .. +1 per axis, so one lane per
            // (row, block) reads that block's bucket once and places its
            // octants' rows: octant o of block j is window index 2j + o,
            // cell 2j + o - 1 + (v & 1) per axis when that lies in 0..2.
            for (int i = threadIdx.x; i < tile_rows * 8; i += kThreads) {
                const int lr = i >> 3;
                const int jb = i & 7;
                const int row = r0 + lr;
                if (row >= active) continue;
                const int4 c = load_coord(coords, row);
                const int jx = jb >> 2, jy = (jb >> 1) & 1, jz = jb & 1;
                const TableKey key = table_key(c.x, ((static_cast<int64_t>(c.y) - 1) >> 1) + jx,
                                               ((static_cast<int64_t>(c.z) - 1) >> 1) + jy,
                                               ((static_cast<int64_t>(c.w) - 1) >> 1) + jz);
                // key and rows of a slot are read together
                uint32_t slot = static_cast<uint32_t>(key.hash) & table.mask;
                int32_t raw[8];
                bool hit = false;
                for (uint32_t probe = 0; probe <= table.mask; ++probe) {
                    const unsigned long long k = table.buckets[slot].key;
#pragma unroll
                    for (int o = 0; o < 8; ++o) raw[o] = table.buckets[slot].rows[o];
                    if (table.holds(k, key)) {
                        hit = true;
                        break;
                    }
                    if (k == kEmptyKey) break;
                    slot = (slot + 1) & table.mask;
                }
                if (!hit) {
#pragma unroll
                    for (int o = 0; o < 8; ++o) raw[o] = 0;
                }
                const int sx = (c.y & 1) - 1, sy = (c.z & 1) - 1, sz = (c.w & 1) - 1;
                int32_t* f = found + lr * cells;
#pragma unroll
                for (int o = 0; o < 8; ++o) {
                    const int cx = 2 * jx + (o >> 2) + sx;
                    const int cy = 2 * jy + ((o >> 1) & 1) + sy;
                    const int cz = 2 * jz + (o & 1) + sz;
                    if (cx >= 0 && cx <= 2 && cy >= 0 && cy <= 2 && cz >= 0 && cz <= 2) {
                        const int r = bucket_row(raw[o]);
                        f[(cx * 3 + cy) * 3 + cz] = r;
                        // A later row with the coordinate of an earlier one
                        // gives a second edge for some (out_row, kernel_id).
                        if (cx == 1 && cy == 1 && cz == 1 && r >= 0 && r != row) {
                            atomicOr(status, LATTICE_STATUS_REPEATED_EDGE);
                        }
                    }
                }
            }
        }
        for (int i = threadIdx.x; !windowed && i < tile_rows * cells; i += kThreads) {
            const int row = r0 + i / cells;
            const int d = i - (i / cells) * cells;
            int r = -1;
            if (row < active) {
                const int ix = d / (dy_n * dz_n);
                const int iy = (d - ix * dy_n * dz_n) / dz_n;
                const int iz = d - ix * dy_n * dz_n - iy * dz_n;
                const int4 c = load_coord(coords, row);
                r = first_row(table, c.x, static_cast<int64_t>(c.y) + ix - reach.x,
                              static_cast<int64_t>(c.z) + iy - reach.y, static_cast<int64_t>(c.w) + iz - reach.z);
                // A later row with the coordinate of an earlier one gives a
                // second edge for some (out_row, kernel_id).
                if (ix == reach.x && iy == reach.y && iz == reach.z && r >= 0 && r != row) {
                    atomicOr(status, LATTICE_STATUS_REPEATED_EDGE);
                }
            }
            found[i] = r;
        }
        __syncthreads();
        int2 mine = make_int2(0, 0);
        for (int i = threadIdx.x; i < tile_rows * K; i += kThreads) {
            const int in = r0 + i / K;
            const int k = i - (i / K) * K;
            const int j = in * K + k;
            int rep = -1;
            int members = 0;  // candidates equal to this one
            int before = 0;   // of those, with a smaller kernel id
            if (in < active) {
                {
                    const int32_t* f = found + (in - r0) * cells;
                    const int ix = k / yz;
                    const int iy = (k - ix * yz) / g.size.z;
                    const int iz = k - ix * yz - iy * g.size.z;
                    // Offsets i' of one axis meet offset i exactly when
                    // i - i' is a multiple of the period; the input cell
                    // then moves by (i - i') / period * step.
                    const int ax0 = ix % period.x, ay0 = iy % period.y, az0 = iz % period.z;
                    const int tx0 = (ix - ax0) / period.x, ty0 = (iy - ay0) / period.y, tz0 = (iz - az0) / period.z;
                    rep = j;
                    for (int ax = ax0, tx = tx0; ax < g.size.x; ax += period.x, --tx) {
                        const int cx = tx * step.x + reach.x;
                        for (int ay = ay0, ty = ty0; ay < g.size.y; ay += period.y, --ty) {
                            const int cy = ty * step.y + reach.y;
                            for (int az = az0, tz = tz0; az < g.size.z; az += period.z, --tz) {
                                const int r = f[(cx * dy_n + cy) * dz_n + tz * step.z + reach.z];
                                const int kk = ax * yz + ay * g.size.z + az;
                                if (r >= 0) {
                                    rep = min(rep, r * K + kk);
                                    ++members;
                                    before += kk < k ? 1 : 0;
                                }
                            }
                        }
                    }
                    // The representative lists its output row's candidates
                    // (in * K + k) in kernel-id order, the row's edge order.
                    if (member_ids != nullptr && rep == j) {
                        int32_t* dst = member_ids + static_cast<long long>(j) * max_members;
                        int m = 0;
                        for (int ax = ax0, tx = tx0; ax < g.size.x; ax += period.x, --tx) {
                            const int cx = tx * step.x + reach.x;
                            for (int ay = ay0, ty = ty0; ay < g.size.y; ay += period.y, --ty) {
                                const int cy = ty * step.y + reach.y;
                                for (int az = az0, tz = tz0; az < g.size.z; az += period.z, --tz) {
                                    const int r = f[(cx * dy_n + cy) * dz_n + tz * step.z + reach.z];
                                    if (r >= 0) dst[m++] = r * K + ax * yz + ay * g.size.z + az;
                                }
                            }
                        }
                    }
                }
            }
            reps[j] = rep;
            flags[j] = rep == j ? 1 : 0;
            sizes[j] = rep == j ? members : 0;
            if (member_ids == nullptr) ranks[j] = before;  // the listed path places edges without ranks
            if (rep == j) {
                mine.x += 1;
                mine.y += members;
            }
        }
        int2 tot;
        block_scan_pair(mine, &tot);
        if (threadIdx.x == 0) {
            tile_firsts[tile] = tot.x;
            tile_edges[tile] = tot.y;
        }
    }
}

// Output coordinates of the representatives at their first-seen position,
// zero tail; keys[t] (t = k * rows + in) = output row of candidate in*K+k,
// -1 for inactive rows (sorted last).  With edge_offsets (the exclusive scan
// of the representatives' group sizes), and while the status word is clear
// (no repeated input coordinate), the edges are written in their final
// (out_row, kernel_id, in_row) order here: out row positions[j] of a
// representative starts at edge_offsets[j]; with member_ids the
// representative writes its row's edges from its candidate list, otherwise
// candidate j is edge edge_offsets[rep] + ranks[j].
template <bool kK3S2>
__global__ void __launch_bounds__(kThreads)
place_candidates(const int32_t* __restrict__ coords, int rows, const int32_t* __restrict__ active_rows,
                 KernelGeometry g, const int32_t* __restrict__ reps, const int32_t* __restrict__ flags,
                 const int32_t* __restrict__ positions, const int32_t* __restrict__ edge_offsets,
                 const int32_t* __restrict__ ranks, const int32_t* __restrict__ sizes,
                 const int32_t* __restrict__ member_ids, lattice_relation_outputs out,
                 int32_t* __restrict__ keys) {
    static_assert(kMaxRowMembers == 8, "a candidate list is two 16-byte words");
    if constexpr (kK3S2) {  // kernel 3, stride 2, dilation 1: constant divisors
        g.size = Int3{3, 3, 3};
        g.stride = Int3{2, 2, 2};
        g.dilation = Int3{1, 1, 1};
        g.volume = 27;
    }
    const int K = g.volume;
    const int cap = rows * K;
    const int total = min(max(*active_rows, 0), rows) * K;
    const int n_out = out.counts[1];
    const bool emit = edge_offsets != nullptr && *out.status == 0;
    const bool listed = emit && member_ids != nullptr;
    int4* oc = reinterpret_cast<int4*>(out.out_coords);
    // Listed placement: the representatives of one wave own one contiguous
    // run of edges (their group sizes are scanned in candidate order), so
    // each representative spreads its list into the wave's LDS run and the
    // wave then writes the run with whole-line stores.
    __shared__ int32_t run_ids[kThreads / kWave][kWave * kMaxRowMembers];
    __shared__ int32_t run_pos[kThreads / kWave][kWave * kMaxRowMembers];
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (emit && blockIdx.x == 0 && threadIdx.x == 0) out.counts[0] = total;
    // every lane of a block runs the same number of iterations (the wave
    // steps below need all 64 lanes)
    for (int base = blockIdx.x * kThreads; base <= cap; base += gridDim.x * kThreads) {
        const int j = base + threadIdx.x;
        bool rep_here = false;
        int e0 = 0, n_here = 0, pos_here = 0;
        int4 lo = make_int4(0, 0, 0, 0), hi = make_int4(0, 0, 0, 0);
        if (j == cap) {
            if (emit) out.row_offsets[cap] = total;
        } else if (j < cap) {
            const int in = j / K;
            const int k = j - in * K;
            const int rep = reps[j];
            const bool first = flags[j] != 0;
            if (first) {
                int64_t x, y, z;
                oc[positions[j]] = candidate_of(coords, in, k, g, &x, &y, &z);
            }
            if (j >= n_out) oc[j] = make_int4(0, 0, 0, 0);
            if (!emit) keys[static_cast<long long>(k) * rows + in] = rep >= 0 ? positions[rep] : -1;
            if (emit) {
                if (j < total && listed) {
                    if (first) {
                        // the list in two 16-byte loads: one memory round trip
                        const int4* ids = reinterpret_cast<const int4*>(
                            member_ids + static_cast<long long>(j) * kMaxRowMembers);
                        lo = ids[0];
                        hi = ids[1];
                        e0 = edge_offsets[j];
                        pos_here = positions[j];
                        n_here = sizes[j];
                        rep_here = true;
                        out.row_offsets[pos_here] = e0;
                    }
                } else if (j < total) {
                    const int e = edge_offsets[rep] + ranks[j];
                    out.in_rows[e] = in;
                    out.out_rows[e] = positions[rep];
                    out.kernel_ids[e] = k;
                    if (first) out.row_offsets[positions[j]] = edge_offsets[j];
                } else {
                    out.in_rows[j] = 0;
                    out.out_rows[j] = 0;
                    out.kernel_ids[j] = 0;
                }
                if (j >= n_out) out.row_offsets[j] = total;
            }
        }
        if (listed) {
            const uint64_t mask = ballot(rep_here);
            if (mask != 0) {
                // the wave's run: from its first representative's offset to
                // its last one's end
                const int first_lane = __builtin_ctzll(mask);
                const int last_lane = 63 - __builtin_clzll(mask);
                const int run0 = __builtin_amdgcn_readlane(e0, first_lane);
                const int run_n = __builtin_amdgcn_readlane(e0 + n_here, last_lane) - run0;
                if (rep_here) {
                    const int id8[kMaxRowMembers] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    const int r = e0 - run0;
#pragma unroll
                    for (int m = 0; m < kMaxRowMembers; ++m) {
                        if (m < n_here) {
                            run_ids[wave][r + m] = id8[m];
                            run_pos[wave][r + m] = pos_here;
                        }
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                for (int t = lane; t < run_n; t += kWave) {
                    const int id = run_ids[wave][t];
                    const int src = id / K;
                    out.in_rows[run0 + t] = src;
                    out.out_rows[run0 + t] = run_pos[wave][t];
                    out.kernel_ids[run0 + t] = id - src * K;
                }
                // the next iteration's stores into the run wait for these reads
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        }
    }
}

// Edge e of the sorted order: t = sorted_index[e] -> (in, k); flags a
// repeated (out_row, kernel_id).
__global__ void __launch_bounds__(kThreads)
emit_sorted_edges(const int32_t* __restrict__ sorted_keys, const int32_t* __restrict__ sorted_index, int rows,
                  int K, const int32_t* __restrict__ active_rows, lattice_relation_outputs out,
                  const int32_t* run_if) {
    if (run_if != nullptr && *run_if == 0) return;
    const int cap = rows * K;
    const int total = min(max(*active_rows, 0), rows) * K;
    if (blockIdx.x == 0 && threadIdx.x == 0) out.counts[0] = total;
    for (int e = blockIdx.x * kThreads + threadIdx.x; e < cap; e += gridDim.x * kThreads) {
        if (e < total) {
            const int t = sorted_index[e];
            const int k = t / rows;
            out.in_rows[e] = t - k * rows;
            out.out_rows[e] = sorted_keys[e];
            out.kernel_ids[e] = k;
            if (e > 0 && sorted_keys[e - 1] == sorted_keys[e] && sorted_index[e - 1] / rows == k) {
                atomicOr(out.status, LATTICE_STATUS_REPEATED_EDGE);
            }
        } else {
            out.in_rows[e] = 0;
            out.out_rows[e] = 0;
            out.kernel_ids[e] = 0;
        }
    }
}

bool direct_expansion(const KernelGeometry& g) {
    // Offset extent per axis: (size - 1) * dilation.
    return g.stride.x > (g.size.x - 1) * g.dilation.x && g.stride.y > (g.size.y - 1) * g.dilation.y &&
           g.stride.z > (g.size.z - 1) * g.dilation.z;
}

// The deduplicating build's shared region: the candidate lists, or the
// ranks, keys, sorted keys and index plus the radix sort's workspace.
size_t expanded_shared_bytes(long long cap) {
    const size_t c = static_cast<size_t>(std::max<long long>(cap, 1));
    const size_t n = aligned_bytes(c * sizeof(int32_t));
    return std::max(aligned_bytes(c * kMaxRowMembers * sizeof(int32_t)),
                    4 * n + radix_sort_workspace_bytes(static_cast<int>(c), 32));
}

size_t expanded_relation_bytes(int rows, int K, bool direct) {
    const long long cap = static_cast<long long>(std::max(rows, 0)) * K;
    size_t bytes = group_view_bytes(static_cast<int>(cap)) + 4096;
    if (direct) return bytes;
    const size_t n = aligned_bytes(static_cast<size_t>(std::max<long long>(cap, 1)) * sizeof(int32_t));
    const size_t tiles = static_cast<size_t>(std::max(rows, 0)) / kResolveRows + 1;
    bytes += block_table_bytes(std::max(rows, 0)) + 5 * n + expanded_shared_bytes(cap) +
             2 * aligned_bytes(tiles * sizeof(int32_t)) + aligned_bytes(2 * sizeof(int32_t)) +
             scan_workspace_bytes(cap);
    return bytes;
}

int check_expanded_outputs(const lattice_relation_outputs* out, long long cap) {
    LATTICE_REQUIRE(out != nullptr, "relation outputs are required.");
    LATTICE_REQUIRE(out->row_offsets && out->counts && out->status, "relation output pointers must be non-null.");
    LATTICE_REQUIRE(cap == 0 || (out->in_rows && out->out_rows && out->kernel_ids && out->out_coords),
                    "relation output pointers must be non-null.");
    const bool views = out->in_edge_ids != nullptr || out->kernel_edge_ids != nullptr;
    LATTICE_REQUIRE(!views || (out->in_edge_ids && out->kernel_edge_ids && out->in_row_offsets &&
                               out->kernel_row_offsets),
                    "grouped view outputs must be all set or all null.");
    return LATTICE_OK;
}

__global__ void clear_status(int32_t* status) { status[0] = 0; }

int build_expanded_relation(const int32_t* coords, int rows, const int32_t* active_rows, const KernelGeometry& g,
                            bool direct, const lattice_relation_outputs* out, void* workspace,
                            size_t workspace_bytes, hipStream_t stream) {
    const int K = g.volume;
    LATTICE_REQUIRE(rows >= 0, "coords must have shape (N, 4).");
    LATTICE_REQUIRE(rows == 0 || coords != nullptr, "coords must be non-null.");
    LATTICE_REQUIRE(active_rows != nullptr, "active_rows must be non-null.");
    LATTICE_REQUIRE(static_cast<long long>(rows) * K < (1ll << 30), "relation capacity rows * K exceeds 2^30.");
    int rc = check_expanded_outputs(out, static_cast<long long>(rows) * K);
    if (rc != LATTICE_OK) return rc;
    LATTICE_REQUIRE(workspace_bytes >= expanded_relation_bytes(rows, K, direct), "relation workspace too small.");
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    const int cap = rows * K;
    if (direct || cap == 0) {
        // (the deduplicating path clears the status word in its table clear)
        clear_status<<<1, 1, 0, stream>>>(out->status);
        LATTICE_LAUNCH_CHECK();
    }
    if (direct) {
        expand_direct<<<grid_for(static_cast<long long>(cap) + 1, kThreads, 1u << 16), kThreads, 0, stream>>>(
            coords, rows, active_rows, g, *out);
        LATTICE_LAUNCH_CHECK();
    } else if (cap == 0) {
        rc = fill_i32(out->row_offsets, 1, 0, stream);
        if (rc != LATTICE_OK) return rc;
        rc = fill_i32(out->counts, 2, 0, stream);
        if (rc != LATTICE_OK) return rc;
    } else {
        const Prologue prologue{out->status, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr};
        BlockTable table;
        rc = build_block_table(coords, rows, active_rows, prologue, ws, stream, &table);
        if (rc != LATTICE_OK) return rc;
        int32_t* reps = ws.take<int32_t>(cap);
        int32_t* flags = ws.take<int32_t>(cap);
        int32_t* positions = ws.take<int32_t>(cap);
        int32_t* sizes = ws.take<int32_t>(cap);
        int32_t* edge_offsets = ws.take<int32_t>(cap);
        // One region holds either the representatives' candidate lists
        // (read by place_candidates only while the status word is clear) or
        // the fallback's ranks, keys and sort buffers (used only when it is
        // set, or when the lists are not built), so they share it.
        const size_t region_bytes = expanded_shared_bytes(cap);
        char* region = ws.take<char>(region_bytes);
        Workspace shared{region, region ? region_bytes : 0};
        int32_t* member_ids = reinterpret_cast<int32_t*>(region);
        int32_t* ranks = shared.take<int32_t>(cap);
        int32_t* keys = shared.take<int32_t>(cap);
        int32_t* sorted_keys = shared.take<int32_t>(cap);
        int32_t* sorted_index = shared.take<int32_t>(cap);
        const int resolve_tiles = (rows + kResolveRows - 1) / kResolveRows;
        int32_t* tile_firsts = ws.take<int32_t>(resolve_tiles);
        int32_t* tile_edges = ws.take<int32_t>(resolve_tiles);
        LATTICE_REQUIRE(reps && flags && positions && keys && sorted_keys && sorted_index && sizes && ranks &&
                            edge_offsets && tile_firsts && tile_edges,
                        "relation workspace too small.");
        const unsigned grid = grid_for(cap, kThreads, 1u << 14);
        const Int3 reach{(g.size.x - 1) * g.dilation.x / g.stride.x, (g.size.y - 1) * g.dilation.y / g.stride.y,
                         (g.size.z - 1) * g.dilation.z / g.stride.z};
        const long long cells = (2ll * reach.x + 1) * (2ll * reach.y + 1) * (2ll * reach.z + 1);
        // The tiled resolve also ranks every candidate inside its output
        // row, so the edges are placed directly; the stable sort then runs
        // only when the status word reports a repeated input coordinate.  The general resolve always sorts.
        const bool tiled = cells <= kResolveCells;
        const auto gcd = [](int a, int b) {
            while (b != 0) {
                const int t = a % b;
                a = b;
                b = t;
            }
            return a;
        };
        const Int3 period{g.stride.x / gcd(g.stride.x, g.dilation.x), g.stride.y / gcd(g.stride.y, g.dilation.y),
                          g.stride.z / gcd(g.stride.z, g.dilation.z)};
        const Int3 step{g.dilation.x / gcd(g.stride.x, g.dilation.x), g.dilation.y / gcd(g.stride.y, g.dilation.y),
                        g.dilation.z / gcd(g.stride.z, g.dilation.z)};
        // Candidates of one output row: the offsets of each axis that meet
        // an offset i step by the period, at most ceil(size / period) of them.
        const int row_members = ((g.size.x + period.x - 1) / period.x) * ((g.size.y + period.y - 1) / period.y) *
                                ((g.size.z + period.z - 1) / period.z);
        // (place_candidates reads a list as two 16-byte words: a workspace that
        // is not 16-byte aligned takes the ranked placement instead)
        const bool k3s2 = g.size.x == 3 && g.size.y == 3 && g.size.z == 3 && g.stride.x == 2 && g.stride.y == 2 &&
                          g.stride.z == 2 && g.dilation.x == 1 && g.dilation.y == 1 && g.dilation.z == 1;
        const bool listed = tiled && member_ids != nullptr && row_members <= kMaxRowMembers &&
                            (reinterpret_cast<uintptr_t>(member_ids) & 15) == 0;
        if (tiled) {
            const int tiles = (rows + kResolveRows - 1) / kResolveRows;
            const auto kernel = k3s2 ? resolve_candidates_tiled<true> : resolve_candidates_tiled<false>;
            kernel<<<static_cast<unsigned>(std::min(tiles, 1 << 16)), kThreads, 0, stream>>>(
                table, coords, rows, active_rows, g, reach, period, step, out->status, reps, flags, sizes, ranks,
                tile_firsts, tile_edges, listed ? member_ids : nullptr, kMaxRowMembers);
        } else {
            resolve_candidates<<<grid, kThreads, 0, stream>>>(table, coords, rows, active_rows, g, reps,
                                                              flags);
        }
        LATTICE_LAUNCH_CHECK();
        if (tiled) {
            const int tiles = (rows + kResolveRows - 1) / kResolveRows;
            scan_tile_pairs<<<1, kThreads, 0, stream>>>(tile_firsts, tile_edges, tiles, out->counts);
            LATTICE_LAUNCH_CHECK();
            finalize_tiles<<<static_cast<unsigned>(std::min(tiles, 1 << 16)), kThreads, 0, stream>>>(
                flags, sizes, tile_firsts, tile_edges, rows, K, positions, edge_offsets);
            LATTICE_LAUNCH_CHECK();
        } else {
            rc = exclusive_scan(flags, positions, cap, out->counts + 1, ws, stream);
            if (rc != LATTICE_OK) return rc;
        }
        const auto place = k3s2 ? place_candidates<true> : place_candidates<false>;
        place<<<grid_for(static_cast<long long>(cap) + 1, kThreads, 1u << 14), kThreads, 0, stream>>>(
            coords, rows, active_rows, g, reps, flags, positions, tiled ? edge_offsets : nullptr, ranks, sizes,
            listed ? member_ids : nullptr, *out, keys);
        LATTICE_LAUNCH_CHECK();
        const int32_t* run_if = tiled ? out->status : nullptr;
        SortKeys sk{keys, 1, nullptr, cap, false};
        sk.run_if = run_if;
        rc = radix_sort_indices(sk, cap, bit_width(cap), sorted_keys, sorted_index, shared, stream);
        if (rc != LATTICE_OK) return rc;
        emit_sorted_edges<<<run_if != nullptr ? std::min(grid, kConditionalGrid) : grid, kThreads, 0, stream>>>(
            sorted_keys, sorted_index, rows, K, active_rows, *out, run_if);
        LATTICE_LAUNCH_CHECK();
        int32_t* tail = ws.take<int32_t>(2);
        LATTICE_REQUIRE(tail, "relation workspace too small.");
        rc = launch_group_offsets(sorted_keys, cap, cap, out->row_offsets, tail, stream, run_if);
        if (rc != LATTICE_OK) return rc;
    }
    if (out->in_edge_ids == nullptr) return LATTICE_OK;
    Workspace views{static_cast<char*>(workspace), workspace_bytes};
    return build_group_views(out->in_rows, out->kernel_ids, out->counts, cap, rows, K, out->in_row_offsets,
                             out->in_edge_ids, out->kernel_row_offsets, out->kernel_edge_ids, views, stream);
}

}  // namespace
}  // namespace lattice

extern "C" size_t lattice_hip_expanded_relation_workspace_bytes(int rows, const int kernel_size[3],
                                                                const int stride[3], const int dilation[3],
                                                                int generative) {
    const int zero[3] = {0, 0, 0};
    if (validate_geometry(kernel_size, stride, zero, dilation) != LATTICE_OK) return 0;
    const KernelGeometry g = make_geometry(kernel_size, stride, zero, dilation);
    return expanded_relation_bytes(rows, g.volume, generative != 0 || direct_expansion(g));
}

extern "C" int lattice_hip_build_generative_relation(const int32_t* coords, int rows, const int32_t* active_rows,
                                                     const int kernel_size[3], const int stride[3],
                                                     const lattice_relation_outputs* out, void* workspace,
                                                     size_t workspace_bytes, void* stream_ptr) {
    const int zero[3] = {0, 0, 0};
    const int one[3] = {1, 1, 1};
    int rc = validate_geometry(kernel_size, stride, zero, one);
    if (rc != LATTICE_OK) return rc;
    return build_expanded_relation(coords, rows, active_rows, make_geometry(kernel_size, stride, zero, one), true,
                                   out, workspace, workspace_bytes, as_stream(stream_ptr));
}

extern "C" int lattice_hip_build_transposed_kernel_relation(const int32_t* coords, int rows,
                                                            const int32_t* active_rows, const int kernel_size[3],
                                                            const int stride[3], const int padding[3],
                                                            const int dilation[3],
                                                            const lattice_relation_outputs* out, void* workspace,
                                                            size_t workspace_bytes, void* stream_ptr) {
    int rc = validate_geometry(kernel_size, stride, padding, dilation);
    if (rc != LATTICE_OK) return rc;
    const KernelGeometry g = make_geometry(kernel_size, stride, padding, dilation);
    return build_expanded_relation(coords, rows, active_rows, g, direct_expansion(g), out, workspace,
                                   workspace_bytes, as_stream(stream_ptr));
}

extern "C" size_t lattice_hip_group_by_key_workspace_bytes(int n) { return group_view_bytes(std::max(n, 0)); }

extern "C" int lattice_hip_group_by_key(const int32_t* keys, int n, const int32_t* count, int groups,
                                       int32_t* offsets, int32_t* ids, void* workspace, size_t workspace_bytes,
                                       void* stream_ptr) {
    LATTICE_REQUIRE(n >= 0 && groups >= 0, "group_by_key needs non-negative sizes.");
    LATTICE_REQUIRE(offsets && (n == 0 || (keys && ids)), "group_by_key pointers must be non-null.");
    LATTICE_REQUIRE(workspace_bytes >= lattice_hip_group_by_key_workspace_bytes(n),
                    "group_by_key workspace too small.");
    Workspace ws{static_cast<char*>(workspace), workspace_bytes};
    return build_group_view(keys, count, n, groups, offsets, ids, ws, as_stream(stream_ptr));
}
