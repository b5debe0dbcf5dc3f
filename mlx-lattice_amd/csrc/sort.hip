// Stable LSD radix sort of (key, index) pairs with digits of up to 11 bits
// (reduce-then-scan): a key of b bits takes ceil(b / 11) passes of equal
// digit width (27 bits: 3 x 9, 20 bits: 2 x 10).  Per digit pass:
//   1. sort_count: each tile of 2048 items counts its digits in LDS, writes
//      them digit-major, count[d * tiles + tile], and adds them to the
//      per-digit totals;
//   2. sort_scan: the count matrix becomes the output offset of every
//      (digit, tile), one block per 16 digit rows;
//   3. sort_scatter: each tile ranks its items stably per digit in LDS and
//      scatters them to offset + rank.
// A 27-bit row mask sorts in 3 passes (10 launches with the one fill of the
// totals); no block waits on another.

#include <hip/hip_runtime.h>

#include <algorithm>

#include "scan.h"
#include "sort.h"

namespace lattice {
namespace {

constexpr int kSortThreads = 1024;  // 16 waves: short per-wave rank chains
constexpr int kSortItems = 2;                          // per thread
constexpr int kSortTile = kSortThreads * kSortItems;  // items per tile
constexpr int kMaxRadixBits = 11;
constexpr int kDigits = 1 << kMaxRadixBits;  // digit slots of the widest pass
constexpr int kSortWaves = kSortThreads / kWave;

struct PassPlan {
    int shift;
    int bits;
    int rows;  // digit rows of the count matrix: 2^bits, at least kScanRows
};

// Items of one pass: pass 0 reads the source keys (index = position),
// later passes the previous pass's (key, index) buffers.
struct PassInput {
    SortKeys src;
    const uint32_t* keys;
    const int32_t* index;
    bool first;
};

__device__ inline uint32_t source_key(const SortKeys& k, int i, int valid_count) {
    int v = k.src[static_cast<long long>(i) * k.stride];
    if (k.groups >= 0 && (i >= valid_count || v < 0 || v >= k.groups)) v = k.groups;
    const uint32_t key = static_cast<uint32_t>(v);
    return k.flip_sign ? key ^ 0x80000000u : key;
}

__device__ inline int valid_items(const PassInput& in, int n) {
    return in.first && in.src.count != nullptr ? min(max(in.src.count[0], 0), n) : n;
}

__device__ inline void load_item(const PassInput& in, int i, int valid_src, uint32_t& key, int32_t& index) {
    if (in.first) {
        key = source_key(in.src, i, valid_src);
        index = i;
    } else {
        key = in.keys[i];
        index = in.index[i];
    }
}

// Row stride of the digit x tile count matrix: tiles rounded up to whole
// 16-byte vectors; the block of the last tile zeroes the padding.
__host__ __device__ inline int padded_tiles(int tiles) { return (tiles + 3) & ~3; }

__global__ void __launch_bounds__(kSortThreads)
sort_count(PassInput in, int n, PassPlan plan, int tiles, uint32_t* __restrict__ counts,
           uint32_t* __restrict__ digit_totals) {
    if (in.src.run_if != nullptr && *in.src.run_if == 0) return;
    __shared__ uint32_t hist[kDigits];
    for (int d = threadIdx.x; d < plan.rows; d += kSortThreads) hist[d] = 0;
    __syncthreads();
    const int valid_src = valid_items(in, n);
    const uint32_t digit_mask = (1u << plan.bits) - 1u;
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const int i = blockIdx.x * kSortTile + r * kSortThreads + threadIdx.x;
        if (i < n) {
            uint32_t key;
            int32_t index;
            load_item(in, i, valid_src, key, index);
            atomicAdd(&hist[(key >> plan.shift) & digit_mask], 1u);
        }
    }
    __syncthreads();
    const int stride = padded_tiles(tiles);
    for (int d = threadIdx.x; d < plan.rows; d += kSortThreads) {
        counts[static_cast<long long>(d) * stride + blockIdx.x] = hist[d];
        if (hist[d] != 0) atomicAdd(&digit_totals[d], hist[d]);
        if (static_cast<int>(blockIdx.x) == tiles - 1) {
            for (int p = tiles; p < stride; ++p) counts[static_cast<long long>(d) * stride + p] = 0;
        }
    }
}

// Output offset of every (digit, tile): offset(d, t) = base(d) + sum of
// count(d, t') for t' < t, where base(d) is the number of keys with smaller
// digits (from the digit totals).  kScanRows digit rows per block, one wave
// per kScanRows / kScanWaves rows; rows are read as 16-byte vectors, 256
// tiles per chunk, and every load of a chunk is issued before any value is
// used: the counts were written by blocks on other XCDs, so each dependent
// round trip is long, and this kernel takes two of them for up to 1024
// tiles' worth of rows.
constexpr int kScanBlockThreads = 256;
constexpr int kScanWaves = kScanBlockThreads / kWave;
constexpr int kScanRows = 16;
constexpr int kScanRowsPerWave = kScanRows / kScanWaves;

__device__ inline uint32_t wave_inclusive_scan(uint32_t v, int lane) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t u = __shfl_up(v, off, kWave);
        if (lane >= off) v += u;
    }
    return v;
}

__global__ void __launch_bounds__(kScanBlockThreads)
sort_scan(uint32_t* __restrict__ counts, const uint32_t* __restrict__ digit_totals, int tiles,
          const int32_t* run_if) {
    if (run_if != nullptr && *run_if == 0) return;
    __shared__ uint32_t base[kDigits];
    __shared__ uint32_t wave_sum[kScanWaves];
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    // base(d) for the block's rows: exclusive scan of the digit totals
    // (zero past the pass's digits),
    // kDigits / kScanBlockThreads per thread.
    {
        constexpr int kPer = kDigits / kScanBlockThreads;
        uint32_t vals[kPer];
        uint32_t sum = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            vals[j] = digit_totals[threadIdx.x * kPer + j];
            sum += vals[j];
        }
        const uint32_t incl = wave_inclusive_scan(sum, lane);
        if (lane == kWave - 1) wave_sum[wave] = incl;
        __syncthreads();
        uint32_t run = incl - sum;
        for (int w = 0; w < wave; ++w) run += wave_sum[w];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            base[threadIdx.x * kPer + j] = run;
            run += vals[j];
        }
        __syncthreads();
    }
    const int stride = padded_tiles(tiles);
    const int vecs = stride / 4;  // vectors per row
    const int chunks = (vecs + kWave - 1) / kWave;
    uint4* c4 = reinterpret_cast<uint4*>(counts);
    const int row0 = blockIdx.x * kScanRows + wave * kScanRowsPerWave;
    uint32_t carry[kScanRowsPerWave];
#pragma unroll
    for (int r = 0; r < kScanRowsPerWave; ++r) carry[r] = base[row0 + r];
    for (int c = 0; c < chunks; ++c) {
        const int v = c * kWave + lane;
        uint4 x[kScanRowsPerWave];
#pragma unroll
        for (int r = 0; r < kScanRowsPerWave; ++r) {
            x[r] = v < vecs ? c4[static_cast<long long>(row0 + r) * vecs + v] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < kScanRowsPerWave; ++r) {
            const uint32_t s = x[r].x + x[r].y + x[r].z + x[r].w;
            const uint32_t incl = wave_inclusive_scan(s, lane);
            uint32_t run = carry[r] + incl - s;
            carry[r] += __shfl(incl, kWave - 1, kWave);
            if (v < vecs) {
                uint4 o;
                o.x = run;
                run += x[r].x;
                o.y = run;
                run += x[r].y;
                o.z = run;
                run += x[r].z;
                o.w = run;
                c4[static_cast<long long>(row0 + r) * vecs + v] = o;
            }
        }
    }
}

// Stable ranks of a tile's items per digit, then the scatter.  Wave w
// holds the tile's items w * 128 .. w * 128 + 127 (round r, lane l: item
// w * 128 + r * 64 + l), so index order is (wave, round, lane): each wave
// ranks its rounds in order against its own per-digit running counts (no
// block barrier between rounds; LDS accesses of one wave execute in
// order), then one exclusive scan over the sixteen waves' counts places
// the waves.  Sixteen waves of two rounds rank a 2048-item tile in a
// quarter of the serial steps of four waves of eight rounds (the sorted
// view of 400k masks: 105 -> 90 us); the per-wave counts take 128 KB of
// LDS at 11-bit digits, one block per CU.  The last pass writes the caller's arrays (keys restored to their
// signed form).
__global__ void __launch_bounds__(kSortThreads)
sort_scatter(PassInput in, int n, PassPlan plan, int tiles, const uint32_t* __restrict__ offsets, bool final,
             uint32_t* __restrict__ keys_out, int32_t* __restrict__ idx_out, int32_t* __restrict__ final_keys) {
    if (in.src.run_if != nullptr && *in.src.run_if == 0) return;
    __shared__ uint32_t wave_run[kSortWaves][kDigits];
    __shared__ uint32_t offset[kDigits];
    const int t = threadIdx.x;
    const int wave = t / kWave;
    const int lane = lane_id();
    const int tile = blockIdx.x;
    for (int d = t; d < plan.rows; d += kSortThreads) {
        offset[d] = offsets[static_cast<long long>(d) * padded_tiles(tiles) + tile];
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) wave_run[w][d] = 0;
    }
    __syncthreads();
    const int valid_src = valid_items(in, n);

    uint32_t key[kSortItems];
    int32_t index[kSortItems];
    uint32_t rank[kSortItems];
    int digit[kSortItems];
    const uint32_t digit_mask = (1u << plan.bits) - 1u;
    const int base = tile * kSortTile + wave * (kSortItems * kWave);
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const int i = base + r * kWave + lane;
        digit[r] = -1;
        if (i < n) {
            load_item(in, i, valid_src, key[r], index[r]);
            digit[r] = static_cast<int>((key[r] >> plan.shift) & digit_mask);
        }
    }
    uint32_t* run = wave_run[wave];
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        const bool has = digit[r] >= 0;
        uint64_t peers = ballot(has);
        for (int b = 0; b < plan.bits; ++b) {
            const bool bit = has && ((digit[r] >> b) & 1);
            const uint64_t ones = ballot(bit);
            peers &= bit ? ones : ~ones;
        }
        const uint64_t below = peers & ((1ull << lane) - 1ull);
        if (has) rank[r] = run[digit[r]] + static_cast<uint32_t>(__popcll(below));
        if (has && below == 0) run[digit[r]] += static_cast<uint32_t>(__popcll(peers));
    }
    __syncthreads();
    for (int d = t; d < plan.rows; d += kSortThreads) {
        uint32_t sum = 0;
#pragma unroll
        for (int w = 0; w < kSortWaves; ++w) {
            const uint32_t c = wave_run[w][d];
            wave_run[w][d] = sum;
            sum += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kSortItems; ++r) {
        if (digit[r] < 0) continue;
        const uint32_t pos = offset[digit[r]] + run[digit[r]] + rank[r];
        idx_out[pos] = index[r];
        if (!final) {
            keys_out[pos] = key[r];
        } else if (final_keys != nullptr) {
            final_keys[pos] = static_cast<int32_t>(in.src.flip_sign ? key[r] ^ 0x80000000u : key[r]);
        }
    }
}

int pass_count(int end_bit) { return (end_bit + kMaxRadixBits - 1) / kMaxRadixBits; }

// Pass p of `passes` over end_bit bits: equal widths, the remainder spread
// over the first passes.
PassPlan pass_plan(int p, int passes, int end_bit) {
    const int base = end_bit / passes, extra = end_bit % passes;
    const int shift = p * base + std::min(p, extra);
    const int bits = base + (p < extra ? 1 : 0);
    return PassPlan{shift, bits, std::max(1 << bits, kScanRows)};
}

// Digit rows of the count matrix for an end_bit sort: those of its widest
// pass (the first; pass_plan spreads the remainder bits first).
int count_rows(int end_bit) {
    end_bit = std::min(std::max(end_bit, 1), 32);
    return pass_plan(0, pass_count(end_bit), end_bit).rows;
}

}  // namespace

size_t radix_sort_workspace_bytes(int n, int end_bit) {
    const size_t items = static_cast<size_t>(std::max(n, 1));
    const size_t tiles = (items + kSortTile - 1) / kSortTile;
    size_t bytes = 4 * aligned_bytes(items * sizeof(uint32_t));  // two (key, index) buffers
    bytes += aligned_bytes(static_cast<size_t>(padded_tiles(static_cast<int>(tiles))) * count_rows(end_bit) *
                           sizeof(uint32_t));  // digit x tile counts
    bytes += aligned_bytes(4 * kDigits * sizeof(uint32_t));  // digit totals of up to 4 passes
    return bytes + 256;
}

int radix_sort_indices(const SortKeys& keys, int n, int end_bit, int32_t* sorted_keys, int32_t* sorted_index,
                       Workspace& ws, hipStream_t stream) {
    LATTICE_REQUIRE(end_bit >= 1 && end_bit <= 32, "radix sort end_bit must be in [1, 32].");
    if (n <= 0) return LATTICE_OK;
    const int passes = pass_count(end_bit);
    const int tiles = (n + kSortTile - 1) / kSortTile;
    uint32_t* key_buf[2] = {ws.take<uint32_t>(n), ws.take<uint32_t>(n)};
    int32_t* idx_buf[2] = {ws.take<int32_t>(n), ws.take<int32_t>(n)};
    uint32_t* counts = ws.take<uint32_t>(static_cast<size_t>(padded_tiles(tiles)) * count_rows(end_bit));
    uint32_t* totals = ws.take<uint32_t>(static_cast<size_t>(passes) * kDigits);
    LATTICE_REQUIRE(key_buf[0] && key_buf[1] && idx_buf[0] && idx_buf[1] && counts && totals,
                    "radix sort workspace too small.");
    int rc = fill_i32(reinterpret_cast<int*>(totals), static_cast<long long>(passes) * kDigits, 0, stream);
    if (rc != LATTICE_OK) return rc;
    for (int p = 0; p < passes; ++p) {
        const PassPlan plan = pass_plan(p, passes, end_bit);
        const bool final = p == passes - 1;
        const int in = (p + 1) % 2;  // buffers written by pass p - 1
        const int out = p % 2;
        const PassInput input{keys, p == 0 ? nullptr : key_buf[in], p == 0 ? nullptr : idx_buf[in], p == 0};
        uint32_t* pass_totals = totals + static_cast<size_t>(p) * kDigits;
        sort_count<<<tiles, kSortThreads, 0, stream>>>(input, n, plan, tiles, counts, pass_totals);
        LATTICE_LAUNCH_CHECK();
        sort_scan<<<plan.rows / kScanRows, kScanBlockThreads, 0, stream>>>(counts, pass_totals, tiles, keys.run_if);
        LATTICE_LAUNCH_CHECK();
        sort_scatter<<<tiles, kSortThreads, 0, stream>>>(input, n, plan, tiles, counts, final,
                                                          final ? nullptr : key_buf[out],
                                                          final ? sorted_index : idx_buf[out],
                                                          final ? sorted_keys : nullptr);
        LATTICE_LAUNCH_CHECK();
    }
    return LATTICE_OK;
}

}  // namespace lattice
