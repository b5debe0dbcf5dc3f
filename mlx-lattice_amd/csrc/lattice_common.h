// Shared helpers of the gfx950 sparse-convolution library: error plumbing,
// launch helpers, wavefront intrinsics, the packed 64-bit coordinate key and
// the open-addressing hash probe.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <climits>
#include <cstdint>
#include <string>

#include "lattice_hip.h"

namespace lattice {

// ---------------------------------------------------------------- errors --

void set_error(const std::string& message);

#define LATTICE_REQUIRE(cond, msg)                                   \
    do {                                                             \
        if (!(cond)) {                                               \
            ::lattice::set_error(msg);                               \
            return LATTICE_ERROR_INVALID_ARGUMENT;                   \
        }                                                            \
    } while (0)

#define LATTICE_HIP_TRY(expr)                                        \
    do {                                                             \
        hipError_t lattice_err_ = (expr);                            \
        if (lattice_err_ != hipSuccess) {                            \
            ::lattice::set_error(std::string("HIP error: ") +        \
                                 hipGetErrorString(lattice_err_) +   \
                                 " at " #expr);                      \
            return LATTICE_ERROR_HIP;                                \
        }                                                            \
    } while (0)

#define LATTICE_LAUNCH_CHECK() LATTICE_HIP_TRY(hipGetLastError())

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

inline unsigned grid_for(long long work, int per_block, unsigned cap = 1u << 20) {
    long long blocks = (work + per_block - 1) / per_block;
    if (blocks < 1) blocks = 1;
    if (blocks > cap) blocks = cap;
    return static_cast<unsigned>(blocks);
}

// Bump allocator over a caller workspace; every carve is 256-byte aligned.
struct Workspace {
    char* base;
    size_t size;
    size_t used = 0;
    template <typename T>
    T* take(size_t count) {
        size_t bytes = (count * sizeof(T) + 255) & ~size_t(255);
        if (used + bytes > size) return nullptr;
        T* out = reinterpret_cast<T*>(base + used);
        used += bytes;
        return out;
    }
};

inline size_t aligned_bytes(size_t bytes) { return (bytes + 255) & ~size_t(255); }

// ------------------------------------------------------- wave intrinsics --

constexpr int kWave = 64;

__device__ inline int lane_id() {
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0));
}

// Number of set bits of `mask` held by lanes below the calling lane.
__device__ inline int lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

__device__ inline uint64_t ballot(bool pred) { return __ballot(pred); }

// ------------------------------------------------------- coordinate keys --
//
// A table slot holds one 64-bit key word, in one of two forms.
//
//  * Packed (the fast form): batch << 54 | (x + 2^17) << 36 | (y + 2^17) << 18
//    | (z + 2^17).  Injective over batch in [0, 1022] and x, y, z in
//    [-2^17, 2^17), so equal words mean equal keys.
//  * Wide (every other key, any int32 batch and any int64 axis value):
//    0x3ff << 54 | tag << 32 | claim_row.  The batch field 1023 never occurs
//    in a packed word, so the two forms never compare equal.  `tag` is 22
//    bits of a hash of the full key and `claim_row` is the row whose insert
//    claimed the slot.  Equal tags do not prove equal keys: the key of the
//    claiming row is recomputed from the table's immutable source rows (the
//    input coordinates, or the points) and compared in full.  The source rows
//    are never written during a build, so this comparison needs no ordering
//    with the claiming thread.
//
// The all-ones word (wide form, claim row 0xffffffff, never a real row)
// marks an empty slot.  Keys of one build mix both forms freely; a table
// keyed only by packed words behaves exactly as a packed-only table.

constexpr uint64_t kEmptyKey = ~0ull;
constexpr uint64_t kWideMark = 0x3ffull << 54;
constexpr int64_t kAxisBias = 131072;     // 2^17
constexpr int64_t kAxisSpan = 262144;     // 2^18

__host__ __device__ inline bool pack_key(int64_t b, int64_t x, int64_t y, int64_t z,
                                         uint64_t* key) {
    uint64_t ux = static_cast<uint64_t>(x + kAxisBias);
    uint64_t uy = static_cast<uint64_t>(y + kAxisBias);
    uint64_t uz = static_cast<uint64_t>(z + kAxisBias);
    bool ok = b >= 0 && b <= LATTICE_MAX_BATCH && ux < uint64_t(kAxisSpan) &&
              uy < uint64_t(kAxisSpan) && uz < uint64_t(kAxisSpan);
    *key = (static_cast<uint64_t>(b) << 54) | (ux << 36) | (uy << 18) | uz;
    return ok;
}

// 64-bit finaliser (MurmurHash3 fmix64): spreads the structured key bits.
__host__ __device__ inline uint64_t mix64(uint64_t k) {
    k ^= k >> 33;
    k *= 0xff51afd7ed558ccdull;
    k ^= k >> 33;
    k *= 0xc4ceb9fe1a85ec53ull;
    k ^= k >> 33;
    return k;
}

// Full key: batch and three int64 axis values.
struct FullKey {
    int64_t b, x, y, z;
};

__host__ __device__ inline bool operator==(const FullKey& a, const FullKey& c) {
    return a.b == c.b && a.x == c.x && a.y == c.y && a.z == c.z;
}

// A key ready for a table: its packed word, or the wide tag with the full
// key kept for the comparison; `hash` places it in the table.
struct TableKey {
    uint64_t word;  // packed word, or kWideMark | tag << 32 for a wide key
    uint64_t hash;
    FullKey full;
    bool wide;
};

__host__ __device__ inline TableKey table_key(int64_t b, int64_t x, int64_t y, int64_t z) {
    TableKey k;
    k.full = {b, x, y, z};
    uint64_t packed;
    if (pack_key(b, x, y, z, &packed)) {
        k.word = packed;
        k.hash = mix64(packed);
        k.wide = false;
    } else {
        uint64_t h = mix64(static_cast<uint64_t>(z) ^ 0x9e3779b97f4a7c15ull);
        h = mix64(h ^ static_cast<uint64_t>(y));
        h = mix64(h ^ static_cast<uint64_t>(x));
        h = mix64(h ^ static_cast<uint64_t>(b));
        k.hash = h;
        k.word = kWideMark | (((h >> 40) & 0x3fffffull) << 32);
        k.wide = true;
    }
    return k;
}

__host__ __device__ inline bool is_wide_word(uint64_t w) { return (w & kWideMark) == kWideMark && w != kEmptyKey; }

// Whether a slot word may hold the wide key `k` (same tag): the caller then
// compares the full key of the claiming row.
__host__ __device__ inline bool same_tag(uint64_t w, const TableKey& k) {
    return w != kEmptyKey && (w & 0xffffffff00000000ull) == k.word;
}

__host__ __device__ inline int32_t claim_row(uint64_t w) { return static_cast<int32_t>(static_cast<uint32_t>(w)); }

// Key sources: recompute the key of a table row from the immutable rows the
// table was built from.  Each defines key_of(row).

// The coordinate of an input row (b, x, y, z).
struct CoordSource {
    const int32_t* coords;
    __device__ inline FullKey key_of(int32_t row) const {
        const int4 c = reinterpret_cast<const int4*>(coords)[row];
        return {c.x, c.y, c.z, c.w};
    }
};

// The 2x2x2 block of an input row (b, x >> 1, y >> 1, z >> 1).
struct BlockSource {
    const int32_t* coords;
    __device__ inline FullKey key_of(int32_t row) const {
        const int4 c = reinterpret_cast<const int4*>(coords)[row];
        return {c.x, c.y >> 1, c.z >> 1, c.w >> 1};
    }
};

// Open-addressing table of 16-byte slots (key word, first row),
// power-of-two capacity, linear probing.  A stored row is the minimum input
// row that inserted the key, i.e. its first occurrence.  Key and row share
// one slot, so an insert's compare-and-swap and its atomic min, and a
// lookup's key and row, touch one line.
struct alignas(16) CoordSlot {
    unsigned long long key;
    int32_t row;
    int32_t pad;
};
static_assert(sizeof(CoordSlot) == 16, "one 16-byte slot per key");

// Cleared slot: empty key, row INT_MAX (as one 16-byte store).
__host__ __device__ inline int4 empty_coord_slot() { return int4{-1, -1, 0x7fffffff, 0}; }

// Every probe loop stops after `capacity` probes.  The tables are sized
// above their key count (at least one empty slot always remains), so a
// probe meets its key or an empty slot first; the bound only keeps a sizing
// mistake from spinning forever.  A lookup that exhausts the table answers
// "absent" (it visited every slot); an insert that does sets
// LATTICE_STATUS_TABLE_OVERFLOW in `status` (when given) and gives up.
__device__ inline void flag_table_overflow(int32_t* status) {
    if (status != nullptr) atomicOr(status, LATTICE_STATUS_TABLE_OVERFLOW);
}

struct CoordTable {
    CoordSlot* slots;
    uint32_t mask;  // capacity - 1
    int32_t* status = nullptr;  // overflow flag word, or null

    // Inserts `row` under key `k` (keeping the minimum row) and returns the
    // key's slot.  `src` recomputes the key of a claiming row.
    template <typename Source>
    __device__ inline uint32_t insert(const TableKey& k, int32_t row, const Source& src) const {
        uint32_t slot = static_cast<uint32_t>(k.hash) & mask;
        const unsigned long long mine = k.wide ? (k.word | static_cast<uint32_t>(row)) : k.word;
        for (uint32_t probe = 0; probe <= mask; ++probe) {
            const unsigned long long prev = atomicCAS(&slots[slot].key, static_cast<unsigned long long>(kEmptyKey),
                                                      mine);
            const bool hit = prev == kEmptyKey || (k.wide ? same_tag(prev, k) && src.key_of(claim_row(prev)) == k.full
                                                          : prev == k.word);
            if (hit) {
                // The stored row only decreases, so a row at or below ours,
                // even a stale read of it, makes the atomic a no-op: skip it
                // (a key inserted by several rows mostly needs one).
                if (prev == kEmptyKey || slots[slot].row > row) atomicMin(&slots[slot].row, row);
                return slot;
            }
            slot = (slot + 1) & mask;
        }
        // Full table: flag it and hand back a valid slot (its results are void).
        flag_table_overflow(status);
        return static_cast<uint32_t>(k.hash) & mask;
    }

    // Slot of key `k`, or -1.
    template <typename Source>
    __device__ inline int32_t find_slot(const TableKey& k, const Source& src) const {
        uint32_t slot = static_cast<uint32_t>(k.hash) & mask;
        for (uint32_t probe = 0; probe <= mask; ++probe) {
            const uint64_t w = slots[slot].key;
            if (k.wide ? same_tag(w, k) && src.key_of(claim_row(w)) == k.full : w == k.word) {
                return static_cast<int32_t>(slot);
            }
            if (w == kEmptyKey) return -1;
            slot = (slot + 1) & mask;
        }
        return -1;
    }

    // First row of key `k`, or -1.  Packed keys read the key and the row
    // from one 16-byte load.
    template <typename Source>
    __device__ inline int32_t find(const TableKey& k, const Source& src) const {
        if (!k.wide) {
            uint32_t slot = static_cast<uint32_t>(k.hash) & mask;
            for (uint32_t probe = 0; probe <= mask; ++probe) {
                const int4 v = *reinterpret_cast<const int4*>(slots + slot);
                const uint64_t w = static_cast<uint64_t>(static_cast<uint32_t>(v.x)) |
                                   (static_cast<uint64_t>(static_cast<uint32_t>(v.y)) << 32);
                if (w == k.word) return v.z;
                if (w == kEmptyKey) return -1;
                slot = (slot + 1) & mask;
            }
            return -1;
        }
        const int32_t slot = find_slot(k, src);
        return slot < 0 ? -1 : slots[slot].row;
    }
};

// Block-bucketed coordinate table for the kernel-map queries.  A bucket is
// one 64-byte line holding a 2x2x2 block of the lattice: the key word of
// the block (batch, x>>1, y>>1, z>>1) and the first input row of each of its
// eight voxels.  The 27 neighbours of a voxel lie in at most eight blocks,
// so a row's probes touch at most eight lines, lanes probing the same block
// share one line request, and a probe reads its key and its row from the
// same line.  Rows are stored as kRowBias - row so that the cleared value 0
// means "absent" and atomicMax keeps the smallest (first) row.  Wide block
// keys are compared through BlockSource over the table's input coordinates.
constexpr int32_t kRowBias = 0x7fffffff;

struct alignas(64) BlockBucket {
    unsigned long long key;
    int32_t rows[8];
    int32_t pad[6];
};
static_assert(sizeof(BlockBucket) == 64, "one bucket per 64-byte line");

__host__ __device__ inline bool fits_int32(int64_t v) { return v >= INT32_MIN && v <= INT32_MAX; }

// Block key and octant of a voxel; false when an axis value lies outside
// int32 (no input coordinate can match it).
__host__ __device__ inline bool block_of(int64_t b, int64_t x, int64_t y, int64_t z, TableKey* block_key,
                                         int* octant) {
    if (!fits_int32(x) || !fits_int32(y) || !fits_int32(z)) return false;
    *block_key = table_key(b, x >> 1, y >> 1, z >> 1);  // arithmetic shift = floor(v / 2)
    *octant = static_cast<int>(((x & 1) << 2) | ((y & 1) << 1) | (z & 1));
    return true;
}

struct BlockTable {
    BlockBucket* buckets;
    uint32_t mask;  // bucket count - 1; the count exceeds the block count
    BlockSource src;  // the input coordinates the table was built from
    int32_t* status = nullptr;  // overflow flag word, or null

    // kExact: the voxel's slot keeps the smallest row (an atomic max on the
    // biased row).  Otherwise a plain store: the slot then holds one of the
    // rows with the voxel's coordinate (the smallest unless a coordinate
    // repeats), and the caller restores the smallest afterwards
    // (query_rows_k3 does so from each row's self lookup).
    template <bool kExact = true>
    __device__ inline void insert(const TableKey& block_key, int octant, int32_t row) const {
        uint32_t slot = static_cast<uint32_t>(block_key.hash) & mask;
        const unsigned long long mine =
            block_key.wide ? (block_key.word | static_cast<uint32_t>(row)) : block_key.word;
        for (uint32_t probe = 0; probe <= mask; ++probe) {
            // One compare-and-swap claims an empty slot or reports its key.
            const unsigned long long k = atomicCAS(&buckets[slot].key, static_cast<unsigned long long>(kEmptyKey),
                                                   mine);
            const bool hit = k == kEmptyKey ||
                             (block_key.wide ? same_tag(k, block_key) && src.key_of(claim_row(k)) == block_key.full
                                             : k == block_key.word);
            if (hit) {
                if constexpr (kExact) {
                    atomicMax(&buckets[slot].rows[octant], kRowBias - row);
                } else {
                    buckets[slot].rows[octant] = kRowBias - row;
                }
                return;
            }
            slot = (slot + 1) & mask;
        }
        flag_table_overflow(status);
    }

    // Whether slot word `w` holds block key `k`.
    __device__ inline bool holds(uint64_t w, const TableKey& k) const {
        return k.wide ? same_tag(w, k) && src.key_of(claim_row(w)) == k.full : w == k.word;
    }

    // Bucket of the block, or -1.
    __device__ inline int32_t find_bucket(const TableKey& block_key) const {
        uint32_t slot = static_cast<uint32_t>(block_key.hash) & mask;
        for (uint32_t probe = 0; probe <= mask; ++probe) {
            const unsigned long long k = buckets[slot].key;
            if (holds(k, block_key)) return static_cast<int32_t>(slot);
            if (k == kEmptyKey) return -1;
            slot = (slot + 1) & mask;
        }
        return -1;
    }

    // First row of the voxel, or -1.
    __device__ inline int32_t find(const TableKey& block_key, int octant) const {
        uint32_t slot = static_cast<uint32_t>(block_key.hash) & mask;
        for (uint32_t probe = 0; probe <= mask; ++probe) {
            const unsigned long long k = buckets[slot].key;
            const int32_t r = buckets[slot].rows[octant];
            if (holds(k, block_key)) return r == 0 ? -1 : kRowBias - r;
            if (k == kEmptyKey) return -1;
            slot = (slot + 1) & mask;
        }
        return -1;
    }
};

// floor division for a positive divisor (quantization_detail.h:3-10).
__host__ __device__ inline int64_t floor_div_pos(int64_t v, int64_t d) {
    int64_t q = v / d;
    int64_t r = v % d;
    if (r != 0 && r < 0) --q;
    return q;
}

struct Int3 {
    int x, y, z;
};

}  // namespace lattice
