// Shared helpers of the gfx950 sparse-convolution library: error plumbing,
// launch helpers, wavefront intrinsics, the packed 64-bit coordinate key and
// the open-addressing hash probe.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
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

// ------------------------------------------------------ packed coord key --
//
// key = batch << 54 | (x + 2^17) << 36 | (y + 2^17) << 18 | (z + 2^17).
// Injective over batch in [0, 1022] and x, y, z in [-2^17, 2^17); the
// all-ones word (batch 1023) is never produced and marks an empty slot.

constexpr uint64_t kEmptyKey = ~0ull;
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

// Open-addressing table of 16-byte slots (key, first row), power-of-two
// capacity, linear probing.  A stored row is the minimum input row that
// inserted the key, i.e. its first occurrence.  Key and row share one slot,
// so an insert's compare-and-swap and its atomic min, and a lookup's key
// and row, touch one line.
struct alignas(16) CoordSlot {
    unsigned long long key;
    int32_t row;
    int32_t pad;
};
static_assert(sizeof(CoordSlot) == 16, "one 16-byte slot per key");

// Cleared slot: empty key, row INT_MAX (as one 16-byte store).
__host__ __device__ inline int4 empty_coord_slot() { return int4{-1, -1, 0x7fffffff, 0}; }

struct CoordTable {
    CoordSlot* slots;
    uint32_t mask;  // capacity - 1

    __device__ inline void insert(uint64_t key, int32_t row) const {
        uint32_t slot = static_cast<uint32_t>(mix64(key)) & mask;
        while (true) {
            unsigned long long prev = atomicCAS(&slots[slot].key, static_cast<unsigned long long>(kEmptyKey),
                                                static_cast<unsigned long long>(key));
            if (prev == kEmptyKey || prev == key) {
                atomicMin(&slots[slot].row, row);
                return;
            }
            slot = (slot + 1) & mask;
        }
    }

    __device__ inline int32_t find(uint64_t key) const {
        uint32_t slot = static_cast<uint32_t>(mix64(key)) & mask;
        while (true) {
            const int4 v = *reinterpret_cast<const int4*>(slots + slot);
            const uint64_t k = static_cast<uint64_t>(static_cast<uint32_t>(v.x)) |
                               (static_cast<uint64_t>(static_cast<uint32_t>(v.y)) << 32);
            if (k == key) return v.z;
            if (k == kEmptyKey) return -1;
            slot = (slot + 1) & mask;
        }
    }
};

// Block-bucketed coordinate table for the kernel-map queries.  A bucket is
// one 64-byte line holding a 2x2x2 block of the lattice: the packed key of
// the block (batch, x>>1, y>>1, z>>1) and the first input row of each of its
// eight voxels.  The 27 neighbours of a voxel lie in at most eight blocks,
// so a row's probes touch at most eight lines, lanes probing the same block
// share one line request, and a probe reads its key and its row from the
// same line.  Rows are stored as kRowBias - row so that the cleared value 0
// means "absent" and atomicMax keeps the smallest (first) row.
constexpr int32_t kRowBias = 0x7fffffff;

struct alignas(64) BlockBucket {
    unsigned long long key;
    int32_t rows[8];
    int32_t pad[6];
};
static_assert(sizeof(BlockBucket) == 64, "one bucket per 64-byte line");

// Block key and octant of a voxel; false when it does not fit the packed key.
__host__ __device__ inline bool block_of(int64_t b, int64_t x, int64_t y, int64_t z, uint64_t* block_key,
                                         int* octant) {
    uint64_t key;
    if (!pack_key(b, x, y, z, &key)) return false;
    pack_key(b, x >> 1, y >> 1, z >> 1, block_key);  // arithmetic shift = floor(v / 2)
    *octant = static_cast<int>(((x & 1) << 2) | ((y & 1) << 1) | (z & 1));
    return true;
}

struct BlockTable {
    BlockBucket* buckets;
    uint32_t mask;  // bucket count - 1; the count exceeds the block count

    __device__ inline void insert(uint64_t block_key, int octant, int32_t row) const {
        uint32_t slot = static_cast<uint32_t>(mix64(block_key)) & mask;
        while (true) {
            // One compare-and-swap claims an empty slot or reports its key.
            unsigned long long k = atomicCAS(&buckets[slot].key, static_cast<unsigned long long>(kEmptyKey),
                                             static_cast<unsigned long long>(block_key));
            if (k == kEmptyKey) k = block_key;
            if (k == block_key) {
                atomicMax(&buckets[slot].rows[octant], kRowBias - row);
                return;
            }
            slot = (slot + 1) & mask;
        }
    }

    // First row of the voxel, or -1.
    __device__ inline int32_t find(uint64_t block_key, int octant) const {
        uint32_t slot = static_cast<uint32_t>(mix64(block_key)) & mask;
        while (true) {
            const unsigned long long k = buckets[slot].key;
            const int32_t r = buckets[slot].rows[octant];
            if (k == block_key) return r == 0 ? -1 : kRowBias - r;
            if (k == kEmptyKey) return -1;
            slot = (slot + 1) & mask;
        }
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
