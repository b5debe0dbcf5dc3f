// Device-wide exclusive prefix sum over int32 (in place allowed) and the
// error-message store shared by the library.
//
// Three phases per level: each 256-thread block scans 4096 items and writes
// its total; the totals are scanned recursively; the block offsets are added
// back.  The grand total is written to `total` (device) when non-NULL.

#include "lattice_common.h"
#include "scan.h"

namespace lattice {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& message) { g_last_error = message; }
const char* last_error() { return g_last_error.c_str(); }

namespace {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanTile = kScanThreads * kScanItems;

__device__ inline int wave_inclusive_scan(int v) {
    const int lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        int up = __shfl_up(v, d, kWave);
        if (lane >= d) v += up;
    }
    return v;
}

// Block-wide exclusive scan of one value per thread; returns the exclusive
// prefix and the block total through `total`.
__device__ inline int block_exclusive_scan(int v, int* total) {
    __shared__ int wave_sums[kScanThreads / kWave];
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    int inc = wave_inclusive_scan(v);
    if (lane == kWave - 1) wave_sums[wave] = inc;
    __syncthreads();
    int before = 0;
    int sum = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / kWave; ++w) {
        int s = wave_sums[w];
        if (w < wave) before += s;
        sum += s;
    }
    __syncthreads();
    *total = sum;
    return before + inc - v;
}

__global__ void __launch_bounds__(kScanThreads)
scan_tiles(const int* __restrict__ in, int* out, int n, int* tile_sums) {
    const long long base = static_cast<long long>(blockIdx.x) * kScanTile +
                           static_cast<long long>(threadIdx.x) * kScanItems;
    int vals[kScanItems];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        long long idx = base + i;
        vals[i] = idx < n ? in[idx] : 0;
        sum += vals[i];
    }
    int total = 0;
    int prefix = block_exclusive_scan(sum, &total);
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        long long idx = base + i;
        if (idx < n) out[idx] = prefix;
        prefix += vals[i];
    }
    if (threadIdx.x == 0 && tile_sums != nullptr) tile_sums[blockIdx.x] = total;
}

__global__ void __launch_bounds__(kScanThreads)
add_tile_offsets(int* out, int n, const int* __restrict__ tile_offsets) {
    const int add = tile_offsets[blockIdx.x];
    const long long base = static_cast<long long>(blockIdx.x) * kScanTile;
    for (int i = threadIdx.x; i < kScanTile; i += kScanThreads) {
        long long idx = base + i;
        if (idx < n) out[idx] += add;
    }
}

// total = out[n-1] + in_last (the last input, captured before an in-place scan).
__global__ void write_total(const int* out, int n, const int* last_in, int* total) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        *total = n > 0 ? out[n - 1] + *last_in : 0;
    }
}

__global__ void copy_last(const int* in, int n, int* dst) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *dst = n > 0 ? in[n - 1] : 0;
}

__global__ void fill_i32_kernel(int* p, long long n, int value) {
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x) {
        p[i] = value;
    }
}

}  // namespace

int fill_i32(int* p, long long n, int value, hipStream_t stream) {
    if (n <= 0) return LATTICE_OK;
    fill_i32_kernel<<<grid_for(n, 256, 8192), 256, 0, stream>>>(p, n, value);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

size_t scan_workspace_bytes(long long n) {
    size_t bytes = aligned_bytes(sizeof(int));  // captured last element
    long long level = n;
    while (level > kScanTile) {
        level = (level + kScanTile - 1) / kScanTile;
        bytes += aligned_bytes(static_cast<size_t>(level) * sizeof(int));
    }
    return bytes + 256;
}

static int scan_level(const int* in, int* out, long long n, Workspace& ws,
                      hipStream_t stream) {
    const unsigned tiles = static_cast<unsigned>((n + kScanTile - 1) / kScanTile);
    if (tiles <= 1) {
        scan_tiles<<<1, kScanThreads, 0, stream>>>(in, out, static_cast<int>(n), nullptr);
        LATTICE_LAUNCH_CHECK();
        return LATTICE_OK;
    }
    int* sums = ws.take<int>(tiles);
    if (sums == nullptr) {
        set_error("scan workspace too small");
        return LATTICE_ERROR_INVALID_ARGUMENT;
    }
    scan_tiles<<<tiles, kScanThreads, 0, stream>>>(in, out, static_cast<int>(n), sums);
    LATTICE_LAUNCH_CHECK();
    int rc = scan_level(sums, sums, tiles, ws, stream);
    if (rc != LATTICE_OK) return rc;
    add_tile_offsets<<<tiles, kScanThreads, 0, stream>>>(out, static_cast<int>(n), sums);
    LATTICE_LAUNCH_CHECK();
    return LATTICE_OK;
}

int exclusive_scan(const int* in, int* out, long long n, int* total, Workspace& ws,
                   hipStream_t stream) {
    if (n <= 0) {
        return total != nullptr ? fill_i32(total, 1, 0, stream) : LATTICE_OK;
    }
    int* last = ws.take<int>(1);
    if (last == nullptr) {
        set_error("scan workspace too small");
        return LATTICE_ERROR_INVALID_ARGUMENT;
    }
    if (total != nullptr) {
        copy_last<<<1, 64, 0, stream>>>(in, static_cast<int>(n), last);
        LATTICE_LAUNCH_CHECK();
    }
    int rc = scan_level(in, out, n, ws, stream);
    if (rc != LATTICE_OK) return rc;
    if (total != nullptr) {
        write_total<<<1, 64, 0, stream>>>(out, static_cast<int>(n), last, total);
        LATTICE_LAUNCH_CHECK();
    }
    return LATTICE_OK;
}

}  // namespace lattice

extern "C" const char* lattice_hip_last_error(void) { return lattice::last_error(); }
extern "C" const char* lattice_hip_version(void) { return "lattice-hip 0.1.0 (gfx950)"; }
