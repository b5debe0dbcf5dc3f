// Stable device radix sort of (key, index) pairs, shared by the sorted
// implicit-GEMM view (row masks) and the grouped CSR views (edge groups).
#pragma once

#include "lattice_common.h"

namespace lattice {

// Where pass 0 reads its keys: key(i) = src[i * stride].
//   * groups >= 0: slots at or past count[0] (device, optional) and values
//     outside [0, groups) get the key `groups`, which sorts last;
//   * flip_sign: the key is ordered as a signed int32 (sign bit flipped for
//     the sort, restored in the sorted keys written out).
struct SortKeys {
    const int32_t* src;
    int stride;
    const int32_t* count;
    int groups;
    bool flip_sign;
    // When non-null, the sort runs only if *run_if != 0 (read on the
    // device, so a caller can skip it without a host synchronisation).
    const int32_t* run_if = nullptr;
};

size_t radix_sort_workspace_bytes(int n, int end_bit);

// Sorts keys on bits [0, end_bit) (1..32), stably: equal keys keep their
// index order.  Writes the sorted keys (may be NULL) and the source index
// of each sorted position.  No host synchronisation, no memset nodes.
int radix_sort_indices(const SortKeys& keys, int n, int end_bit, int32_t* sorted_keys, int32_t* sorted_index,
                       Workspace& ws, hipStream_t stream);

}  // namespace lattice
