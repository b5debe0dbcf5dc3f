// Device-wide helpers shared by the relation and view builders.
#pragma once

#include "lattice_common.h"

namespace lattice {

const char* last_error();

// Bytes of workspace exclusive_scan() carves for `n` items.
size_t scan_workspace_bytes(long long n);

// out[i] = sum(in[0..i)); in == out allowed.  `total` (device, optional)
// receives the sum of all n items.
int exclusive_scan(const int* in, int* out, long long n, int* total, Workspace& ws,
                   hipStream_t stream);

// p[0..n) = value with a kernel (no memset node, so the call can be captured
// into a graph).
int fill_i32(int* p, long long n, int value, hipStream_t stream);

}  // namespace lattice
