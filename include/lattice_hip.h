/*
 * lattice_hip.h — C ABI of the MI355X (gfx950) sparse-convolution hot path.
 *
 * Plain pointers, sizes and an opaque stream handle only.  Every pointer
 * named "device" is HIP device memory; "host" pointers are read on the host
 * before the call returns.  All work is enqueued on `stream` (a hipStream_t
 * passed as void*, NULL = the default stream) and stays asynchronous: no
 * entry point synchronises the stream or reads device memory back.
 * Entry points never allocate or free memory: outputs and scratch
 * ("workspace") are provided by the caller, sized by the *_workspace_bytes
 * queries.
 *
 * Return value: LATTICE_OK or an error code; lattice_hip_last_error() returns
 * a message for the calling thread's last failure.  Argument errors mirror
 * the reference's std::invalid_argument (mapped to ValueError by the Python
 * bindings), unsupported-path and HIP errors its std::runtime_error.
 *
 * The entry points replace the following reference interfaces (paths are
 * relative to the mlx-lattice source tree):
 *   build_kernel_relation            native/features/coordinates/api.h:67-79,
 *                                    relations.cpp:540-581, bindings/coords.cpp:414-449
 *   build_submanifold_kernel_relation relations.cpp:583-597, bindings/coords.cpp:480-507
 *   build_target_kernel_relation     relations.cpp:672-722, bindings/coords.cpp:550-589
 *   build_generative_relation        relations.cpp:599-629, bindings/coords.cpp:451-479
 *   build_transposed_kernel_relation relations.cpp:631-670, bindings/coords.cpp:509-548
 *   build_relation_implicit_gemm_view relations.cpp:498-538, bindings/coords.cpp:590-626
 *   sorted implicit-GEMM view        mlx_lattice/core/relations/views.py:467-510
 *   sparse_conv_features             native/features/convolution/api.cpp:119-246,
 *                                    bindings/convolution.cpp:90-146
 *   sparse_conv_features_sorted_implicit_gemm
 *                                    api.cpp:248-281, bindings/convolution.cpp:147-234
 *   sparse_quantized_conv_features   convolution/quantized.cpp:198-268,
 *                                    bindings/convolution.cpp:12-89
 *   conv input / weight gradients    convolution/primitive.cpp:137-176,
 *                                    597-680 (the conv primitive's vjp),
 *                                    cpu/algorithms.cpp:355-481
 *   sparse_pool_features (+ vjp)     native/features/pooling/primitive.cpp,
 *                                    pooling/cpu/algorithms.cpp:180-331,
 *                                    bindings/pooling.cpp:15-66
 *   global pools                     mlx_lattice/ops/pool.py:198-236
 *   sparse_quantize, voxelize_features, build_point_voxel_map,
 *   interpolate_point_features (+ vjps)
 *                                    native/features/coordinates/quantization.cpp,
 *                                    cpu/quantization_detail.h:66-391,
 *                                    mlx_lattice/core/coords/quantization.py
 */
#ifndef LATTICE_HIP_H_
#define LATTICE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum lattice_status {
    LATTICE_OK = 0,
    LATTICE_ERROR_INVALID_ARGUMENT = 1,
    LATTICE_ERROR_UNSUPPORTED = 2,
    LATTICE_ERROR_HIP = 3
};

enum lattice_dtype {
    LATTICE_F32 = 0,
    LATTICE_F16 = 1,
    LATTICE_BF16 = 2
};

/* Weight layouts of the float conv (native/features/convolution/contract.h:19-22). */
enum lattice_weight_layout {
    LATTICE_WEIGHT_KERNEL_MAJOR = 0, /* (K, C_in, C_out) contiguous */
    LATTICE_WEIGHT_DENSE_5D = 1      /* (C_out, Kx, Ky, Kz, C_in) contiguous */
};

/* Store-side epilogue flags of the conv entries (the `epilogue` argument
 * after `bias`).  LATTICE_EPILOGUE_RELU applies the reference's
 * `maximum(feats, 0)` (ops/feature.py:54-56) to every stored value, after
 * the rounding and the optional bias: v where v > 0 or v is NaN, +0
 * otherwise.  The result equals a separate ReLU over the conv's output bit
 * for bit, on every row.  No counterpart in the reference's conv
 * primitives: it saves the separate pass over all output rows that a
 * conv followed by ReLU would make. */
enum lattice_epilogue_flags {
    LATTICE_EPILOGUE_NONE = 0,
    LATTICE_EPILOGUE_RELU = 1
};

/* Bits of the device status word written by the relation builders.  Every
 * int32 coordinate is accepted (as by the reference's CoordHash over all
 * four words, cpu/common_detail.h:68-77); LATTICE_STATUS_COORD_RANGE is
 * kept for ABI stability and is never set. */
enum lattice_relation_flags {
    LATTICE_STATUS_COORD_RANGE = 1,   /* unused: no coordinate is out of range */
    LATTICE_STATUS_REPEATED_EDGE = 2, /* transposed relation: two edges share (out_row, kernel_id) */
    LATTICE_STATUS_REPEATED_PAIR = 4, /* transposed dense map: two edges share (in_row, kernel_id) */
    LATTICE_STATUS_REPEATED_COORD = 8, /* submanifold relation: an active row repeats an earlier row's coordinate */
    LATTICE_STATUS_TABLE_OVERFLOW = 16 /* a coordinate table filled up (a sizing error; the relation is void) */
};

/* Packed-key range: a key with batch in [0, LATTICE_MAX_BATCH] and axes in
 * [LATTICE_MIN_COORD, LATTICE_MAX_COORD] (a 2x2x2 block key: the block
 * coordinates) takes the one-compare packed form; every other key takes
 * the wide form, compared in full against the table's source rows.  Both
 * give the same results; only the speed of a lookup differs. */
#define LATTICE_MAX_BATCH 1022
#define LATTICE_MIN_COORD (-131072)
#define LATTICE_MAX_COORD 131071

const char* lattice_hip_last_error(void);
const char* lattice_hip_version(void);

/* next_pow2(max(2*rows, 1)): relations.cpp:95-105. */
int lattice_hip_coord_hash_capacity(int rows);
/* Bucket count of the 2x2x2 block table the relation builders query: a
 * power of two above 1.5 * rows, so at least a third of the buckets stay
 * empty whatever the coordinates (no reference counterpart: the reference
 * hashes single voxels). */
int lattice_hip_block_table_capacity(int rows);

/* Kernel offsets in the reference order (offsets.cpp:11-45): odd sizes
 * -r..r, even sizes 0..k-1, x outer, z inner, times dilation.  Writes K*3
 * ints to `out` (host) when non-NULL; returns K, or -1 on invalid input. */
int lattice_hip_kernel_offsets(const int kernel_size[3], const int dilation[3],
                               int32_t* out);

/* Output buffers of a relation build.  Capacities follow the reference:
 * forward: out_capacity = rows, edge_capacity = rows*K (relations.cpp:550-553);
 * target:  out_capacity = target_rows, edge_capacity = target_rows*K.
 * Only active prefixes are defined for in_rows/out_rows/kernel_ids/
 * in_edge_ids/kernel_edge_ids (counts[0] entries); row_offsets, the CSR row
 * offsets, counts, out_coords (zero tail), out_in_map (-1 tail) and
 * row_masks (zero tail) are fully written.  The four grouped-view pointers
 * (in_row_offsets, in_edge_ids, kernel_row_offsets, kernel_edge_ids) are
 * either all set, or all NULL to skip the views (they can be built later
 * with lattice_hip_build_relation_grouped_views). */
typedef struct lattice_relation_outputs {
    int32_t* in_rows;            /* device [edge_capacity] */
    int32_t* out_rows;           /* device [edge_capacity] */
    int32_t* kernel_ids;         /* device [edge_capacity] */
    int32_t* row_offsets;        /* device [out_capacity + 1] */
    int32_t* out_coords;         /* device [out_capacity, 4]; NULL for target relations */
    int32_t* counts;             /* device [2] = [E, N_out] */
    int32_t* in_row_offsets;     /* device [in_capacity + 1] */
    int32_t* in_edge_ids;        /* device [edge_capacity] */
    int32_t* kernel_row_offsets; /* device [K + 1] */
    int32_t* kernel_edge_ids;    /* device [edge_capacity] */
    int32_t* out_in_map;         /* device [out_capacity, K] (implicit-GEMM view) */
    int32_t* row_masks;          /* device [out_capacity, ceil(K/32)] */
    int32_t* status;             /* device [1]: lattice_relation_flags bits */
} lattice_relation_outputs;

size_t lattice_hip_kernel_relation_workspace_bytes(int rows, int kernel_count);
/* Set in workspace_bytes of lattice_hip_build_kernel_relation: the
 * workspace is the one an earlier lattice_hip_build_kernel_relation call
 * used over the same coords and active_rows (any kernel geometry), and its
 * block table of those coordinates, which no later step of a build
 * modifies, is reused instead of cleared and rebuilt.  No counterpart in
 * the reference: a submanifold relation and the downsample relation of the
 * same level hash the same coordinates. */
#define LATTICE_RELATION_TABLE_READY ((size_t)1 << 62)
/* Bytes of the 2x2x2 block table of `rows` input rows (the first part of
 * the lattice_hip_build_kernel_relation workspace). */
size_t lattice_hip_block_table_bytes(int rows);
size_t lattice_hip_target_relation_workspace_bytes(int rows, int target_rows,
                                                   int kernel_count);

/* Forward relation: write_kernel_relation (cpu/relation_build_detail.h:3-41).
 * stride (1,1,1) with padding (0,0,0) keeps input rows as output rows
 * (submanifold); otherwise outputs are the first-seen floor-divided cells.
 * coords: device int32 [rows, 4]; active_rows: device int32 [1]. */
int lattice_hip_build_kernel_relation(
    const int32_t* coords, int rows, const int32_t* active_rows,
    const int kernel_size[3], const int stride[3], const int padding[3],
    const int dilation[3], const lattice_relation_outputs* out,
    void* workspace, size_t workspace_bytes, void* stream);
/* lattice_hip_build_kernel_relation with the block table in memory of its
 * own: `table` holds at least lattice_hip_block_table_bytes(rows) bytes
 * (LATTICE_RELATION_TABLE_READY may be set in table_bytes when it already
 * holds the table of these coords and active_rows), `workspace` at least
 * lattice_hip_kernel_relation_workspace_bytes(rows, K) -
 * lattice_hip_block_table_bytes(rows).  A caller that keeps the table for
 * the next relation over the same coordinates keeps only the table.  No
 * reference counterpart (the reference hashes each build anew). */
int lattice_hip_build_kernel_relation_with_table(
    const int32_t* coords, int rows, const int32_t* active_rows,
    const int kernel_size[3], const int stride[3], const int padding[3],
    const int dilation[3], const lattice_relation_outputs* out, void* table,
    size_t table_bytes, void* workspace, size_t workspace_bytes, void* stream);

/* Target relation: write_target_kernel_relation (relation_build_detail.h:43-80). */
int lattice_hip_build_target_kernel_relation(
    const int32_t* coords, int rows, const int32_t* active_rows,
    const int32_t* target_coords, int target_rows,
    const int32_t* target_active_rows, const int kernel_size[3],
    const int stride[3], const int padding[3], const int dilation[3],
    const lattice_relation_outputs* out, void* workspace,
    size_t workspace_bytes, void* stream);

/* Generative and transposed relations (relation_build_detail.h:82-196;
 * native builders relations.cpp:599-670).  Every active input row expands
 * into K candidates coord * stride + offset[k] - padding; output and edge
 * capacities are rows * K, so out->out_coords holds rows * K rows and
 * out->out_in_map / out->row_masks are not used (may be NULL).
 *   generative: output row in*K + k per candidate (no padding, no
 *     dilation), one edge per row (write_generative_relation :82-117);
 *   transposed: the same layout when every stride exceeds the offsets'
 *     extent (can_use_direct_transposed_relation, relations.cpp:107-127);
 *     otherwise first-seen deduplicated output rows and edges in
 *     (out_row, kernel_id, in_row) order (:119-196).  A repeated input
 *     coordinate sets LATTICE_STATUS_REPEATED_EDGE in out->status. */
size_t lattice_hip_expanded_relation_workspace_bytes(
    int rows, const int kernel_size[3], const int stride[3],
    const int dilation[3], int generative);
int lattice_hip_build_generative_relation(
    const int32_t* coords, int rows, const int32_t* active_rows,
    const int kernel_size[3], const int stride[3],
    const lattice_relation_outputs* out, void* workspace,
    size_t workspace_bytes, void* stream);
int lattice_hip_build_transposed_kernel_relation(
    const int32_t* coords, int rows, const int32_t* active_rows,
    const int kernel_size[3], const int stride[3], const int padding[3],
    const int dilation[3], const lattice_relation_outputs* out,
    void* workspace, size_t workspace_bytes, void* stream);

/* Stable grouping of n int32 keys into `groups` groups (the counting sort
 * of write_relation_grouped_view, relation_views_detail.h:84-120, for any
 * key array): offsets[groups + 1] and ids[n], ids listing the positions of
 * group 0, then group 1, ... each in increasing position order.  Keys
 * outside [0, groups) and positions at or past *count (device, optional)
 * are left out (sorted past offsets[groups]). */
size_t lattice_hip_group_by_key_workspace_bytes(int n);
int lattice_hip_group_by_key(const int32_t* keys, int n, const int32_t* count,
                             int groups, int32_t* offsets, int32_t* ids,
                             void* workspace, size_t workspace_bytes,
                             void* stream);

/* ---- point -> voxel quantization (core/coords/quantization.py;
 * cpu/quantization_detail.h:66-391; native quantization.cpp) ----
 * Points are float32 [rows, 3], batch indices int32 [rows]; voxel_size and
 * origin are host float[3].  Float arithmetic is binary32 with one rounding
 * per operation (no contracted multiply-adds). */

/* sparse_quantize (quantization.py:92-118; write_sparse_quantization,
 * quantization_detail.h:91-128): voxel (batch, floor((p - origin) /
 * voxel_size)), first-seen point order.  Outputs (capacity = rows):
 * coords int32 [rows, 4] (zero tail), voxel_count int32 [1], inverse_rows
 * int32 [rows] (-1 for inactive points), counts int32 [rows] (zero tail).
 * Voxels are deduplicated on their int64 value and written as int32 (low
 * 32 bits); `status` is zeroed. */
size_t lattice_hip_sparse_quantize_workspace_bytes(int rows);
int lattice_hip_sparse_quantize(
    const float* points, const int32_t* batch_indices, int rows,
    const int32_t* active_rows, const float voxel_size[3],
    const float origin[3], int32_t* coords, int32_t* voxel_count,
    int32_t* inverse_rows, int32_t* counts, int32_t* status, void* workspace,
    size_t workspace_bytes, void* stream);

/* voxelize_features (quantization.py:121-149; write_voxel_features,
 * quantization_detail.h:141-170): out[v] = sum over the points of voxel v,
 * in point order, of feats[p] * scale (scale 1 for mode 0 = sum, 1 /
 * max(counts[v], 1) for mode 1 = mean).  voxel_offsets / point_ids: the
 * grouping of inverse_rows by voxel (lattice_hip_group_by_key, with the
 * active point count).  feats and out are float32. */
int lattice_hip_voxelize_features(int mode, const float* feats, int channels,
                                  const int32_t* counts, int voxel_rows,
                                  const int32_t* voxel_offsets,
                                  const int32_t* point_ids, float* out,
                                  void* stream);
/* write_voxel_feature_grad (quantization_detail.h:172-200). */
int lattice_hip_voxelize_features_grad(int mode, const float* cot,
                                       int voxel_rows, int channels,
                                       const int32_t* inverse_rows,
                                       const int32_t* counts, int point_rows,
                                       const int32_t* point_active,
                                       float* grad, void* stream);

/* build_point_voxel_map (quantization.py:152-195; write_point_voxel_map,
 * quantization_detail.h:213-331): rows_out int32 [point_rows, 8] and
 * weights_out float32 [point_rows, 8]; interpolation 0 = nearest (corner 0
 * only, weight 1), 1 = linear (eight corners, trilinear weights); -1 / 0
 * where no voxel is found.  Voxel coordinates map to their first row. */
size_t lattice_hip_point_voxel_map_workspace_bytes(int voxel_rows);
int lattice_hip_build_point_voxel_map(
    const float* points, const int32_t* batch_indices, int point_rows,
    const int32_t* point_active, const int32_t* voxel_coords, int voxel_rows,
    const int32_t* voxel_active, const float voxel_size[3],
    const float origin[3], int interpolation, int32_t* rows_out,
    float* weights_out, int32_t* status, void* workspace,
    size_t workspace_bytes, void* stream);

/* interpolate_point_features (quantization.py:198-213; write_point_features,
 * quantization_detail.h:333-361) and its gradient (write_point_feature_grad,
 * :363-391), the latter over the grouping of the map's (point, corner)
 * entries by voxel row (lattice_hip_group_by_key over rows_out). */
int lattice_hip_interpolate_point_features(const float* values,
                                           int voxel_rows, int channels,
                                           const int32_t* rows,
                                           const float* weights,
                                           int point_rows, float* out,
                                           void* stream);
int lattice_hip_interpolate_point_features_grad(const float* point_grad,
                                                int channels,
                                                const float* weights,
                                                const int32_t* voxel_offsets,
                                                const int32_t* entry_ids,
                                                int voxel_rows, float* out,
                                                void* stream);

/* Grouped CSR views of a relation: write_relation_grouped_view
 * (relation_views_detail.h:84-120; relations.cpp:438-476).  Stable
 * partition of the active edge ids by input row and by kernel offset:
 * in_row_offsets [in_capacity + 1], kernel_row_offsets [kernel_count + 1];
 * edge-id arrays [edge_capacity] defined on their first counts[0] entries. */
size_t lattice_hip_relation_grouped_views_workspace_bytes(int edge_capacity);
int lattice_hip_build_relation_grouped_views(
    const int32_t* in_rows, const int32_t* kernel_ids, const int32_t* counts,
    int edge_capacity, int in_capacity, int kernel_count,
    int32_t* in_row_offsets, int32_t* in_edge_ids, int32_t* kernel_row_offsets,
    int32_t* kernel_edge_ids, void* workspace, size_t workspace_bytes,
    void* stream);

/* Dense out_in_map + row masks: write_relation_implicit_gemm_view
 * (relation_views_detail.h:122-169).  offsets: device int32 [K, 3]. */
size_t lattice_hip_implicit_gemm_view_workspace_bytes(int source_rows);
int lattice_hip_build_relation_implicit_gemm_view(
    const int32_t* source_coords, int source_rows,
    const int32_t* source_active_rows, const int32_t* output_coords,
    int output_rows, const int32_t* output_active_rows,
    const int32_t* offsets, int kernel_count, const int stride[3],
    const int padding[3], int32_t* out_in_map, int32_t* row_masks,
    int32_t* status, void* workspace, size_t workspace_bytes, void* stream);

/* Tile-sorted view (core/relations/views.py:467-510): reorder_rows = stable
 * argsort of the single-word row masks; sorted_out_in_map [rows, K] (may be
 * NULL: the same values are the transpose of the K-major view);
 * sorted_kv_out_in_map [K, rows]; tile_masks [ceil(rows/64)*4] = OR of the
 * masks of each 16-row quarter of each 64-row tile.  K <= 32. */
size_t lattice_hip_sorted_view_workspace_bytes(int rows);
int lattice_hip_build_sorted_implicit_gemm_view(
    const int32_t* out_in_map, const int32_t* row_masks, int rows,
    int kernel_count, int32_t* reorder_rows, int32_t* sorted_out_in_map,
    int32_t* sorted_kv_out_in_map, int32_t* tile_masks, void* workspace,
    size_t workspace_bytes, void* stream);

/* Float sparse conv over the output CSR (cpu/algorithms.cpp:180-302):
 * out[o] = sum_{e in CSR(o)} feats[in_rows[e]] @ W[kernel_ids[e]] with an
 * fp32 accumulator; rows >= counts[1] are zero.  feats [n_in, c_in];
 * out [out_capacity, c_out], both in `dtype`.
 * bias (optional, [c_out] in `dtype`, NULL = none) fuses the operator's
 * `feats + bias` (ops/conv.py:460-469) into the store: the conv result is
 * rounded to `dtype`, then the bias is added and the sum rounded again, so
 * the output equals the separate add bit for bit, on every row (rows
 * without edges hold the bias).  The same holds for the two entries
 * below.  epilogue: LATTICE_EPILOGUE_* flags, applied after the bias. */
int lattice_hip_sparse_conv_features(
    int dtype, const void* feats, int n_in, int c_in, const void* weights,
    int weight_layout, int kernel_count, int c_out, const int32_t* in_rows,
    const int32_t* kernel_ids, const int32_t* counts, int edge_capacity,
    const int32_t* row_offsets, int out_capacity, void* out, const void* bias,
    int epilogue, void* stream);

/* The same sum (cpu/algorithms.cpp:180-302; quantized weights as in
 * cpu/quantized.cpp:64-141) for few input channels, over the relation's
 * dense map out_in_map[row * K + k] (input row or -1; the implicit-GEMM
 * view of relation_views_detail.h:122-169) instead of the CSR: a row's K
 * offsets x c_in channels form one contraction on the matrix cores (fp32
 * accumulate; the sum's order differs from the CSR route's, its value
 * does not beyond fp32 rounding).  float16/bfloat16 features with c_in 4
 * or 8 and rows aligned to their size, c_out 16 or 32, K * c_in <= 256
 * (lattice_hip_conv_dense_map_supported); rows >= counts[1] hold the bias
 * alone; bias and epilogue as above.  The quantized entry takes the packed
 * weights, scales and biases of lattice_hip_sparse_quantized_conv_features
 * and dequantises them once per block (w = q * scale + bias,
 * rounded once to the feature dtype). */
int lattice_hip_conv_dense_map_supported(int dtype, int c_in, int c_out,
                                         int kernel_count);
int lattice_hip_sparse_conv_features_dense_map(
    int dtype, const void* feats, int n_in, int c_in, const void* weights,
    int weight_layout, int kernel_count, int c_out, const int32_t* out_in_map,
    const int32_t* counts, int out_capacity, void* out, const void* bias,
    int epilogue, void* stream);
int lattice_hip_sparse_quantized_conv_features_dense_map(
    int dtype, const void* feats, int n_in, int c_in, const uint32_t* weights,
    const void* scales, const void* biases, int kernel_count, int c_out,
    int storage_c_in, int group_size, int bits, const int32_t* out_in_map,
    const int32_t* counts, int out_capacity, void* out, const void* bias,
    int epilogue, void* stream);

/* Implicit-GEMM conv over the sorted view (the reference's sorted plan):
 * row i of the mask-sorted order gathers feats[sorted_kv_out_in_map[k, i]]
 * (-1 = no contribution) for every kernel offset k and writes its result to
 * out[reorder_rows[i]] (row i itself when reorder_rows is NULL).
 * tile_masks[4*t + q] is the OR of the row masks of rows 64t+16q..+15 and
 * decides which offsets a 64-row tile visits.  fp16/bf16 with
 * c_in % 32 == 0, c_out in {16, 32, 64, 128, 256} and K <= 32 run on the
 * matrix cores (fp32 accumulate); other shapes return
 * LATTICE_ERROR_UNSUPPORTED (as do feature tables of 2 GiB or more, whose
 * rows the kernel addresses with 32-bit offsets).  weights: (C_out, Kx, Ky,
 * Kz, C_in).  workspace (optional, lattice_hip_conv_workspace_bytes) holds
 * the launch's tile schedule: with it, row tiles run longest-first; with
 * NULL they run in order.  The result does not depend on the schedule.
 * When workspace_bytes carries LATTICE_CONV_ORDER_READY, the workspace
 * already holds the order lattice_hip_conv_tile_order wrote for the same
 * tile_masks and out_capacity, and the call only reads it (no schedule
 * launch): a caller that keeps the sorted view keeps its order with it. */
#define LATTICE_CONV_ORDER_READY ((size_t)1 << 63)
size_t lattice_hip_conv_workspace_bytes(int out_capacity);
/* Longest-first order of the 128-row tiles of a sorted view (the cost of a
 * tile is the number of offsets its rows use), into `order`
 * (lattice_hip_conv_workspace_bytes(out_capacity) bytes).  No counterpart
 * in the reference: it lets a caller compute the matrix-core conv's tile
 * schedule once per sorted view instead of once per conv call. */
int lattice_hip_conv_tile_order(const int32_t* tile_masks, int out_capacity,
                                int32_t* order, size_t order_bytes,
                                void* stream);
int lattice_hip_sparse_conv_features_sorted_implicit_gemm(
    int dtype, const void* feats, int n_in, int c_in, const void* weights,
    int weight_layout, int kernel_count, int c_out,
    const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks,
    const int32_t* reorder_rows, int out_capacity, void* out, const void* bias,
    int epilogue, void* workspace, size_t workspace_bytes, void* stream);

/* Streamed matrix-core route of the entry above (no counterpart in the
 * reference, which has one conv entry per layout; this one takes the weight
 * already in the kernel's fragment order).  fp16/bf16 features, c_in a
 * multiple of 32 up to 256, c_out in {64, 128, 256}, kernel_count <= 32 and
 * (n_in + 1) * c_in * 2 <= 2^32 bytes of features.  Same sum, output rows,
 * bias, epilogue, workspace and tile order as the entry above; the result is
 * bit-identical to it.  weight_fragments holds
 * lattice_hip_conv_weight_fragments_bytes(...) bytes written by
 * lattice_hip_conv_weight_fragments from the (C_out, Kx, Ky, Kz, C_in)
 * weight; a caller keeps them as long as the weight is unchanged. */
size_t lattice_hip_conv_weight_fragments_bytes(int dtype, int kernel_count,
                                               int c_in, int c_out);
int lattice_hip_conv_weight_fragments(int dtype, const void* weights,
                                      int kernel_count, int c_in, int c_out,
                                      void* fragments, size_t fragments_bytes,
                                      void* stream);
int lattice_hip_sparse_conv_features_sorted_fragments(
    int dtype, const void* feats, int n_in, int c_in,
    const void* weight_fragments, int kernel_count, int c_out,
    const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks,
    const int32_t* reorder_rows, int out_capacity, void* out, const void* bias,
    int epilogue, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of the entry above: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops or harnesses that forbid hipMalloc): the
 * longest-first tile schedule lives in a library-owned device array of
 * 128 KiB per GPU (kept until the process ends), so the call allocates
 * nothing and takes no workspace.  out_capacity must not exceed
 * LATTICE_NOALLOC_CONV_MAX_ROWS (LATTICE_ERROR_INVALID_ARGUMENT otherwise).
 * The calling thread's current device must be the stream's.  Calls on one
 * GPU share the array: outside graph capture each call's stream waits for
 * the previous call's launches (an event the library records, whatever the
 * stream), so calls on different streams run one after another; launches
 * captured into a graph are not ordered, and replays that overlap another
 * use of the array on that GPU race.  Results are bit-identical to the
 * entry above. */
#define LATTICE_NOALLOC_CONV_MAX_ROWS 2097088
int lattice_hip_sparse_conv_features_sorted_implicit_gemm_noalloc(
    int dtype, const void* feats, int n_in, int c_in, const void* weights,
    int weight_layout, int kernel_count, int c_out,
    const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks,
    const int32_t* reorder_rows, int out_capacity, void* out, const void* bias,
    int epilogue, void* stream);

/* Conv over a direct generative / transposed relation (output row
 * in * K + k holds the single edge (in, k); lattice_hip_build_generative_relation
 * and the direct case of lattice_hip_build_transposed_kernel_relation):
 * out[in * K + k] = feats[in] @ W[k] for in < *active_rows, zero rows (plus
 * bias) for the others.  The same sum as the CSR and sorted routes over
 * that relation, as a dense matrix-core GEMM with no gather.  fp16/bf16,
 * c_in, c_out in {32, 64, 128, 256} with c_in * c_out <= 16384; weights (C_out,
 * Kx, Ky, Kz, C_in); out [n_in * K, c_out]; bias and epilogue as above. */
int lattice_hip_sparse_conv_features_expand(
    int dtype, const void* feats, int n_in, const int32_t* active_rows,
    int c_in, const void* weights, int kernel_count, int c_out, void* out,
    const void* bias, int epilogue, void* stream);

/* Quantized conv (cpu/quantized.cpp:64-141): weights uint32
 * [K, storage_c_in*bits/32, c_out] with codes LSB-first along C_in,
 * scales/biases [K, storage_c_in/group_size, c_out] in the feature dtype,
 * w = q*scale + bias, fp32 accumulator.  When sorted_kv_out_in_map,
 * tile_masks and reorder_rows are non-NULL the MFMA route with the dequant
 * fused into the
 * B-operand staging is used (fp16/bf16, c_in % 32 == 0); otherwise the CSR
 * route.  bias and epilogue as for lattice_hip_sparse_conv_features. */
int lattice_hip_sparse_quantized_conv_features(
    int dtype, const void* feats, int n_in, int c_in, const uint32_t* weights,
    const void* scales, const void* biases, int kernel_count, int c_out,
    int storage_c_in, int group_size, int bits, const int32_t* in_rows,
    const int32_t* kernel_ids, const int32_t* counts, int edge_capacity,
    const int32_t* row_offsets, const int32_t* sorted_kv_out_in_map,
    const int32_t* tile_masks, const int32_t* reorder_rows, int out_capacity,
    void* out, const void* bias, int epilogue, void* workspace,
    size_t workspace_bytes, void* stream);

/* Streamed matrix-core route of the quantized conv above (no counterpart in
 * the reference; the dequant stays fused: the packed codes, scale and bias
 * of each B fragment are loaded in one 16-byte load per lane and turned
 * into w = q*scale + bias in registers right before the fragment's MFMAs).
 * Shapes as for lattice_hip_sparse_conv_features_sorted_fragments.
 * weight_fragments holds lattice_hip_quantized_weight_fragments_bytes(...)
 * bytes written by lattice_hip_quantized_weight_fragments from the packed
 * weights, scales and biases (layout of the entry above); a caller keeps
 * them as long as the weight is unchanged.  bits is the weight's (4 or 8). */
size_t lattice_hip_quantized_weight_fragments_bytes(int dtype,
                                                    int kernel_count,
                                                    int c_in, int c_out);
int lattice_hip_quantized_weight_fragments(
    int dtype, const uint32_t* weights, const void* scales,
    const void* biases, int kernel_count, int c_in, int c_out,
    int storage_c_in, int group_size, int bits, void* fragments,
    size_t fragments_bytes, void* stream);
int lattice_hip_sparse_quantized_conv_features_sorted_fragments(
    int dtype, const void* feats, int n_in, int c_in,
    const void* weight_fragments, int bits, int kernel_count, int c_out,
    const int32_t* sorted_kv_out_in_map, const int32_t* tile_masks,
    const int32_t* reorder_rows, int out_capacity, void* out, const void* bias,
    int epilogue, void* workspace, size_t workspace_bytes, void* stream);

/* Input gradient of the float conv (SparseConvFeaturesInputGrad,
 * primitive.cpp:192-260, 597-639; cpu/algorithms.cpp:355-410):
 * grad[in, ci] = sum over the edges of input row `in` in the input-grouped
 * CSR (in_row_offsets [in_capacity + 1], in_edge_ids) and over co of
 * cot[out_rows[e], co] * W[kernel_ids[e], ci, co], fp32 accumulator, one
 * rounding.  cot [out_capacity, c_out]; grad [in_capacity, c_in], both in
 * `dtype`; rows without edges are zero. */
int lattice_hip_sparse_conv_input_grad(
    int dtype, const void* cot, int out_capacity, int c_out,
    const void* weights, int weight_layout, int kernel_count, int c_in,
    const int32_t* out_rows, const int32_t* kernel_ids, const int32_t* counts,
    int edge_capacity, const int32_t* in_row_offsets,
    const int32_t* in_edge_ids, int in_capacity, void* grad, void* stream);

/* Transposed dense map of a forward or submanifold relation, for the
 * input gradient on the matrix cores (no counterpart in the reference, whose
 * Metal route walks the input-grouped CSR): in_out_map [in_capacity, K]
 * holds the output row of edge (in, out, k) or -1, row_masks
 * [in_capacity, ceil(K/32)] its offset bits, in the layout of
 * build_relation_implicit_gemm_view (relations.cpp:498-538).  The sorted
 * view of this map and the implicit-GEMM conv with the weight transposed to
 * (C_in, Kx, Ky, Kz, C_out) then give the input gradient when every
 * (input row, k) has at most one output row.  A submanifold relation over
 * repeated coordinates breaks that (each copy of a coordinate is an output
 * row with the same neighbours): status (int32[1], optional) is cleared
 * and gets LATTICE_STATUS_REPEATED_PAIR when two edges share (in_row, k),
 * and in_out_map then holds one of their output rows (the relation build's
 * LATTICE_STATUS_REPEATED_COORD announces this case in advance; such a
 * relation's input gradient takes lattice_hip_sparse_conv_input_grad). */
int lattice_hip_build_transposed_implicit_gemm_map(
    const int32_t* in_rows, const int32_t* out_rows, const int32_t* kernel_ids,
    const int32_t* counts, int edge_capacity, int in_capacity,
    int kernel_count, int32_t* in_out_map, int32_t* row_masks,
    int32_t* status, void* stream);

/* Weight gradient of the float conv (SparseConvFeaturesWeightGrad,
 * primitive.cpp:403-440, 641-680; cpu/algorithms.cpp:413-481):
 * grad[k, ci, co] = sum over the edges of offset k in the kernel-grouped CSR
 * (kernel_row_offsets [K + 1], kernel_edge_ids) of
 * feats[in_rows[e], ci] * cot[out_rows[e], co], fp32 accumulator, one
 * rounding, written in `weight_layout`.  fp16/bf16 with c_in and c_out
 * multiples of 8 run on the matrix cores and need the workspace
 * (lattice_hip_conv_weight_grad_workspace_bytes, 0 for other shapes); the
 * result is deterministic.  Other shapes take a lane-per-weight kernel. */
size_t lattice_hip_conv_weight_grad_workspace_bytes(int dtype,
                                                    int kernel_count,
                                                    int c_in, int c_out,
                                                    int edge_capacity);
int lattice_hip_sparse_conv_weight_grad(
    int dtype, const void* feats, int n_in, int c_in, const void* cot,
    int out_capacity, int c_out, int weight_layout, int kernel_count,
    const int32_t* in_rows, const int32_t* out_rows, const int32_t* counts,
    int edge_capacity, const int32_t* kernel_row_offsets,
    const int32_t* kernel_edge_ids, void* grad, void* workspace,
    size_t workspace_bytes, void* stream);

/* Sparse pooling over a kernel relation (SparsePoolFeatures,
 * pooling/cpu/algorithms.cpp:180-242; binding sparse_pool_features,
 * bindings/pooling.cpp:15-66).  mode 0 sum, 1 max, 2 avg; fp32 features
 * [n_in, channels].  Every output row starts at the reduction identity
 * (-inf for max, 0 otherwise); rows below counts[1] reduce
 * feats[in_rows[e]] over their CSR edges (row_offsets [out_capacity + 1]);
 * avg divides by max(degree, 1).  out [out_capacity, channels]. */
int lattice_hip_sparse_pool_features(
    int mode, const float* feats, int n_in, int channels,
    const int32_t* in_rows, int edge_capacity, const int32_t* row_offsets,
    const int32_t* counts, int out_capacity, float* out, void* stream);

/* Pooling gradient (the primitive's vjp, pooling/primitive.cpp:109-160,
 * cpu/algorithms.cpp:245-331) over the input-grouped CSR (in_row_offsets
 * [n_in + 1], in_edge_ids): grad[in, c] = sum over the row's edges into out
 * rows below counts[1] of cot[out, c] * scale, scale 1 (sum),
 * 1/max(degree, 1) (avg), and for max 1/(tied inputs of the out row) when
 * feats[in, c] equals pooled[out, c], else 0.  grad [n_in, channels]. */
int lattice_hip_sparse_pool_features_grad(
    int mode, const float* cot, const float* feats, const float* pooled,
    int n_in, int channels, const int32_t* in_rows, const int32_t* out_rows,
    int edge_capacity, const int32_t* row_offsets, const int32_t* counts,
    const int32_t* in_row_offsets, const int32_t* in_edge_ids,
    int out_capacity, float* grad, void* stream);

/* Per-batch global pooling (global_sum_pool / global_avg_pool /
 * global_max_pool, ops/pool.py:139-236): out[b, c] reduces rows
 * batch_offsets[b] .. batch_offsets[b+1] of feats [rows, channels] (fp32);
 * avg divides by the batch's row count (empty batches give zeros for sum and
 * avg; callers reject empty batches for max, as the reference does). */
int lattice_hip_global_pool(int mode, const float* feats, int channels,
                            const int64_t* batch_offsets, int batches,
                            float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LATTICE_HIP_H_ */
