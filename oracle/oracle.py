"""ctypes wrapper over the CPU oracle (``oracle/liblattice_oracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``.  The product path never imports
this module.

Each function restates a reference CPU routine (file:line citations are in
``lattice_oracle.cpp``) over numpy arrays.  Relation outputs follow the
reference's static capacities; the relation-level checks compare only the
active prefixes, as the reference's own parity tests do
(tests/cases/coords_cases.py:60-78).

Pinning (what checks each function besides this restatement):
- kernel_offsets, kernel_relation, target_kernel_relation, grouped_view,
  implicit_gemm_view: the reference's known-answer tests transcribed into
  tests/golden/reference_known_answers.json, plus an independent numpy
  brute-force (dict lookups) on seeded clouds in tests/test_oracle.py.
- conv_features: known answers (tests/ops/test_conv.py:44-83, 326-398,
  638-671) and the textbook identity with a dense 3D cross-correlation on a
  fully occupied box, plus an fp64 edge-sum restatement.
- conv_input_grad, conv_weight_grad: the reference's gradient known
  answers (tests/ops/test_conv.py:401-487), torch autograd of the dense
  conv3d on a fully occupied box, and adjointness with conv_features
  (<conv(x, W), g> = <x, input_grad(g)> = <W, weight_grad(x, g)>).
- pool_features, pool_grad: the reference's pooling known answers
  (tests/ops/test_pool.py:32-117), a numpy brute force and the identity
  sum pooling == conv with all-ones weights.
- quantized_conv_features: the dequantized contract (packed conv equals the
  float conv of the dequantized weight) and the unpack formula on hand-built
  words.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / 'liblattice_oracle.so'
_lib = None

_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags='C_CONTIGUOUS')
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags='C_CONTIGUOUS')
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags='C_CONTIGUOUS')
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags='C_CONTIGUOUS')
_vp = ctypes.c_void_p
_int = ctypes.c_int


def build() -> Path:
    """Compile the oracle with its Makefile (g++ only)."""
    subprocess.run(['make', '-s', '-C', str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(_LIB_PATH))
        handle.oracle_kernel_offsets.argtypes = [_i32p, _i32p, _vp]
        handle.oracle_kernel_offsets.restype = _int
        handle.oracle_kernel_relation.argtypes = [
            _i32p, _int, _int, _i32p, _int, _i32p, _i32p,
            _i32p, _i32p, _i32p, _i32p, _i32p, _i32p]
        handle.oracle_target_kernel_relation.argtypes = [
            _i32p, _int, _int, _i32p, _int, _int, _i32p, _int, _i32p, _i32p,
            _i32p, _i32p, _i32p, _i32p, _i32p]
        handle.oracle_generative_relation.argtypes = [
            _i32p, _int, _int, _i32p, _int, _i32p,
            _i32p, _i32p, _i32p, _i32p, _i32p, _i32p]
        handle.oracle_transposed_kernel_relation.argtypes = [
            _i32p, _int, _int, _i32p, _int, _i32p, _i32p,
            _i32p, _i32p, _i32p, _i32p, _i32p, _i32p]
        handle.oracle_direct_transposed.argtypes = [_i32p, _int, _i32p]
        handle.oracle_direct_transposed.restype = _int
        handle.oracle_grouped_view.argtypes = [
            _i32p, _int, _int, _int, _i32p, _i32p]
        handle.oracle_implicit_gemm_view.argtypes = [
            _i32p, _int, _int, _i32p, _int, _int, _i32p, _int, _i32p, _i32p,
            _i32p, _i32p]
        handle.oracle_conv_features.argtypes = [
            _int, _vp, _vp, _int, _int, _int, _int, _int, _i32p, _i32p,
            _i32p, _int, _i32p, _int, _vp, _int]
        handle.oracle_conv_input_grad.argtypes = [
            _int, _vp, _vp, _int, _int, _int, _int, _int, _i32p, _i32p,
            _i32p, _int, _i32p, _i32p, _int, _vp, _int]
        handle.oracle_conv_weight_grad.argtypes = [
            _int, _vp, _vp, _int, _int, _int, _int, _i32p, _i32p, _i32p,
            _int, _i32p, _i32p, _int, _vp, _int]
        handle.oracle_pool_features.argtypes = [
            _int, _f32p, _int, _i32p, _i32p, _i32p, _int, _f32p]
        handle.oracle_pool_grad.argtypes = [
            _int, _f32p, _f32p, _f32p, _int, _i32p, _i32p, _i32p, _i32p,
            _i32p, _i32p, _int, _int, _f32p]
        handle.oracle_quantized_conv_features.argtypes = [
            _int, _vp, _u32p, _vp, _vp, _int, _int, _int, _int, _int, _int,
            _i32p, _i32p, _i32p, _int, _i32p, _int, _vp, _int]
        handle.oracle_dequantize_mapped.argtypes = [
            _u32p, _f32p, _f32p, _int, _int, _int, _int, _int, _int, _f32p]
        handle.oracle_sparse_quantize.argtypes = [
            _f32p, _i32p, _int, _int, _f32p, _f32p, _i32p, _i32p, _i32p]
        handle.oracle_sparse_quantize.restype = _int
        handle.oracle_voxelize_features.argtypes = [
            _int, _f32p, _int, _int, _int, _i32p, _i32p, _int, _f32p]
        handle.oracle_voxelize_features_grad.argtypes = [
            _int, _f32p, _int, _int, _int, _i32p, _i32p, _int, _f32p]
        handle.oracle_point_voxel_map.argtypes = [
            _f32p, _i32p, _int, _int, _i32p, _int, _int, _f32p, _f32p, _int,
            _i32p, _f32p]
        handle.oracle_point_features.argtypes = [
            _f32p, _int, _int, _i32p, _f32p, _int, _f32p]
        handle.oracle_point_features_grad.argtypes = [
            _f32p, _int, _int, _i32p, _f32p, _int, _f32p]
        handle.oracle_hardware_concurrency.restype = _int
        _lib = handle
    return _lib


def hardware_concurrency() -> int:
    return int(lib().oracle_hardware_concurrency())


def _triple(v) -> np.ndarray:
    if isinstance(v, int):
        v = (v, v, v)
    return np.ascontiguousarray(v, dtype=np.int32)


def kernel_offsets(kernel_size, dilation=1) -> np.ndarray:
    size = _triple(kernel_size)
    dil = _triple(dilation)
    k = lib().oracle_kernel_offsets(size, dil, None)
    out = np.zeros((k, 3), dtype=np.int32)
    lib().oracle_kernel_offsets(size, dil, out.ctypes.data)
    return out


def kernel_relation(coords: np.ndarray, active_rows: int | None = None,
                    kernel_size=3, stride=1, padding=0, dilation=1) -> dict:
    """Forward relation (identity out when stride=1, padding=0)."""
    coords = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
    rows = coords.shape[0]
    active = rows if active_rows is None else int(active_rows)
    offs = kernel_offsets(kernel_size, dilation)
    k = offs.shape[0]
    out = dict(
        in_rows=np.zeros(rows * k, np.int32),
        out_rows=np.zeros(rows * k, np.int32),
        kernel_ids=np.zeros(rows * k, np.int32),
        row_offsets=np.zeros(rows + 1, np.int32),
        out_coords=np.zeros((rows, 4), np.int32),
        counts=np.zeros(2, np.int32),
    )
    lib().oracle_kernel_relation(
        coords, rows, active, offs, k, _triple(stride), _triple(padding),
        out['in_rows'], out['out_rows'], out['kernel_ids'],
        out['row_offsets'], out['out_coords'], out['counts'])
    _add_views(out, rows, k)
    return out


def target_kernel_relation(coords, target, active_rows=None,
                           target_active_rows=None, kernel_size=3, stride=1,
                           padding=0, dilation=1) -> dict:
    coords = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
    target = np.ascontiguousarray(target, dtype=np.int32).reshape(-1, 4)
    rows, trows = coords.shape[0], target.shape[0]
    active = rows if active_rows is None else int(active_rows)
    tactive = trows if target_active_rows is None else int(target_active_rows)
    offs = kernel_offsets(kernel_size, dilation)
    k = offs.shape[0]
    out = dict(
        in_rows=np.zeros(trows * k, np.int32),
        out_rows=np.zeros(trows * k, np.int32),
        kernel_ids=np.zeros(trows * k, np.int32),
        row_offsets=np.zeros(trows + 1, np.int32),
        out_coords=target.copy(),
        counts=np.zeros(2, np.int32),
    )
    lib().oracle_target_kernel_relation(
        coords, rows, active, target, trows, tactive, offs, k,
        _triple(stride), _triple(padding), out['in_rows'], out['out_rows'],
        out['kernel_ids'], out['row_offsets'], out['counts'])
    _add_views(out, rows, k)
    return out


def _expanded_relation(fn, coords, active_rows, kernel_size, stride,
                       padding, dilation) -> dict:
    coords = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 4)
    rows = coords.shape[0]
    active = rows if active_rows is None else int(active_rows)
    offs = kernel_offsets(kernel_size, dilation)
    k = offs.shape[0]
    cap = rows * k
    out = dict(
        in_rows=np.zeros(cap, np.int32),
        out_rows=np.zeros(cap, np.int32),
        kernel_ids=np.zeros(cap, np.int32),
        row_offsets=np.zeros(cap + 1, np.int32),
        out_coords=np.zeros((cap, 4), np.int32),
        counts=np.zeros(2, np.int32),
    )
    args = [coords, rows, active, offs, k, _triple(stride)]
    if padding is not None:
        args.append(_triple(padding))
    fn(*args, out['in_rows'], out['out_rows'], out['kernel_ids'],
       out['row_offsets'], out['out_coords'], out['counts'])
    _add_views(out, rows, k)
    return out


def generative_relation(coords, active_rows=None, kernel_size=2,
                        stride=2) -> dict:
    """write_generative_relation (relation_build_detail.h:82-117)."""
    return _expanded_relation(lib().oracle_generative_relation, coords,
                              active_rows, kernel_size, stride, None, 1)


def transposed_kernel_relation(coords, active_rows=None, kernel_size=2,
                               stride=2, padding=0, dilation=1) -> dict:
    """write_transposed_kernel_relation (relation_build_detail.h:119-196)."""
    return _expanded_relation(lib().oracle_transposed_kernel_relation, coords,
                              active_rows, kernel_size, stride, padding,
                              dilation)


def direct_transposed(kernel_size, stride, dilation=1) -> bool:
    offs = kernel_offsets(kernel_size, dilation)
    return bool(lib().oracle_direct_transposed(offs, offs.shape[0],
                                               _triple(stride)))


def grouped_view(group_ids: np.ndarray, edge_count: int, group_count: int):
    group_ids = np.ascontiguousarray(group_ids, dtype=np.int32)
    offsets = np.zeros(group_count + 1, np.int32)
    edge_ids = np.zeros(group_ids.shape[0], np.int32)
    lib().oracle_grouped_view(group_ids, group_ids.shape[0], int(edge_count),
                              group_count, offsets, edge_ids)
    return offsets, edge_ids


def _add_views(out: dict, in_capacity: int, k: int) -> None:
    e = int(out['counts'][0])
    out['in_row_offsets'], out['in_edge_ids'] = grouped_view(
        out['in_rows'], e, in_capacity)
    out['kernel_row_offsets'], out['kernel_edge_ids'] = grouped_view(
        out['kernel_ids'], e, k)


def implicit_gemm_view(source_coords, source_active, output_coords,
                       output_active, offsets, stride=1, padding=0):
    src = np.ascontiguousarray(source_coords, dtype=np.int32).reshape(-1, 4)
    dst = np.ascontiguousarray(output_coords, dtype=np.int32).reshape(-1, 4)
    offs = np.ascontiguousarray(offsets, dtype=np.int32).reshape(-1, 3)
    k = offs.shape[0]
    words = (k + 31) // 32
    out_in_map = np.zeros((dst.shape[0], k), np.int32)
    row_masks = np.zeros((dst.shape[0], words), np.int32)
    lib().oracle_implicit_gemm_view(
        src, src.shape[0], int(source_active), dst, dst.shape[0],
        int(output_active), offs, k, _triple(stride), _triple(padding),
        out_in_map, row_masks)
    return out_in_map, row_masks


def conv_features(feats: np.ndarray, weight: np.ndarray, relation: dict,
                  out_capacity: int | None = None,
                  threads: int = 0) -> np.ndarray:
    """Reference CPU float conv (fp32 or fp16 feats; 5D or mapped weight)."""
    feats = np.ascontiguousarray(feats)
    weight = np.ascontiguousarray(weight)
    if feats.dtype == np.float32:
        dtype = 0
    elif feats.dtype == np.float16:
        dtype = 1
    else:
        raise ValueError('oracle conv supports float32 and float16.')
    if weight.dtype != feats.dtype:
        raise ValueError('weight dtype must match feats.')
    if weight.ndim == 5:
        layout, k, c_out = 1, int(np.prod(weight.shape[1:4])), weight.shape[0]
    elif weight.ndim == 3:
        layout, k, c_out = 0, weight.shape[0], weight.shape[2]
    else:
        raise ValueError('weight must be 3D or 5D.')
    c_in = feats.shape[1]
    cap = (relation['row_offsets'].shape[0] - 1
           if out_capacity is None else out_capacity)
    out = np.zeros((cap, c_out), dtype=feats.dtype)
    lib().oracle_conv_features(
        dtype, feats.ctypes.data, weight.ctypes.data, layout, feats.shape[0],
        c_in, c_out, k, relation['in_rows'], relation['kernel_ids'],
        relation['counts'], relation['in_rows'].shape[0],
        relation['row_offsets'], cap, out.ctypes.data, int(threads))
    return out


def _float_dtype(arr: np.ndarray) -> int:
    if arr.dtype == np.float32:
        return 0
    if arr.dtype == np.float16:
        return 1
    raise ValueError('oracle gradients support float32 and float16.')


def _weight_layout(weight_shape) -> tuple[int, int, int, int]:
    """(layout, K, C_in, C_out) of a 5D or mapped weight shape."""
    if len(weight_shape) == 5:
        return 1, int(np.prod(weight_shape[1:4])), weight_shape[4], weight_shape[0]
    if len(weight_shape) == 3:
        return 0, weight_shape[0], weight_shape[1], weight_shape[2]
    raise ValueError('weight must be 3D or 5D.')


def conv_input_grad(cot: np.ndarray, weight: np.ndarray, relation: dict,
                    in_capacity: int, threads: int = 0) -> np.ndarray:
    """Reference CPU input gradient (eval_input_grad_typed): ``(in_capacity,
    C_in)`` in the cotangent dtype."""
    cot = np.ascontiguousarray(cot)
    weight = np.ascontiguousarray(weight, dtype=cot.dtype)
    layout, k, c_in, c_out = _weight_layout(weight.shape)
    grad = np.zeros((in_capacity, c_in), dtype=cot.dtype)
    lib().oracle_conv_input_grad(
        _float_dtype(cot), cot.ctypes.data, weight.ctypes.data, layout,
        in_capacity, c_in, c_out, k, relation['out_rows'],
        relation['kernel_ids'], relation['counts'],
        relation['in_rows'].shape[0], relation['in_row_offsets'],
        relation['in_edge_ids'], cot.shape[0], grad.ctypes.data, int(threads))
    return grad


def conv_weight_grad(feats: np.ndarray, cot: np.ndarray, weight_shape,
                     relation: dict, threads: int = 0) -> np.ndarray:
    """Reference CPU weight gradient (eval_weight_grad_typed), in the
    weight's shape and the cotangent dtype."""
    feats = np.ascontiguousarray(feats)
    cot = np.ascontiguousarray(cot, dtype=feats.dtype)
    layout, k, c_in, c_out = _weight_layout(tuple(weight_shape))
    grad = np.zeros(tuple(weight_shape), dtype=cot.dtype)
    lib().oracle_conv_weight_grad(
        _float_dtype(cot), feats.ctypes.data, cot.ctypes.data, layout, c_in,
        c_out, k, relation['in_rows'], relation['out_rows'],
        relation['counts'], relation['in_rows'].shape[0],
        relation['kernel_row_offsets'], relation['kernel_edge_ids'],
        cot.shape[0], grad.ctypes.data, int(threads))
    return grad


_POOL_MODES = {'sum': 0, 'max': 1, 'avg': 2}


def pool_features(feats: np.ndarray, relation: dict, mode: str,
                  out_capacity: int | None = None) -> np.ndarray:
    """Reference CPU sparse pooling (pooling/cpu/algorithms.cpp eval)."""
    feats = np.ascontiguousarray(feats, dtype=np.float32)
    cap = (relation['row_offsets'].shape[0] - 1
           if out_capacity is None else out_capacity)
    out = np.zeros((cap, feats.shape[1]), np.float32)
    lib().oracle_pool_features(_POOL_MODES[mode], feats, feats.shape[1],
                               relation['in_rows'], relation['row_offsets'],
                               relation['counts'], cap, out)
    return out


def pool_grad(cot: np.ndarray, feats: np.ndarray, pooled: np.ndarray,
              relation: dict, mode: str) -> np.ndarray:
    """Reference CPU pooling gradient (pooling/cpu/algorithms.cpp
    eval_grad) over the input-grouped CSR."""
    cot = np.ascontiguousarray(cot, dtype=np.float32)
    feats = np.ascontiguousarray(feats, dtype=np.float32)
    pooled = np.ascontiguousarray(pooled, dtype=np.float32)
    grad = np.zeros(feats.shape, np.float32)
    lib().oracle_pool_grad(
        _POOL_MODES[mode], cot, feats, pooled, feats.shape[1],
        relation['in_rows'], relation['out_rows'], relation['row_offsets'],
        relation['counts'], relation['in_row_offsets'],
        relation['in_edge_ids'], feats.shape[0], cot.shape[0], grad)
    return grad


def quantized_conv_features(feats, weights, scales, biases, relation: dict,
                            *, in_channels, out_channels, storage_in_channels,
                            group_size, bits, out_capacity=None,
                            threads: int = 0) -> np.ndarray:
    feats = np.ascontiguousarray(feats)
    dtype = 0 if feats.dtype == np.float32 else 1
    scales = np.ascontiguousarray(scales, dtype=feats.dtype)
    biases = np.ascontiguousarray(biases, dtype=feats.dtype)
    weights = np.ascontiguousarray(weights, dtype=np.uint32)
    cap = (relation['row_offsets'].shape[0] - 1
           if out_capacity is None else out_capacity)
    out = np.zeros((cap, out_channels), dtype=feats.dtype)
    lib().oracle_quantized_conv_features(
        dtype, feats.ctypes.data, weights, scales.ctypes.data,
        biases.ctypes.data, in_channels, out_channels, storage_in_channels,
        group_size, bits, weights.shape[0], relation['in_rows'],
        relation['kernel_ids'], relation['counts'],
        relation['in_rows'].shape[0], relation['row_offsets'], cap,
        out.ctypes.data, int(threads))
    return out


def dequantize_mapped(weights, scales, biases, *, in_channels, out_channels,
                      storage_in_channels, group_size, bits) -> np.ndarray:
    weights = np.ascontiguousarray(weights, dtype=np.uint32)
    k = weights.shape[0]
    out = np.zeros((k, in_channels, out_channels), np.float32)
    lib().oracle_dequantize_mapped(
        weights, np.ascontiguousarray(scales, np.float32),
        np.ascontiguousarray(biases, np.float32), k, in_channels,
        out_channels, storage_in_channels, group_size, bits, out)
    return out


def conv_features_fp64(feats, weight_mapped, relation: dict,
                       out_capacity: int | None = None) -> np.ndarray:
    """Exact-order-free fp64 edge sum ``out[o] += f[in] @ W[k]``.

    Independent of the C restatement: a numpy scatter-add over the active
    edge prefix, used as the tolerance anchor for float features.
    """
    e = int(relation['counts'][0])
    n_out = int(relation['counts'][1])
    cap = (relation['row_offsets'].shape[0] - 1
           if out_capacity is None else out_capacity)
    w = np.asarray(weight_mapped, dtype=np.float64)
    f = np.asarray(feats, dtype=np.float64)
    ins = relation['in_rows'][:e]
    outs = relation['out_rows'][:e]
    ks = relation['kernel_ids'][:e]
    out = np.zeros((cap, w.shape[2]), np.float64)
    for k in range(w.shape[0]):
        sel = ks == k
        if not sel.any():
            continue
        np.add.at(out, outs[sel], f[ins[sel]] @ w[k])
    out[n_out:] = 0.0
    return out


def mapped_weight(weight: np.ndarray) -> np.ndarray:
    """(C_out, Kx, Ky, Kz, C_in) -> (K, C_in, C_out)
    (ops/_relation_exec.py:217-250)."""
    if weight.ndim == 3:
        return weight
    c_out = weight.shape[0]
    c_in = weight.shape[4]
    return np.ascontiguousarray(
        weight.transpose(1, 2, 3, 4, 0).reshape(-1, c_in, c_out))



# ------------------------------------------------- point quantization ----


def _ftriple(v) -> np.ndarray:
    if isinstance(v, (int, float)):
        v = (v, v, v)
    return np.ascontiguousarray(v, dtype=np.float32)


def _batches(batch_indices, rows):
    if batch_indices is None:
        return np.zeros(rows, np.int32)
    return np.ascontiguousarray(batch_indices, dtype=np.int32)


def sparse_quantize(points, voxel_size=1.0, batch_indices=None, origin=0.0,
                    active_rows=None) -> dict:
    """write_sparse_quantization (quantization_detail.h:91-128)."""
    pts = np.ascontiguousarray(points, dtype=np.float32).reshape(-1, 3)
    rows = pts.shape[0]
    active = rows if active_rows is None else int(active_rows)
    out = dict(coords=np.zeros((rows, 4), np.int32),
               inverse_rows=np.zeros(rows, np.int32),
               counts=np.zeros(rows, np.int32))
    n = lib().oracle_sparse_quantize(
        pts, _batches(batch_indices, rows), rows, active,
        _ftriple(voxel_size), _ftriple(origin), out['coords'],
        out['inverse_rows'], out['counts'])
    out['active_rows'] = np.array([n], np.int32)
    return out


_VOXEL_MODES = {'sum': 0, 'mean': 1}


def voxelize_features(feats, inverse_rows, counts, reduction='mean',
                      active_rows=None) -> np.ndarray:
    f = np.ascontiguousarray(feats, dtype=np.float32)
    rows, channels = f.shape
    active = rows if active_rows is None else int(active_rows)
    counts = np.ascontiguousarray(counts, dtype=np.int32)
    out = np.zeros((counts.shape[0], channels), np.float32)
    lib().oracle_voxelize_features(
        _VOXEL_MODES[reduction], f, rows, active, channels,
        np.ascontiguousarray(inverse_rows, dtype=np.int32), counts,
        counts.shape[0], out)
    return out


def voxelize_features_grad(cot, inverse_rows, counts, point_rows,
                           reduction='mean', active_rows=None) -> np.ndarray:
    g = np.ascontiguousarray(cot, dtype=np.float32)
    channels = g.shape[1]
    active = point_rows if active_rows is None else int(active_rows)
    out = np.zeros((point_rows, channels), np.float32)
    lib().oracle_voxelize_features_grad(
        _VOXEL_MODES[reduction], g, point_rows, active, channels,
        np.ascontiguousarray(inverse_rows, dtype=np.int32),
        np.ascontiguousarray(counts, dtype=np.int32), g.shape[0], out)
    return out


def point_voxel_map(points, voxel_coords, voxel_active=None, voxel_size=1.0,
                    batch_indices=None, point_active=None, origin=0.0,
                    interpolation='linear'):
    """write_point_voxel_map (quantization_detail.h:213-331)."""
    pts = np.ascontiguousarray(points, dtype=np.float32).reshape(-1, 3)
    vox = np.ascontiguousarray(voxel_coords, dtype=np.int32).reshape(-1, 4)
    n = pts.shape[0]
    rows = np.zeros((n, 8), np.int32)
    weights = np.zeros((n, 8), np.float32)
    lib().oracle_point_voxel_map(
        pts, _batches(batch_indices, n), n,
        n if point_active is None else int(point_active), vox, vox.shape[0],
        vox.shape[0] if voxel_active is None else int(voxel_active),
        _ftriple(voxel_size), _ftriple(origin),
        {'nearest': 0, 'linear': 1}[interpolation], rows, weights)
    return rows, weights


def point_features(values, rows, weights) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    out = np.zeros((rows.shape[0], v.shape[1]), np.float32)
    lib().oracle_point_features(v, v.shape[0], v.shape[1], rows,
                                np.ascontiguousarray(weights, np.float32),
                                rows.shape[0], out)
    return out


def point_features_grad(point_grad, rows, weights, voxel_rows) -> np.ndarray:
    g = np.ascontiguousarray(point_grad, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    out = np.zeros((voxel_rows, g.shape[1]), np.float32)
    lib().oracle_point_features_grad(g, voxel_rows, g.shape[1], rows,
                                     np.ascontiguousarray(weights, np.float32),
                                     rows.shape[0], out)
    return out
