"""Sparse pooling operators (mlx_lattice/ops/pool.py:27-270).

Local pooling builds (or reuses) a forward kernel relation and reduces the
input rows of every output row on the gfx950 pooling kernel; global pooling
reduces each batch of a collated tensor.  Same names, arguments, validation
messages and float32-only contract as the reference.  Local pooling is
differentiable in the features (the reference primitive's vjp,
native/features/pooling/primitive.cpp:109-160), including the max tie policy.
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Literal

import torch

from mlx_lattice_amd.core import KernelSpec, SparseTensor
from mlx_lattice_amd.core.types import Triple
from mlx_lattice_amd.ops._relation_exec import (
    sparse_pool_features_from_relation,
)

PoolMode = Literal['sum', 'max', 'avg']

__all__ = [
    'avg_pool3d',
    'global_avg_pool',
    'global_max_pool',
    'global_sum_pool',
    'max_pool3d',
    'pool3d',
    'sum_pool3d',
]


def pool3d(x: SparseTensor, *, mode: PoolMode = 'sum',
           kernel_size: int | Sequence[int] = 2,
           stride: int | Sequence[int] = 2,
           padding: int | Sequence[int] = 0,
           dilation: int | Sequence[int] = 1) -> SparseTensor:
    """Local sparse 3D pooling with ``sum``, ``max`` or ``avg`` (pool.py:27-55).

    The output sparse stride is ``x.stride * stride``.  Features must be
    float32.
    """
    spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                      dilation=dilation)
    return _fused_pool(x, spec, mode,
                       output_stride=_mul_stride(x.stride, spec.stride))


def sum_pool3d(x: SparseTensor, *, kernel_size: int | Sequence[int] = 2,
               stride: int | Sequence[int] = 2,
               padding: int | Sequence[int] = 0,
               dilation: int | Sequence[int] = 1) -> SparseTensor:
    """Sum of the contributing input rows of each output row."""
    return pool3d(x, mode='sum', kernel_size=kernel_size, stride=stride,
                  padding=padding, dilation=dilation)


def max_pool3d(x: SparseTensor, *, kernel_size: int | Sequence[int] = 2,
               stride: int | Sequence[int] = 2,
               padding: int | Sequence[int] = 0,
               dilation: int | Sequence[int] = 1) -> SparseTensor:
    """Channel-wise maximum over the contributing input rows."""
    return pool3d(x, mode='max', kernel_size=kernel_size, stride=stride,
                  padding=padding, dilation=dilation)


def avg_pool3d(x: SparseTensor, *, kernel_size: int | Sequence[int] = 2,
               stride: int | Sequence[int] = 2,
               padding: int | Sequence[int] = 0,
               dilation: int | Sequence[int] = 1) -> SparseTensor:
    """Sparse sum divided by the number of contributing relation edges."""
    return pool3d(x, mode='avg', kernel_size=kernel_size, stride=stride,
                  padding=padding, dilation=dilation)


def global_sum_pool(x: SparseTensor) -> torch.Tensor:
    """Sum features per batch; needs ``x.batch_counts``; ``(B, C)``."""
    return _batch_reduction(x, 'sum')


def global_avg_pool(x: SparseTensor) -> torch.Tensor:
    """Average features per batch; empty batches give zero rows."""
    return _batch_reduction(x, 'avg')


def global_max_pool(x: SparseTensor) -> torch.Tensor:
    """Max-reduce features per batch; empty batches are rejected."""
    return _batch_reduction(x, 'max')


# ---------------------------------------------------------------- local --


def _fused_pool(x: SparseTensor, spec: KernelSpec, mode: str, *,
                output_stride: Triple) -> SparseTensor:
    _validate_pool_dtype(x.feats)
    if x.coords.dtype != torch.int32:
        raise ValueError('sparse pooling requires int32 coordinates.')
    if mode not in ('sum', 'max', 'avg'):
        raise ValueError("mode must be 'sum', 'max', or 'avg'.")
    relation = x.coord_manager.kernel_relation(
        x.coord_key, kernel_size=spec.size, stride=spec.stride,
        padding=spec.padding, dilation=spec.dilation)
    if relation.n_out_capacity is None or relation.n_kernels is None:
        raise ValueError('kernel relation is missing static shape metadata.')
    if relation.out_coords is None:
        raise ValueError('kernel relation is missing output coordinates.')
    feats = sparse_pool_features_from_relation(
        x.feats, relation, input_exclusive=_input_exclusive(spec), mode=mode)
    return SparseTensor(relation.out_coords, feats, stride=output_stride,
                        coord_manager=x.coord_manager,
                        active_rows=relation.out_count)


# --------------------------------------------------------------- global --


def _batch_reduction(x: SparseTensor, mode: str) -> torch.Tensor:
    _validate_pool_dtype(x.feats)
    if x.batch_counts is None:
        raise ValueError('batch_counts metadata is required for global pooling.')
    counts = tuple(int(c) for c in x.batch_counts)
    if mode == 'max' and any(c == 0 for c in counts):
        raise ValueError('global_max_pool does not support empty batches.')
    if len(counts) == 1:
        # One batch reduces every row (pool.py:200-211).
        counts = (int(x.feats.shape[0]),)
    from mlx_lattice_amd._native import ext

    return ext.global_pool(x.feats, list(counts), mode)


# ----------------------------------------------------------- validation --


def _validate_pool_dtype(feats: torch.Tensor) -> None:
    if feats.dtype != torch.float32:
        raise ValueError('pooling currently supports float32 tensors.')


def _input_exclusive(spec: KernelSpec) -> bool:
    """Each input row feeds at most one output row (pool.py:250-258)."""
    return all(s >= (k - 1) * d + 1 for s, k, d in
               zip(spec.stride, spec.size, spec.dilation, strict=True))


def _mul_stride(lhs: Triple, rhs: Triple) -> Triple:
    return (lhs[0] * rhs[0], lhs[1] * rhs[1], lhs[2] * rhs[2])
