"""Point <-> voxel operators (mlx_lattice/ops/quantization.py:33-221):
``voxelize`` quantizes points and aggregates their features into a sparse
voxel tensor, ``voxelize_with_quantization`` reuses a quantization, and
``devoxelize`` samples voxel features back at points."""

from __future__ import annotations

from collections.abc import Sequence

import torch

from mlx_lattice_amd.core.coords.quantization import (
    PointVoxelInterpolation,
    PointVoxelMap,
    SparseQuantization,
    _validate_reduction,
    build_point_voxel_map,
    interpolate_point_features,
    sparse_quantize,
    voxelize_features,
)
from mlx_lattice_amd.core.tensor import SparseTensor
from mlx_lattice_amd.core.types import triple

__all__ = [
    'build_point_voxel_map',
    'devoxelize',
    'interpolate_point_features',
    'sparse_quantize',
    'voxelize',
    'voxelize_with_quantization',
]


def voxelize(points: torch.Tensor, feats: torch.Tensor,
             voxel_size: float | Sequence[float] = 1.0, *,
             batch_indices: torch.Tensor | None = None,
             origin: float | Sequence[float] = 0.0,
             active_rows: torch.Tensor | None = None,
             reduction: str = 'mean',
             stride: int | Sequence[int] = 1) -> SparseTensor:
    """Quantize points and aggregate features into a sparse voxel tensor
    with coordinates ``(batch, floor((point - origin) / voxel_size))``
    (ops/quantization.py:61-99)."""
    if feats.ndim != 2:
        raise ValueError('feats must have shape (N, C).')
    if points.shape[0] != feats.shape[0]:
        raise ValueError('points and feats must have matching rows.')
    reduction = _validate_reduction(reduction)
    quantization = sparse_quantize(points, voxel_size,
                                   batch_indices=batch_indices,
                                   origin=origin, active_rows=active_rows)
    return voxelize_with_quantization(quantization, feats,
                                      active_rows=active_rows,
                                      reduction=reduction, stride=stride)


def voxelize_with_quantization(quantization: SparseQuantization,
                               feats: torch.Tensor, *,
                               active_rows: torch.Tensor | None = None,
                               reduction: str = 'mean',
                               stride: int | Sequence[int] = 1,
                               template: SparseTensor | None = None
                               ) -> SparseTensor:
    """Apply a precomputed quantization to feature rows
    (ops/quantization.py:128-168); a ``template`` must share the
    quantization's coordinate and active-row arrays."""
    voxel_feats = voxelize_features(feats, quantization,
                                    active_rows=active_rows,
                                    reduction=_validate_reduction(reduction))
    if template is not None:
        if template.coords is not quantization.coords:
            raise ValueError(
                'template must use the quantization coordinate array.')
        if template.active_rows is not quantization.active_rows:
            raise ValueError(
                'template must use the quantization active_rows array.')
        return template.replace(feats=voxel_feats)
    return SparseTensor(quantization.coords, voxel_feats,
                        stride=triple(stride, name='stride'),
                        active_rows=quantization.active_rows)


def devoxelize(points: torch.Tensor, voxels: SparseTensor,
               voxel_size: float | Sequence[float] = 1.0, *,
               batch_indices: torch.Tensor | None = None,
               point_active_rows: torch.Tensor | None = None,
               origin: float | Sequence[float] = 0.0,
               interpolation: PointVoxelInterpolation = 'linear',
               point_voxel_map: PointVoxelMap | None = None) -> torch.Tensor:
    """Sample sparse voxel features back onto dense point rows
    (ops/quantization.py:171-205)."""
    point_map = point_voxel_map
    if point_map is None:
        point_map = build_point_voxel_map(
            points, voxels.coords, voxels.active_rows, voxel_size,
            batch_indices=batch_indices, point_active_rows=point_active_rows,
            origin=origin, interpolation=interpolation)
    return interpolate_point_features(voxels.feats, point_map)


