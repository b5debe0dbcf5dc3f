"""Point -> voxel quantization and point <-> voxel feature maps
(mlx_lattice/core/coords/quantization.py:16-270) over the gfx950 kernels.

``sparse_quantize`` voxelizes float32 points into first-seen ordered voxel
coordinates with inverse rows and per-voxel counts; ``voxelize_features``
aggregates point features into voxels (sum / mean); ``build_point_voxel_map``
and ``interpolate_point_features`` sample voxel features back at points
(nearest / trilinear).  Both feature maps are differentiable through torch
autograd with the reference's gradients (quantization_detail.h:172-200,
363-391).  The voxel -> points and voxel -> (point, corner) groupings the
deterministic kernels need are built on first use and cached on the
quantization / map object.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field
from typing import Literal

import torch

from mlx_lattice_amd.core.coords.validation import validate_coords

VoxelReduction = Literal['sum', 'mean']
PointVoxelInterpolation = Literal['nearest', 'linear']

__all__ = [
    'PointVoxelInterpolation',
    'PointVoxelMap',
    'SparseQuantization',
    'VoxelReduction',
    'build_point_voxel_map',
    'interpolate_point_features',
    'sparse_quantize',
    'voxelize_features',
]


def _ext():
    from mlx_lattice_amd._native import ext

    return ext


@dataclass(frozen=True, eq=False)
class SparseQuantization:
    """Unique voxel coordinates ``(batch, x, y, z)`` plus point -> voxel
    metadata (quantization.py:16-57): ``inverse_rows`` maps each point row
    to its voxel row (-1 for inactive points) and ``counts`` holds the
    number of active points per voxel."""

    coords: torch.Tensor
    active_rows: torch.Tensor
    inverse_rows: torch.Tensor
    counts: torch.Tensor
    _grouping: dict = field(default_factory=dict, repr=False, compare=False)

    def __post_init__(self) -> None:
        validate_coords(self.coords)
        if self.coords.dtype != torch.int32:
            raise ValueError('quantized coords must be int32.')
        if (tuple(self.active_rows.shape) != (1,)
                or self.active_rows.dtype != torch.int32):
            raise ValueError(
                'active_rows must have shape (1,) and int32 dtype.')
        if (tuple(self.inverse_rows.shape) != (self.coords.shape[0],)
                or self.inverse_rows.dtype != torch.int32):
            raise ValueError(
                'inverse_rows must have shape (N,) and int32 dtype.')
        if (tuple(self.counts.shape) != (self.coords.shape[0],)
                or self.counts.dtype != torch.int32):
            raise ValueError('counts must have shape (N,) and int32 dtype.')

    @property
    def capacity(self) -> int:
        return int(self.coords.shape[0])

    @property
    def active_count(self) -> torch.Tensor:
        return self.active_rows

    def voxel_groups(self, point_active_rows: torch.Tensor | None
                     ) -> tuple[torch.Tensor, torch.Tensor]:
        """(voxel_offsets, point_ids): the points of every voxel in point
        order, limited to the first ``point_active_rows`` points when given.
        The grouping over all points is cached; one grouping for a given
        active-row tensor is kept (matched by identity)."""
        key = 'all' if point_active_rows is None else 'active'
        cached = self._grouping.get(key)
        if cached is None or cached[0] is not point_active_rows:
            offsets, ids = _ext().group_by_key(
                self.inverse_rows, point_active_rows, self.capacity)
            cached = (point_active_rows, offsets, ids)
            self._grouping[key] = cached
        return cached[1], cached[2]


@dataclass(frozen=True, eq=False)
class PointVoxelMap:
    """Fixed-width point -> voxel interpolation rows and weights
    (quantization.py:60-88), both ``(N, 8)``."""

    rows: torch.Tensor
    weights: torch.Tensor
    _grouping: dict = field(default_factory=dict, repr=False, compare=False)

    def __post_init__(self) -> None:
        if (self.rows.ndim != 2 or self.rows.shape[1] != 8
                or self.rows.dtype != torch.int32):
            raise ValueError('rows must have shape (N, 8) and int32 dtype.')
        if tuple(self.weights.shape) != tuple(self.rows.shape):
            raise ValueError('weights must have the same shape as rows.')
        if self.weights.dtype != torch.float32:
            raise ValueError('weights must be float32.')

    @property
    def point_count(self) -> int:
        return int(self.rows.shape[0])

    def voxel_entries(self, voxel_rows: int
                      ) -> tuple[torch.Tensor, torch.Tensor]:
        """(voxel_offsets, entry_ids): the (point, corner) entries
        ``point * 8 + corner`` hitting every voxel, in entry order."""
        cached = self._grouping.get(voxel_rows)
        if cached is None:
            cached = _ext().group_by_key(self.rows.reshape(-1), None,
                                         voxel_rows)
            self._grouping[voxel_rows] = cached
        return cached


def sparse_quantize(points: torch.Tensor,
                    voxel_size: float | Sequence[float] = 1.0, *,
                    batch_indices: torch.Tensor | None = None,
                    origin: float | Sequence[float] = 0.0,
                    active_rows: torch.Tensor | None = None
                    ) -> SparseQuantization:
    """Voxelize float32 points ``(N, 3)`` (quantization.py:91-118)."""
    _validate_points(points)
    batches = _batch_indices(batch_indices, points)
    rows = _active_rows(active_rows, points)
    native = _ext().sparse_quantize(
        points, batches, rows, list(_float_triple(voxel_size, 'voxel_size')),
        list(_float_triple(origin, 'origin')))
    return SparseQuantization(*native)


def voxelize_features(feats: torch.Tensor, quantization: SparseQuantization,
                      *, active_rows: torch.Tensor | None = None,
                      reduction: VoxelReduction = 'mean') -> torch.Tensor:
    """Aggregate float32 point features into voxels (quantization.py:
    121-149): ``sum`` adds the point rows, ``mean`` divides each by its
    voxel count.  Differentiable in ``feats``."""
    if feats.ndim != 2:
        raise ValueError('feats must have shape (N, C).')
    if feats.dtype != torch.float32:
        raise ValueError('voxelize currently supports float32 features.')
    if feats.shape[0] != quantization.capacity:
        raise ValueError('feats and quantization metadata must share rows.')
    reduction = _validate_reduction(reduction)
    if active_rows is not None:
        _active_rows(active_rows, feats)
    if torch.is_grad_enabled() and feats.requires_grad:
        return _VoxelizeFeatures.apply(feats, quantization, active_rows,
                                       reduction)
    return _voxelize(feats, quantization, active_rows, reduction)


def _voxelize(feats, quantization, rows, reduction):
    offsets, ids = quantization.voxel_groups(rows)
    return _ext().voxelize_features_grouped(
        feats.contiguous(), quantization.counts, offsets, ids, reduction)


class _VoxelizeFeatures(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, quantization, rows, reduction):
        ctx.quantization = quantization
        ctx.rows = rows
        ctx.reduction = reduction
        ctx.point_rows = int(feats.shape[0])
        return _voxelize(feats, quantization, rows, reduction)

    @staticmethod
    def backward(ctx, grad_out):
        q = ctx.quantization
        rows = ctx.rows
        if rows is None:
            rows = torch.full((1,), ctx.point_rows, dtype=torch.int32,
                              device=grad_out.device)
        grad = _ext().voxelize_features_grad(
            grad_out.contiguous(), q.inverse_rows, q.counts, rows,
            ctx.point_rows, ctx.reduction)
        return grad, None, None, None


def build_point_voxel_map(points: torch.Tensor, voxel_coords: torch.Tensor,
                          voxel_active_rows: torch.Tensor,
                          voxel_size: float | Sequence[float] = 1.0, *,
                          batch_indices: torch.Tensor | None = None,
                          point_active_rows: torch.Tensor | None = None,
                          origin: float | Sequence[float] = 0.0,
                          interpolation: PointVoxelInterpolation = 'linear'
                          ) -> PointVoxelMap:
    """Fixed-width rows and weights from points to voxel centres
    (quantization.py:152-195)."""
    _validate_points(points)
    validate_coords(voxel_coords)
    if voxel_coords.dtype != torch.int32:
        raise ValueError('voxel_coords must be int32.')
    batches = _batch_indices(batch_indices, points)
    rows = _active_rows(point_active_rows, points)
    if (tuple(voxel_active_rows.shape) != (1,)
            or voxel_active_rows.dtype != torch.int32):
        raise ValueError(
            'voxel_active_rows must have shape (1,) and int32 dtype.')
    native = _ext().build_point_voxel_map(
        points, batches, rows, voxel_coords, voxel_active_rows,
        list(_float_triple(voxel_size, 'voxel_size')),
        list(_float_triple(origin, 'origin')),
        _validate_interpolation(interpolation))
    return PointVoxelMap(*native)


def interpolate_point_features(voxel_feats: torch.Tensor,
                               point_voxel_map: PointVoxelMap
                               ) -> torch.Tensor:
    """Sample float32 voxel features at the points of a map
    (quantization.py:198-213); differentiable in ``voxel_feats``."""
    if voxel_feats.ndim != 2:
        raise ValueError('voxel_feats must have shape (N, C).')
    if voxel_feats.dtype != torch.float32:
        raise ValueError('point interpolation currently supports float32.')
    if torch.is_grad_enabled() and voxel_feats.requires_grad:
        return _InterpolatePointFeatures.apply(voxel_feats, point_voxel_map)
    return _ext().interpolate_point_features(
        voxel_feats, point_voxel_map.rows, point_voxel_map.weights)


class _InterpolatePointFeatures(torch.autograd.Function):
    @staticmethod
    def forward(ctx, voxel_feats, point_voxel_map):
        ctx.point_voxel_map = point_voxel_map
        ctx.voxel_rows = int(voxel_feats.shape[0])
        return _ext().interpolate_point_features(
            voxel_feats, point_voxel_map.rows, point_voxel_map.weights)

    @staticmethod
    def backward(ctx, grad_out):
        m = ctx.point_voxel_map
        offsets, entries = m.voxel_entries(ctx.voxel_rows)
        grad = _ext().interpolate_point_features_grad(
            grad_out.contiguous(), m.weights, offsets, entries,
            ctx.voxel_rows)
        return grad, None


# ------------------------------------------------------------- helpers --


def _validate_points(points: torch.Tensor) -> None:
    if points.ndim != 2 or points.shape[1] != 3:
        raise ValueError('points must have shape (N, 3).')
    if points.dtype != torch.float32:
        raise ValueError('points must be float32.')


def _batch_indices(value: torch.Tensor | None,
                   points: torch.Tensor) -> torch.Tensor:
    rows = int(points.shape[0])
    if value is None:
        return torch.zeros((rows,), dtype=torch.int32, device=points.device)
    if tuple(value.shape) != (rows,) or value.dtype != torch.int32:
        raise ValueError(
            'batch_indices must have shape (N,) and int32 dtype.')
    return value


def _active_rows(value: torch.Tensor | None,
                 like: torch.Tensor) -> torch.Tensor:
    if value is None:
        return torch.full((1,), like.shape[0], dtype=torch.int32,
                          device=like.device)
    if tuple(value.shape) != (1,) or value.dtype != torch.int32:
        raise ValueError('active_rows must have shape (1,) and int32 dtype.')
    return value


def _float_triple(value, name: str) -> tuple[float, float, float]:
    if isinstance(value, (int, float)):
        values = (float(value),) * 3
    else:
        raw = tuple(float(item) for item in value)
        if len(raw) != 3:
            raise ValueError(f'{name} must contain exactly 3 values.')
        values = raw
    if name == 'voxel_size' and any(item <= 0.0 for item in values):
        raise ValueError('voxel_size values must be positive.')
    return values


def _validate_reduction(value: str) -> VoxelReduction:
    if value in ('sum', 'mean'):
        return value
    raise ValueError("reduction must be 'sum' or 'mean'.")


def _validate_interpolation(value: str) -> PointVoxelInterpolation:
    if value in ('nearest', 'linear'):
        return value
    raise ValueError("interpolation must be 'nearest' or 'linear'.")
