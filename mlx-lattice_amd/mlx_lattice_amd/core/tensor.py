"""``SparseTensor``: batched integer coordinates + feature matrix with
coordinate identity metadata (mlx_lattice/core/tensor.py:16-314), over torch
tensors."""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from mlx_lattice_amd.core.coords import (
    CoordinateManager,
    CoordinateMapKey,
    validate_coords,
)
from mlx_lattice_amd.core.types import Triple, triple


@dataclass(frozen=True, slots=True, init=False)
class SparseTensor:
    """Sparse feature tensor indexed by ``(batch, x, y, z)`` coordinates.

    Coordinates have shape ``(N, 4)`` (int32 on the GPU path), features
    ``(N, C)`` share row order with them.  ``coord_key`` / ``coord_manager``
    carry coordinate identity so relations are cached and reused;
    ``active_rows`` is a device int32 ``(1,)`` count of valid rows inside the
    static capacity.
    """

    coords: torch.Tensor
    feats: torch.Tensor
    stride: Triple
    coord_key: CoordinateMapKey
    coord_manager: CoordinateManager
    batch_counts: tuple[int, ...] | None
    active_rows: torch.Tensor

    def __init__(self, coords: torch.Tensor, feats: torch.Tensor,
                 stride: int | Sequence[int] = 1, *,
                 coord_key: CoordinateMapKey | None = None,
                 coord_manager: CoordinateManager | None = None,
                 batch_counts: Sequence[int] | None = None,
                 active_rows: torch.Tensor | None = None) -> None:
        normalized_stride = triple(stride, name='stride')
        manager, key, owned, active = _resolve_coordinate_identity(
            coords, normalized_stride, active_rows, coord_key=coord_key,
            coord_manager=coord_manager)
        if feats.ndim != 2:
            raise ValueError('feats must have shape (N, C).')
        if owned.shape[0] != feats.shape[0]:
            raise ValueError('coords and feats must have the same row count.')
        object.__setattr__(self, 'coords', owned)
        object.__setattr__(self, 'feats', feats)
        object.__setattr__(self, 'stride', normalized_stride)
        object.__setattr__(self, 'coord_key', key)
        object.__setattr__(self, 'coord_manager', manager)
        object.__setattr__(self, 'batch_counts',
                           _batch_counts(batch_counts, rows=owned.shape[0]))
        object.__setattr__(self, 'active_rows', active)

    @property
    def capacity(self) -> int:
        return int(self.coords.shape[0])

    @property
    def active_count(self) -> torch.Tensor:
        return self.active_rows

    @property
    def channels(self) -> int:
        return int(self.feats.shape[1])

    @property
    def shape(self) -> tuple[int, int]:
        return (self.capacity, self.channels)

    @property
    def dtype(self) -> torch.dtype:
        return self.feats.dtype

    @property
    def device(self) -> torch.device:
        return self.feats.device

    @property
    def batch_indices(self) -> torch.Tensor:
        return self.coords[:, 0]

    def astype(self, dtype: torch.dtype) -> SparseTensor:
        """Features converted to ``dtype``; coordinate identity kept."""
        return self.replace(feats=self.feats.to(dtype))

    def replace(self, *, coords: torch.Tensor | None = None,
                feats: torch.Tensor | None = None,
                stride: int | Sequence[int] | None = None) -> SparseTensor:
        """Replace fields; replacing only ``feats`` keeps the coordinate
        identity (tensor.py:172-198)."""
        next_coords = self.coords if coords is None else coords
        next_stride = (self.stride if stride is None
                       else triple(stride, name='stride'))
        reuse_key = next_coords is self.coords and next_stride == self.stride
        return SparseTensor(
            next_coords, self.feats if feats is None else feats, next_stride,
            coord_key=self.coord_key if reuse_key else None,
            coord_manager=self.coord_manager,
            batch_counts=self.batch_counts if reuse_key else None,
            active_rows=self.active_rows if reuse_key else None)

    def same_coords(self, other: SparseTensor) -> bool:
        return (self.coord_manager is other.coord_manager
                and self.coord_key == other.coord_key)

    def reuse_coords_from(self, other: SparseTensor) -> SparseTensor:
        if not self.same_coords(other):
            raise ValueError('sparse tensor coordinates must match.')
        return SparseTensor(other.coords, self.feats, other.stride,
                            coord_key=other.coord_key,
                            coord_manager=other.coord_manager,
                            batch_counts=other.batch_counts,
                            active_rows=other.active_rows)


def _resolve_coordinate_identity(coords, stride, active_rows, *, coord_key,
                                 coord_manager):
    validate_coords(coords)
    if coord_key is None:
        manager = CoordinateManager() if coord_manager is None else coord_manager
        key = manager.insert_coords(coords, stride, active_rows)
        return manager, key, coords, manager.active_rows(key)
    if coord_manager is None:
        raise ValueError('coord_manager is required when coord_key is set.')
    if not coord_manager.owns(coord_key):
        raise ValueError('coord_key does not belong to coord_manager.')
    if coord_key.stride != stride:
        raise ValueError('stride must match coord_key stride.')
    owned = coord_manager.coords(coord_key)
    if coords is not owned:
        raise ValueError(
            'coords must be the manager-owned array for coord_key.')
    active = (coord_manager.active_rows(coord_key) if active_rows is None
              else _active_rows(active_rows))
    return coord_manager, coord_key, owned, active


def _batch_counts(values, *, rows: int):
    if values is None:
        return None
    counts = tuple(int(v) for v in values)
    if any(v < 0 for v in counts):
        raise ValueError('batch_counts must be non-negative.')
    if sum(counts) != rows:
        raise ValueError('batch_counts must cover all sparse rows.')
    return counts


def _active_rows(value: torch.Tensor) -> torch.Tensor:
    if tuple(value.shape) != (1,) or value.dtype != torch.int32:
        raise ValueError('active_rows must have shape (1,) and int32 dtype.')
    return value
