"""Sparse tensor utilities (mlx_lattice/ops/tensor.py:15-64)."""

from __future__ import annotations

from collections.abc import Sequence

import torch

from mlx_lattice_amd.core import SparseTensor
from mlx_lattice_amd.core.types import triple

__all__ = ['sparse_collate']


def sparse_collate(coords: Sequence[torch.Tensor],
                   feats: Sequence[torch.Tensor], *,
                   stride: int | Sequence[int] = 1) -> SparseTensor:
    """Collate unbatched ``(N_i, 3)`` coordinates and ``(N_i, C)`` features
    into one tensor: a batch column is prepended and ``batch_counts`` is
    recorded."""
    if len(coords) != len(feats):
        raise ValueError('coords and feats batch sizes must match.')
    if not coords:
        raise ValueError('expected at least one sparse tensor batch.')
    coord_dtype = coords[0].dtype
    batched_coords, batched_feats = [], []
    for batch, (coord_rows, feat_rows) in enumerate(zip(coords, feats,
                                                        strict=True)):
        if coord_rows.ndim != 2 or coord_rows.shape[1] != 3:
            raise ValueError('collated coords must have shape (N, 3).')
        if coord_rows.dtype not in (torch.int32, torch.int64):
            raise ValueError('collated coords must be int32 or int64.')
        if coord_rows.dtype != coord_dtype:
            raise ValueError('collated coords must share a dtype.')
        if feat_rows.ndim != 2:
            raise ValueError('collated feats must have shape (N, C).')
        if coord_rows.shape[0] != feat_rows.shape[0]:
            raise ValueError(
                'collated coords and feats must have matching rows.')
        batch_col = torch.full((coord_rows.shape[0], 1), batch,
                               dtype=coord_rows.dtype,
                               device=coord_rows.device)
        batched_coords.append(torch.cat([batch_col, coord_rows], 1))
        batched_feats.append(feat_rows)
    return SparseTensor(torch.cat(batched_coords, 0),
                        torch.cat(batched_feats, 0),
                        stride=triple(stride, name='stride'),
                        batch_counts=tuple(int(c.shape[0]) for c in coords))
