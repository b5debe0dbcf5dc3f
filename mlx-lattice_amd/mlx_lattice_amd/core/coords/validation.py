from __future__ import annotations

import torch


def validate_coords(coords: torch.Tensor, *, name: str = 'coords') -> None:
    """Validate a batched sparse coordinate array with shape ``(N, 4)``
    (mlx_lattice/core/coords/validation.py:6-11)."""
    if coords.ndim != 2 or coords.shape[1] != 4:
        raise ValueError(f'{name} must have shape (N, 4).')
    if coords.dtype not in (torch.int32, torch.int64):
        raise ValueError(f'{name} must be int32 or int64.')


def validate_coord_pair(lhs: torch.Tensor, rhs: torch.Tensor, *,
                        lhs_name: str = 'lhs', rhs_name: str = 'rhs') -> None:
    validate_coords(lhs, name=lhs_name)
    validate_coords(rhs, name=rhs_name)
    if lhs.dtype != rhs.dtype:
        raise ValueError('coordinate arrays must have matching dtype.')
