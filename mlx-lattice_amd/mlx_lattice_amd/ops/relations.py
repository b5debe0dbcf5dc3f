"""Functional relation builders over a sparse tensor's coordinate manager
(mlx_lattice/ops/relations.py:39-146): each wraps the manager method of the
same relation kind, which builds the relation once per (key, geometry) and
caches it."""

from __future__ import annotations

from collections.abc import Sequence

from mlx_lattice_amd.core.coords.builders import (
    build_generative_relation,
    build_kernel_relation,
    build_submanifold_kernel_relation,
    build_target_kernel_relation,
    build_transposed_kernel_relation,
    kernel_offsets,
)
from mlx_lattice_amd.core.relations import KernelRelation
from mlx_lattice_amd.core.tensor import SparseTensor

__all__ = [
    'build_generative_relation',
    'build_kernel_relation',
    'build_submanifold_kernel_relation',
    'build_target_kernel_relation',
    'build_transposed_kernel_relation',
    'generative_kernel_relation',
    'kernel_offsets',
    'kernel_relation',
    'submanifold_kernel_relation',
    'target_kernel_relation',
    'transposed_kernel_relation',
]


def kernel_relation(x: SparseTensor, *,
                    kernel_size: int | Sequence[int] = 3,
                    stride: int | Sequence[int] = 1,
                    padding: int | Sequence[int] = 0,
                    dilation: int | Sequence[int] = 1) -> KernelRelation:
    """Forward kernel relation of ``x`` (ops/relations.py:39-60)."""
    return x.coord_manager.kernel_relation(
        x.coord_key, kernel_size=kernel_size, stride=stride, padding=padding,
        dilation=dilation)


def generative_kernel_relation(x: SparseTensor, *,
                               kernel_size: int | Sequence[int] = 2,
                               stride: int | Sequence[int] = 2
                               ) -> KernelRelation:
    """Generative transpose-convolution relation of ``x``
    (ops/relations.py:63-74)."""
    return x.coord_manager.generative_relation(
        x.coord_key, kernel_size=kernel_size, stride=stride)


def submanifold_kernel_relation(x: SparseTensor, *,
                                kernel_size: int | Sequence[int] = 3,
                                dilation: int | Sequence[int] = 1
                                ) -> KernelRelation:
    """Submanifold relation of ``x`` (ops/relations.py:77-92)."""
    return x.coord_manager.submanifold_kernel_relation(
        x.coord_key, kernel_size=kernel_size, dilation=dilation)


def transposed_kernel_relation(x: SparseTensor, *,
                               kernel_size: int | Sequence[int] = 2,
                               stride: int | Sequence[int] = 2,
                               padding: int | Sequence[int] = 0,
                               dilation: int | Sequence[int] = 1
                               ) -> KernelRelation:
    """Transpose-convolution relation of ``x`` (ops/relations.py:95-110)."""
    return x.coord_manager.transposed_kernel_relation(
        x.coord_key, kernel_size=kernel_size, stride=stride, padding=padding,
        dilation=dilation)


def target_kernel_relation(x: SparseTensor, target: SparseTensor, *,
                           kernel_size: int | Sequence[int] = 3,
                           stride: int | Sequence[int] = 1,
                           padding: int | Sequence[int] = 0,
                           dilation: int | Sequence[int] = 1
                           ) -> KernelRelation:
    """Relation from ``x`` to an explicit target tensor
    (ops/relations.py:113-146); a target from another manager is inserted
    into ``x``'s manager first."""
    if x.coord_manager is not target.coord_manager:
        target_key = x.coord_manager.insert_coords(
            target.coords, target.stride, target.active_rows)
    else:
        target_key = target.coord_key
    return x.coord_manager.target_kernel_relation(
        x.coord_key, target_key, kernel_size=kernel_size, stride=stride,
        padding=padding, dilation=dilation)
