"""Relation builders: the Python side of mlx_lattice/core/coords/builders.py
(:42-233, :393-444) over the native ``_ext`` module.

Each builder validates, calls the gfx950 relation kernels through ``_ext`` and
wraps the native 10-tuple (plus the implicit-GEMM view that the same map
query produced) into a ``KernelRelation``.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from mlx_lattice_amd.core.coords.validation import validate_coords
from mlx_lattice_amd.core.relations import (
    KernelRelation,
    KernelSpec,
    RelationImplicitGemmView,
)
from mlx_lattice_amd.core.relations.views import RelationKind
from mlx_lattice_amd.core.types import Triple, triple


def _ext():
    from mlx_lattice_amd._native import ext

    return ext


def kernel_offsets(kernel_size: int | Sequence[int],
                   dilation: int | Sequence[int] = 1) -> tuple[Triple, ...]:
    """Offsets of a dense 3D kernel footprint (builders.py:130-153,
    offsets.cpp:11-45): odd extents ``-r..r``, even extents ``0..k-1``,
    x outer / z inner, times dilation."""
    kernel = triple(kernel_size, name='kernel_size')
    rate = triple(dilation, name='dilation')
    _require_positive(kernel, 'kernel_size')
    _require_positive(rate, 'dilation')
    axes = []
    for size in kernel:
        if size % 2 == 1:
            radius = size // 2
            axes.append(range(-radius, radius + 1))
        else:
            axes.append(range(size))
    return tuple((int(x * rate[0]), int(y * rate[1]), int(z * rate[2]))
                 for x in axes[0] for y in axes[1] for z in axes[2])


def build_relation_implicit_gemm_view(
        relation: KernelRelation) -> RelationImplicitGemmView:
    """Dense output-to-input map for implicit-GEMM kernels
    (builders.py:42-79)."""
    contract = relation.contract
    if contract.kind not in ('forward', 'target', 'submanifold'):
        raise ValueError(
            'implicit GEMM view currently supports forward, target, and '
            'submanifold relations.')
    if (contract.source_coords is None or contract.source_active_rows is None
            or contract.out_coords is None):
        raise ValueError(
            'kernel relation is missing coordinate context for implicit GEMM.')
    output_active = (contract.target_active_rows
                     if contract.kind in ('target', 'submanifold')
                     else contract.out_count)
    if output_active is None:
        raise ValueError(
            'kernel relation is missing output activity for implicit GEMM.')
    offsets = torch.tensor(contract.kernel_offsets, dtype=torch.int32,
                           device=contract.source_coords.device).reshape(-1, 3)
    out_in_map, row_masks = _ext().build_relation_implicit_gemm_view(
        contract.source_coords, contract.source_active_rows,
        contract.out_coords, output_active, offsets, list(contract.stride),
        list(contract.padding))
    return RelationImplicitGemmView(out_in_map, row_masks=row_masks)


def build_kernel_relation(coords: torch.Tensor,
                          active_rows: torch.Tensor | None = None,
                          kernel_size: int | Sequence[int] = 3,
                          stride: int | Sequence[int] = 1,
                          padding: int | Sequence[int] = 0,
                          dilation: int | Sequence[int] = 1, *,
                          table: torch.Tensor | None = None) -> KernelRelation:
    """Forward sparse convolution relation (builders.py:156-191).  ``table``
    (optional): the ``block_table`` of an earlier relation over the same
    coordinates (built on the current stream), which the build then reuses
    instead of hashing the coordinates again."""
    validate_coords(coords)
    spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                      dilation=dilation)
    offsets = kernel_offsets(spec.size, spec.dilation)
    source_active = _active_rows(active_rows, coords)
    native = _ext().build_kernel_relation_with_view(
        coords, source_active, list(spec.size), list(spec.stride),
        list(spec.padding), list(spec.dilation), table=table)
    return _kernel_relation_from_native(
        native, offsets=offsets, in_capacity=int(coords.shape[0]),
        source_coords=coords, source_active_rows=source_active,
        stride=spec.stride, padding=spec.padding, kind='forward')


def build_submanifold_kernel_relation(
        coords: torch.Tensor, active_rows: torch.Tensor | None = None,
        kernel_size: int | Sequence[int] = 3,
        dilation: int | Sequence[int] = 1, *,
        keep_table: bool = False) -> KernelRelation:
    """Submanifold relation whose output support is ``coords``
    (builders.py:194-233).  ``keep_table``: keep the build's block table of
    ``coords`` (a buffer of its own, about 96-192 B per row) as
    ``block_table`` for a later ``build_kernel_relation(..., table=...)``
    over the same coordinates."""
    validate_coords(coords)
    spec = KernelSpec(size=kernel_size, stride=1, padding=0,
                      dilation=dilation)
    if not all(value % 2 == 1 for value in spec.size):
        raise ValueError(
            'submanifold relations require odd kernels, stride=1, '
            'padding=0, and positive dilation.')
    offsets = kernel_offsets(spec.size, spec.dilation)
    source_active = _active_rows(active_rows, coords)
    native = _ext().build_submanifold_kernel_relation_with_view(
        coords, source_active, list(spec.size), list(spec.dilation))
    return _kernel_relation_from_native(
        native, offsets=offsets, in_capacity=int(coords.shape[0]),
        out_coords=coords, source_coords=coords,
        source_active_rows=source_active, target_coords=coords,
        target_active_rows=source_active, stride=spec.stride,
        padding=spec.padding, kind='submanifold', keep_table=keep_table)


def build_target_kernel_relation(
        coords: torch.Tensor, target_coords: torch.Tensor, *,
        active_rows: torch.Tensor | None = None,
        target_active_rows: torch.Tensor | None = None,
        kernel_size: int | Sequence[int] = 3,
        stride: int | Sequence[int] = 1,
        padding: int | Sequence[int] = 0,
        dilation: int | Sequence[int] = 1) -> KernelRelation:
    """Relation from source coords to explicit target coords
    (builders.py:82-127)."""
    validate_coords(coords)
    validate_coords(target_coords)
    if coords.dtype != target_coords.dtype:
        raise ValueError('coordinate arrays must have matching dtype.')
    spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                      dilation=dilation)
    offsets = kernel_offsets(spec.size, spec.dilation)
    source_active = _active_rows(active_rows, coords)
    target_active = _active_rows(target_active_rows, target_coords)
    native = _ext().build_target_kernel_relation_with_view(
        coords, source_active, target_coords, target_active,
        list(spec.size), list(spec.stride), list(spec.padding),
        list(spec.dilation))
    return _kernel_relation_from_native(
        native, offsets=offsets, in_capacity=int(coords.shape[0]),
        source_coords=coords, source_active_rows=source_active,
        target_coords=target_coords, target_active_rows=target_active,
        stride=spec.stride, padding=spec.padding, kind='target')


def build_generative_relation(coords: torch.Tensor,
                              active_rows: torch.Tensor | None = None,
                              kernel_size: int | Sequence[int] = 2,
                              stride: int | Sequence[int] = 2
                              ) -> KernelRelation:
    """Generative transpose-convolution relation (builders.py:236-265):
    output row ``in * K + k`` is ``coord * stride + offset[k]``, one edge
    per output row; offsets without dilation."""
    validate_coords(coords)
    kernel = triple(kernel_size, name='kernel_size')
    step = triple(stride, name='stride')
    _require_positive(kernel, 'kernel_size')
    _require_positive(step, 'stride')
    offsets = kernel_offsets(kernel)
    source_active = _active_rows(active_rows, coords)
    native = _ext().build_generative_relation_lazy(
        coords, source_active, list(kernel), list(step))
    return _kernel_relation_from_native(
        native[:10], offsets=offsets, in_capacity=int(coords.shape[0]),
        source_coords=coords, source_active_rows=source_active, stride=step,
        kind='generative', repeated_edges=False, direct_expansion=True)


def build_transposed_kernel_relation(coords: torch.Tensor,
                                     active_rows: torch.Tensor | None = None,
                                     kernel_size: int | Sequence[int] = 2,
                                     stride: int | Sequence[int] = 2,
                                     padding: int | Sequence[int] = 0,
                                     dilation: int | Sequence[int] = 1
                                     ) -> KernelRelation:
    """Sparse transpose-convolution relation (builders.py:268-306): the
    candidates ``coord * stride + offset - padding`` of every input row,
    one output row each when the stride exceeds the offsets' extent,
    otherwise deduplicated in first-seen order."""
    validate_coords(coords)
    kernel = triple(kernel_size, name='kernel_size')
    step = triple(stride, name='stride')
    pad = triple(padding, name='padding')
    rate = triple(dilation, name='dilation')
    _require_positive(kernel, 'kernel_size')
    _require_positive(step, 'stride')
    if any(value < 0 for value in pad):
        raise ValueError('padding values must be non-negative.')
    _require_positive(rate, 'dilation')
    offsets = kernel_offsets(kernel, rate)
    source_active = _active_rows(active_rows, coords)
    native = _ext().build_transposed_kernel_relation_lazy(
        coords, source_active, list(kernel), list(step), list(pad),
        list(rate))
    status = native[10]
    # can_use_direct_transposed_relation (relations.cpp:107-127)
    direct = all(step[a] > max(o[a] for o in offsets) - min(o[a] for o in offsets)
                 for a in range(3))
    return _kernel_relation_from_native(
        native[:10], offsets=offsets, in_capacity=int(coords.shape[0]),
        source_coords=coords, source_active_rows=source_active, stride=step,
        padding=pad, kind='transposed',
        repeated_edges=False if direct else status,
        direct_expansion=direct)


def _kernel_relation_from_native(
        native, *, offsets: tuple[Triple, ...], in_capacity: int,
        out_coords: torch.Tensor | None = None,
        source_coords: torch.Tensor, source_active_rows: torch.Tensor,
        target_coords: torch.Tensor | None = None,
        target_active_rows: torch.Tensor | None = None,
        stride: Triple = (1, 1, 1), padding: Triple = (0, 0, 0),
        kind: RelationKind = 'forward',
        repeated_edges: bool | torch.Tensor | None = None,
        direct_expansion: bool = False,
        keep_table: bool = False) -> KernelRelation:
    (in_rows, out_rows, kernel_ids, row_offsets, native_out_coords, counts,
     in_row_offsets, in_edge_ids, kernel_row_offsets, kernel_edge_ids,
     *view) = native
    relation_out_coords = (native_out_coords if out_coords is None
                           else out_coords)
    implicit = (RelationImplicitGemmView(view[0], row_masks=view[1])
                if len(view) >= 2 else None)
    # The status word of a submanifold relation flags repeated coordinates;
    # its workspace holds the block table of its coordinates.
    repeated_coords = (view[2] if len(view) >= 3 and kind == 'submanifold'
                       else None)
    block_table = view[3] if len(view) >= 4 and keep_table else None
    grouped_views = None
    if in_row_offsets is None:
        n_kernels = len(offsets)

        def grouped_views():
            return _ext().build_relation_grouped_views(
                in_rows, kernel_ids, counts, in_capacity, n_kernels)
    return KernelRelation(
        in_rows, out_rows, kernel_ids, row_offsets=row_offsets,
        counts=counts, in_row_offsets=in_row_offsets,
        in_edge_ids=in_edge_ids, kernel_row_offsets=kernel_row_offsets,
        kernel_edge_ids=kernel_edge_ids, kernel_offsets=offsets,
        out_coords=relation_out_coords, n_in_capacity=in_capacity,
        n_out_capacity=int(relation_out_coords.shape[0]),
        n_kernels=len(offsets), source_coords=source_coords,
        source_active_rows=source_active_rows, target_coords=target_coords,
        target_active_rows=target_active_rows, stride=stride,
        padding=padding, kind=kind, implicit_gemm=implicit,
        grouped_views=grouped_views, repeated_edges=repeated_edges,
        direct_expansion=direct_expansion, repeated_coords=repeated_coords,
        block_table=block_table)


def _require_positive(values: Triple, name: str) -> None:
    if any(value <= 0 for value in values):
        raise ValueError(f'{name} values must be positive.')


def _active_rows(value: torch.Tensor | None,
                 coords: torch.Tensor) -> torch.Tensor:
    if value is not None:
        if tuple(value.shape) != (1,) or value.dtype != torch.int32:
            raise ValueError(
                'active_rows must have shape (1,) and int32 dtype.')
        return value
    return torch.full((1,), coords.shape[0], dtype=torch.int32,
                      device=coords.device)
