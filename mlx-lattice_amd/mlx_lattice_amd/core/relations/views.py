"""Kernel relation contract and its execution views over torch tensors.

Mirrors mlx_lattice/core/relations/views.py (RelationEdges :19-45,
RelationCSRView :48-62, RelationImplicitGemmView :68-101,
RelationSortedImplicitGemmView :104-146, SparseRelationContract :149-236,
KernelRelation :259-525).  Every array is an int32 torch tensor on the
relation's device; counts stay on the device.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass, field
from typing import Literal

import torch

from mlx_lattice_amd.core.types import Triple

RelationKind = Literal['forward', 'target', 'submanifold', 'transposed',
                       'generative']

_INDEX_DTYPES = (torch.int32, torch.int64)


@dataclass(frozen=True, slots=True)
class RelationEdges:
    """Edge arrays ``(in_row, out_row, kernel_id)`` at the same index."""

    in_rows: torch.Tensor
    out_rows: torch.Tensor
    kernel_ids: torch.Tensor

    def __post_init__(self) -> None:
        _validate_row_array(self.in_rows, name='in_rows')
        _validate_row_array(self.out_rows, name='out_rows')
        _validate_row_array(self.kernel_ids, name='kernel_ids')
        _require_same_rows(self.in_rows, self.out_rows, self.kernel_ids,
                           names=('in_rows', 'out_rows', 'kernel_ids'))

    @property
    def capacity(self) -> int:
        return int(self.in_rows.shape[0])


@dataclass(frozen=True, slots=True)
class RelationCSRView:
    """CSR view: ``row_offsets`` ``(rows + 1,)`` int32 and optional
    ``edge_ids`` remapping CSR order to the canonical edge arrays."""

    row_offsets: torch.Tensor
    edge_ids: torch.Tensor | None = None

    def __post_init__(self) -> None:
        _validate_row_offsets(self.row_offsets)
        if self.edge_ids is not None:
            _validate_row_array(self.edge_ids, name='edge_ids')


RelationView = RelationCSRView


@dataclass(frozen=True, slots=True)
class RelationImplicitGemmView:
    """Dense ``out_in_map[o, k]`` (input row or -1) plus ``row_masks``
    (bit k%32 of word k/32 set when offset k contributes)."""

    out_in_map: torch.Tensor
    row_masks: torch.Tensor

    def __post_init__(self) -> None:
        if self.out_in_map.ndim != 2:
            raise ValueError('out_in_map must have shape (Nout, K).')
        if self.out_in_map.dtype not in _INDEX_DTYPES:
            raise ValueError('out_in_map must be int32 or int64.')
        if self.row_masks.ndim != 2:
            raise ValueError('row_masks must have shape (Nout, M).')
        if self.row_masks.dtype not in _INDEX_DTYPES:
            raise ValueError('row_masks must be int32 or int64.')
        if int(self.row_masks.shape[0]) != int(self.out_in_map.shape[0]):
            raise ValueError('row_masks must have one row per out_in_map row.')
        expected = (int(self.out_in_map.shape[1]) + 31) // 32
        if int(self.row_masks.shape[1]) != expected:
            raise ValueError(
                'row_masks must have ceil(K / 32) words per output row.')


@dataclass(frozen=True, slots=True)
class RelationSortedImplicitGemmView:
    """Mask-sorted implicit-GEMM view consumed by the matrix-core route."""

    sorted_out_in_map: torch.Tensor
    sorted_kv_out_in_map: torch.Tensor
    reorder_rows: torch.Tensor
    tile_masks: torch.Tensor
    _tile_order: torch.Tensor | None = field(default=None, compare=False,
                                             repr=False)

    def __post_init__(self) -> None:
        if self.sorted_out_in_map.ndim != 2:
            raise ValueError('sorted_out_in_map must have shape (Nout, K).')
        if self.sorted_kv_out_in_map.ndim != 2:
            raise ValueError('sorted_kv_out_in_map must have shape (K, Nout).')
        if (int(self.sorted_kv_out_in_map.shape[0])
                != int(self.sorted_out_in_map.shape[1])
                or int(self.sorted_kv_out_in_map.shape[1])
                != int(self.sorted_out_in_map.shape[0])):
            raise ValueError('sorted_kv_out_in_map must be the K-major view '
                             'of sorted_out_in_map.')
        _validate_row_array(self.reorder_rows, name='reorder_rows')
        _validate_row_array(self.tile_masks, name='tile_masks')
        if int(self.reorder_rows.shape[0]) != int(
                self.sorted_out_in_map.shape[0]):
            raise ValueError(
                'reorder_rows must have one row per sorted_out_in_map row.')

    def tile_order(self) -> torch.Tensor:
        """Longest-first order of the view's 128-row tiles for the
        matrix-core conv, computed on first use and kept with the view so
        repeated convs over it skip their per-call schedule."""
        if self._tile_order is None:
            from mlx_lattice_amd._native import ext

            object.__setattr__(self, '_tile_order', ext.conv_tile_order(
                self.tile_masks, int(self.reorder_rows.shape[0])))
        return self._tile_order


class _StatusWord:
    """A device status word copied to pinned host memory when the relation
    is built: the copy is queued on the current stream and never waited
    for there; read() waits only for the copy's event (usually long
    complete by the time a backward pass asks)."""

    def __init__(self, word: torch.Tensor) -> None:
        if word.is_cuda:
            self._host = torch.empty(1, dtype=torch.int32, pin_memory=True)
            self._host.copy_(word, non_blocking=True)
            self._event = torch.cuda.Event()
            self._event.record()
        else:
            self._host = word.clone()
            self._event = None

    def read(self) -> int:
        """The word's value.  Raises RuntimeError when the builder's
        coordinate table overflowed (lattice_relation_flags bit 16): the
        table is sized above its key count, so this marks a sizing error
        and the relation's contents are void."""
        if self._event is not None:
            self._event.synchronize()
        value = int(self._host[0])
        if value & 16:
            raise RuntimeError('relation build: the coordinate table '
                               'overflowed (status word bit 16); the '
                               'relation is invalid.')
        return value


@dataclass(frozen=True, slots=True)
class SparseRelationContract:
    """Counts, capacities, coordinate context and geometry of a relation."""

    counts: torch.Tensor
    kernel_offsets: tuple[Triple, ...]
    out_coords: torch.Tensor | None = None
    n_in_capacity: int | None = None
    n_out_capacity: int | None = None
    n_kernels: int | None = None
    source_coords: torch.Tensor | None = None
    source_active_rows: torch.Tensor | None = None
    target_coords: torch.Tensor | None = None
    target_active_rows: torch.Tensor | None = None
    stride: Triple = (1, 1, 1)
    padding: Triple = (0, 0, 0)
    kind: RelationKind = 'forward'
    # One view object per count: a strided output tensor is keyed in its
    # coordinate manager by the identity of its active-row array, so handing
    # out the same view lets repeated calls reuse the output's relations.
    _edge_count: torch.Tensor = field(init=False, repr=False, compare=False)
    _out_count: torch.Tensor = field(init=False, repr=False, compare=False)

    def __post_init__(self) -> None:
        _validate_counts(self.counts)
        object.__setattr__(self, '_edge_count', self.counts[:1])
        object.__setattr__(self, '_out_count', self.counts[1:2])
        for name in ('out_coords', 'source_coords', 'target_coords'):
            value = getattr(self, name)
            if value is not None:
                _validate_coords(value, name=name)
        for name in ('source_active_rows', 'target_active_rows'):
            value = getattr(self, name)
            if value is not None:
                _validate_active_rows(value, name=name)
        if self.kind not in ('forward', 'target', 'submanifold',
                             'transposed', 'generative'):
            raise ValueError(
                "relation kind must be 'forward', 'target', "
                "'submanifold', 'transposed', or 'generative'.")
        offsets = tuple((int(x), int(y), int(z))
                        for x, y, z in self.kernel_offsets)
        object.__setattr__(self, 'kernel_offsets', offsets)
        object.__setattr__(self, 'stride', tuple(int(v) for v in self.stride))
        object.__setattr__(self, 'padding',
                           tuple(int(v) for v in self.padding))
        n_in = _optional_count(self.n_in_capacity, 'n_in_capacity')
        n_out = _optional_count(self.n_out_capacity, 'n_out_capacity')
        n_kernels = _optional_count(self.n_kernels, 'n_kernels')
        if offsets:
            if n_kernels is not None and n_kernels != len(offsets):
                raise ValueError('n_kernels must match kernel_offsets.')
            n_kernels = len(offsets)
        if self.out_coords is not None:
            out_capacity = int(self.out_coords.shape[0])
            if n_out is not None and n_out != out_capacity:
                raise ValueError(
                    'n_out_capacity must match out_coords capacity.')
            n_out = out_capacity
        object.__setattr__(self, 'n_in_capacity', n_in)
        object.__setattr__(self, 'n_out_capacity', n_out)
        object.__setattr__(self, 'n_kernels', n_kernels)

    @property
    def edge_count(self) -> torch.Tensor:
        return self._edge_count

    @property
    def out_count(self) -> torch.Tensor:
        return self._out_count


@dataclass(frozen=True, slots=True, init=False)
class KernelRelation:
    """Sparse kernel relation with edge, CSR and implicit-GEMM views."""

    contract: SparseRelationContract
    edges: RelationEdges
    output_csr: RelationCSRView
    _input_csr: RelationCSRView | None
    _kernel_csr: RelationCSRView | None
    _grouped_views: Callable[[], tuple] | None
    implicit_gemm: RelationImplicitGemmView | None = None
    sorted_implicit_gemm: RelationSortedImplicitGemmView | None = None
    transposed_sorted_implicit_gemm: RelationSortedImplicitGemmView | None = None
    # Transposed relations only: whether two edges share (out_row, kernel_id)
    # (a repeated input coordinate).  The builder hands over its device
    # status word, copied to pinned memory at build time (a _StatusWord) and
    # read on the first question (dense_map_exact), so building the relation
    # never waits for the device.  None: unknown.
    repeated_edges: bool | _StatusWord | None = None
    # Generative, and transposed relations whose stride exceeds the offsets'
    # extent: output row in * K + k holds the single edge (in, k).
    direct_expansion: bool = False
    # Submanifold relations: whether an active row repeats an earlier row's
    # coordinate (each copy is an output row with the same neighbours, so
    # an input row can have several output rows at one offset).  Held as a
    # _StatusWord copied to pinned memory at build time and read on the
    # first question (transposed_map_exact).  None: no repeats possible.
    repeated_coords: bool | _StatusWord | None = None
    # Submanifold relations built with their workspace: it starts with the
    # block table of the coordinates (the coordinate manager hands it to
    # the next forward relation over the same key).
    block_table: torch.Tensor | None = None

    def __init__(
        self,
        in_rows: torch.Tensor,
        out_rows: torch.Tensor,
        kernel_ids: torch.Tensor,
        *,
        row_offsets: torch.Tensor | None = None,
        counts: torch.Tensor | None = None,
        in_row_offsets: torch.Tensor | None = None,
        in_edge_ids: torch.Tensor | None = None,
        kernel_row_offsets: torch.Tensor | None = None,
        kernel_edge_ids: torch.Tensor | None = None,
        kernel_offsets: tuple[Triple, ...] = (),
        out_coords: torch.Tensor | None = None,
        n_in_capacity: int | None = None,
        n_out_capacity: int | None = None,
        n_kernels: int | None = None,
        source_coords: torch.Tensor | None = None,
        source_active_rows: torch.Tensor | None = None,
        target_coords: torch.Tensor | None = None,
        target_active_rows: torch.Tensor | None = None,
        stride: Triple = (1, 1, 1),
        padding: Triple = (0, 0, 0),
        kind: RelationKind = 'forward',
        implicit_gemm: RelationImplicitGemmView | None = None,
        sorted_implicit_gemm: RelationSortedImplicitGemmView | None = None,
        grouped_views: Callable[[], tuple] | None = None,
        repeated_edges: bool | torch.Tensor | None = None,
        direct_expansion: bool = False,
        repeated_coords: torch.Tensor | None = None,
        block_table: torch.Tensor | None = None,
    ) -> None:
        """``grouped_views``, when given and the input/kernel CSR arrays are
        not, is called on first access of ``input_csr`` / ``kernel_csr`` and
        returns ``(in_row_offsets, in_edge_ids, kernel_row_offsets,
        kernel_edge_ids)``; the forward convolution never reads those
        views, so they are only built for consumers that do."""
        device = in_rows.device
        if counts is None:
            counts = torch.tensor(
                [in_rows.shape[0],
                 0 if out_coords is None else out_coords.shape[0]],
                dtype=torch.int32, device=device)
        _validate_counts(counts)
        contract = SparseRelationContract(
            counts=counts, kernel_offsets=kernel_offsets,
            out_coords=out_coords, n_in_capacity=n_in_capacity,
            n_out_capacity=n_out_capacity, n_kernels=n_kernels,
            source_coords=source_coords,
            source_active_rows=source_active_rows,
            target_coords=target_coords,
            target_active_rows=target_active_rows, stride=stride,
            padding=padding, kind=kind)
        if row_offsets is None:
            cap = int(contract.n_out_capacity or 0)
            row_offsets = torch.zeros(cap + 1, dtype=torch.int32,
                                      device=device)
        _validate_row_offsets(row_offsets)
        edges = RelationEdges(in_rows, out_rows, kernel_ids)
        lazy_views = grouped_views is not None and in_row_offsets is None
        if lazy_views:
            pass
        elif in_row_offsets is None:
            cap = int(contract.n_in_capacity or 0)
            in_row_offsets = torch.zeros(cap + 1, dtype=torch.int32,
                                         device=device)
        if not lazy_views:
            if in_edge_ids is None:
                in_edge_ids = torch.zeros(edges.capacity, dtype=torch.int32,
                                          device=device)
            if kernel_row_offsets is None:
                cap = int(contract.n_kernels or 0)
                kernel_row_offsets = torch.zeros(cap + 1, dtype=torch.int32,
                                                 device=device)
            if kernel_edge_ids is None:
                kernel_edge_ids = torch.zeros(edges.capacity,
                                              dtype=torch.int32, device=device)
        if (contract.n_out_capacity is not None
                and int(row_offsets.shape[0])
                != int(contract.n_out_capacity) + 1):
            raise ValueError(
                'row_offsets must have length n_out_capacity + 1.')
        object.__setattr__(self, 'contract', contract)
        object.__setattr__(self, 'edges', edges)
        object.__setattr__(self, 'output_csr', RelationCSRView(row_offsets))
        object.__setattr__(
            self, '_input_csr', None if lazy_views
            else RelationCSRView(in_row_offsets, in_edge_ids))
        object.__setattr__(
            self, '_kernel_csr', None if lazy_views
            else RelationCSRView(kernel_row_offsets, kernel_edge_ids))
        object.__setattr__(self, '_grouped_views',
                           grouped_views if lazy_views else None)
        object.__setattr__(self, 'implicit_gemm', implicit_gemm)
        object.__setattr__(self, 'sorted_implicit_gemm', sorted_implicit_gemm)
        object.__setattr__(self, 'transposed_sorted_implicit_gemm', None)
        object.__setattr__(
            self, 'repeated_edges',
            _StatusWord(repeated_edges)
            if isinstance(repeated_edges, torch.Tensor) else repeated_edges)
        object.__setattr__(
            self, 'repeated_coords',
            _StatusWord(repeated_coords) if repeated_coords is not None
            else None)
        object.__setattr__(self, 'block_table', block_table)
        object.__setattr__(self, 'direct_expansion', bool(direct_expansion))

    @property
    def input_csr(self) -> RelationCSRView:
        """Edges grouped by input row (stable in edge order)."""
        if self._input_csr is None:
            self._materialize_grouped_views()
        return self._input_csr

    @property
    def kernel_csr(self) -> RelationCSRView:
        """Edges grouped by kernel offset (stable in edge order)."""
        if self._kernel_csr is None:
            self._materialize_grouped_views()
        return self._kernel_csr

    def _materialize_grouped_views(self) -> None:
        in_offsets, in_ids, k_offsets, k_ids = self._grouped_views()
        object.__setattr__(self, '_input_csr',
                           RelationCSRView(in_offsets, in_ids))
        object.__setattr__(self, '_kernel_csr',
                           RelationCSRView(k_offsets, k_ids))

    @property
    def edge_capacity(self) -> int:
        return self.edges.capacity

    @property
    def counts(self) -> torch.Tensor:
        """Native counts array ``[edge_count, out_count]`` (device)."""
        return self.contract.counts

    @property
    def edge_count(self) -> torch.Tensor:
        return self.contract.edge_count

    @property
    def out_count(self) -> torch.Tensor:
        return self.contract.out_count

    @property
    def kernel_offsets(self) -> tuple[Triple, ...]:
        return self.contract.kernel_offsets

    @property
    def out_coords(self) -> torch.Tensor | None:
        return self.contract.out_coords

    @property
    def n_in_capacity(self) -> int | None:
        return self.contract.n_in_capacity

    @property
    def n_out_capacity(self) -> int | None:
        return self.contract.n_out_capacity

    @property
    def n_kernels(self) -> int | None:
        return self.contract.n_kernels

    @property
    def row_offsets(self) -> torch.Tensor:
        return self.output_csr.row_offsets

    @property
    def in_row_offsets(self) -> torch.Tensor:
        return self.input_csr.row_offsets

    @property
    def in_edge_ids(self) -> torch.Tensor:
        if self.input_csr.edge_ids is None:
            raise ValueError('input CSR view is missing edge ids.')
        return self.input_csr.edge_ids

    @property
    def kernel_row_offsets(self) -> torch.Tensor:
        return self.kernel_csr.row_offsets

    @property
    def kernel_edge_ids(self) -> torch.Tensor:
        if self.kernel_csr.edge_ids is None:
            raise ValueError('kernel CSR view is missing edge ids.')
        return self.kernel_csr.edge_ids

    @property
    def out_view(self) -> RelationCSRView:
        return self.output_csr

    @property
    def in_view(self) -> RelationCSRView:
        return self.input_csr

    @property
    def kernel_view(self) -> RelationCSRView:
        return self.kernel_csr

    def require_implicit_gemm(self) -> RelationImplicitGemmView:
        """Return or lazily build the implicit-GEMM view (views.py:452-465)."""
        if self.implicit_gemm is not None:
            return self.implicit_gemm
        if self.contract.kind in ('transposed', 'generative'):
            view = self._expanded_implicit_gemm()
            object.__setattr__(self, 'implicit_gemm', view)
            return view
        from mlx_lattice_amd.core.coords.builders import (
            build_relation_implicit_gemm_view,
        )

        view = build_relation_implicit_gemm_view(self)
        object.__setattr__(self, 'implicit_gemm', view)
        return view

    @property
    def dense_map_exact(self) -> bool:
        """Whether the dense (out_row, offset) -> in_row map holds every edge:
        at most one edge per (out_row, kernel_id).  Forward, submanifold and
        generative relations hold it by construction (a target relation
        too: each (target row, offset) has one candidate input, its first
        row); a transposed relation does unless an input coordinate repeats."""
        if self.contract.kind != 'transposed':
            return True
        if isinstance(self.repeated_edges, _StatusWord):
            # lattice_relation_flags: bit 2 = repeated (out_row, kernel_id)
            flags = self.repeated_edges.read()
            object.__setattr__(self, 'repeated_edges', bool(flags & 2))
        if self.repeated_edges is None:
            return False
        return not self.repeated_edges

    @property
    def transposed_map_exact(self) -> bool:
        """Whether the dense transposed (in_row, offset) -> out_row map holds
        every edge: at most one edge per (in_row, kernel_id).  Forward,
        generative and transposed relations hold it by construction (their
        output coordinates are distinct, or each output row has one edge); a
        submanifold relation does unless a coordinate repeats.  The first
        question reads the build's status word from pinned memory (copied
        when the relation was built), so it waits for that copy only."""
        if self.contract.kind == 'target':
            return False
        if isinstance(self.repeated_coords, _StatusWord):
            # lattice_relation_flags: bit 8 = repeated coordinate
            flags = self.repeated_coords.read()
            object.__setattr__(self, 'repeated_coords', bool(flags & 8))
        return not self.repeated_coords

    def _expanded_implicit_gemm(self) -> RelationImplicitGemmView:
        """Dense map of a generative or transposed relation, scattered from
        its edges: out_in_map[out][k] = in (the expanded relations carry no
        source table to query)."""
        if not self.dense_map_exact:
            raise ValueError('the dense implicit-GEMM map cannot hold a '
                             'relation with repeated (out_row, kernel_id) '
                             'edges.')
        from mlx_lattice_amd._native import ext

        out_in_map, row_masks, _ = ext.build_transposed_implicit_gemm_map(
            self.edges.out_rows, self.edges.in_rows, self.edges.kernel_ids,
            self.counts, int(self.n_out_capacity), int(self.n_kernels))
        return RelationImplicitGemmView(out_in_map, row_masks=row_masks)

    def require_sorted_implicit_gemm(self) -> RelationSortedImplicitGemmView:
        """Return or lazily build the mask-sorted view (views.py:467-510):
        ``reorder_rows`` is the stable argsort of the row masks, the maps are
        gathered in that order and ``tile_masks`` ORs each 16-row quarter of
        every 64-row tile."""
        if self.sorted_implicit_gemm is not None:
            return self.sorted_implicit_gemm
        view = self.require_implicit_gemm()
        if view.row_masks.shape[1] != 1:
            raise ValueError(
                'sorted implicit GEMM view currently supports K <= 32.')
        from mlx_lattice_amd._native import ext

        reorder, sorted_map, kv_map, tiles = ext.build_sorted_implicit_gemm_view(
            view.out_in_map, view.row_masks)
        sorted_view = RelationSortedImplicitGemmView(
            sorted_out_in_map=sorted_map, sorted_kv_out_in_map=kv_map,
            reorder_rows=reorder, tile_masks=tiles)
        object.__setattr__(self, 'sorted_implicit_gemm', sorted_view)
        return sorted_view

    def require_transposed_sorted_implicit_gemm(
            self) -> RelationSortedImplicitGemmView:
        """Mask-sorted view of the transposed relation (input row -> output
        row per offset), built on first use and cached: the matrix-core
        route of the input gradient runs the forward's implicit GEMM over
        it.  Forward relations have at most one output row per (input row,
        offset), generative and transposed relations exactly one, and
        submanifold relations too unless a coordinate repeats
        (``transposed_map_exact``, which the input gradient checks first);
        target relations (whose target may repeat a coordinate) are
        refused."""
        if self.transposed_sorted_implicit_gemm is not None:
            return self.transposed_sorted_implicit_gemm
        if self.contract.kind not in ('forward', 'submanifold', 'transposed',
                                      'generative'):
            raise ValueError('the transposed implicit-GEMM view needs a '
                             'forward, submanifold, transposed or generative '
                             'relation.')
        if self.n_in_capacity is None or self.n_kernels is None:
            raise ValueError('kernel relation is missing static shape metadata.')
        if self.n_kernels > 32:
            raise ValueError(
                'sorted implicit GEMM view currently supports K <= 32.')
        from mlx_lattice_amd._native import ext

        in_out_map, row_masks, _ = ext.build_transposed_implicit_gemm_map(
            self.edges.in_rows, self.edges.out_rows, self.edges.kernel_ids,
            self.counts, int(self.n_in_capacity), int(self.n_kernels))
        reorder, sorted_map, kv_map, tiles = ext.build_sorted_implicit_gemm_view(
            in_out_map, row_masks)
        view = RelationSortedImplicitGemmView(
            sorted_out_in_map=sorted_map, sorted_kv_out_in_map=kv_map,
            reorder_rows=reorder, tile_masks=tiles)
        object.__setattr__(self, 'transposed_sorted_implicit_gemm', view)
        return view


# ---------------------------------------------------------------- helpers --


def _validate_row_array(value: torch.Tensor, *, name: str) -> None:
    if value.ndim != 1:
        raise ValueError(f'{name} must have shape (E,).')
    if value.dtype not in _INDEX_DTYPES:
        raise ValueError(f'{name} must be int32 or int64.')


def _validate_coords(value: torch.Tensor, *, name: str) -> None:
    if value.ndim != 2 or value.shape[1] != 4:
        raise ValueError(f'{name} must have shape (N, 4).')
    if value.dtype not in _INDEX_DTYPES:
        raise ValueError(f'{name} must be int32 or int64.')


def _validate_counts(value: torch.Tensor) -> None:
    if tuple(value.shape) != (2,) or value.dtype != torch.int32:
        raise ValueError(
            'relation counts must have shape (2,) and int32 dtype.')


def _validate_active_rows(value: torch.Tensor, *, name: str) -> None:
    if tuple(value.shape) != (1,) or value.dtype != torch.int32:
        raise ValueError(f'{name} must have shape (1,) and int32 dtype.')


def _validate_row_offsets(value: torch.Tensor) -> None:
    if value.ndim != 1 or value.dtype != torch.int32:
        raise ValueError(
            'row_offsets must have shape (N + 1,) and int32 dtype.')


def _require_same_rows(first: torch.Tensor, *rest: torch.Tensor,
                       names: tuple[str, ...]) -> None:
    rows = int(first.shape[0])
    for name, value in zip(names[1:], rest, strict=True):
        if int(value.shape[0]) != rows:
            raise ValueError(
                f'{names[0]} and {name} must have the same row count.')


def _optional_count(value: int | None, name: str) -> int | None:
    if value is None:
        return None
    normalized = int(value)
    if normalized < 0:
        raise ValueError(f'{name} must be non-negative.')
    return normalized
