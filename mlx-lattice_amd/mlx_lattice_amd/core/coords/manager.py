"""Coordinate identity and relation cache (mlx_lattice/core/coords/
manager.py:29-305), over torch tensors."""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass, field
from itertools import count

import torch

from mlx_lattice_amd.core.coords.builders import (
    build_generative_relation,
    build_kernel_relation,
    build_submanifold_kernel_relation,
    build_target_kernel_relation,
    build_transposed_kernel_relation,
)
from mlx_lattice_amd.core.coords.validation import validate_coords
from mlx_lattice_amd.core.relations import KernelRelation, KernelSpec
from mlx_lattice_amd.core.types import Triple, triple

_manager_ids = count()


def _next_manager_id() -> int:
    return next(_manager_ids)


@dataclass(frozen=True, slots=True)
class CoordinateMapKey:
    """Opaque coordinate identity key owned by a ``CoordinateManager``;
    ``stride`` is part of the identity."""

    id: int
    stride: Triple
    manager_id: int


@dataclass(slots=True)
class CoordinateManager:
    """Owns coordinate arrays and caches relations by (key, target key,
    KernelSpec, kind)."""

    _manager_id: int = field(default_factory=_next_manager_id, init=False)
    _next_id: int = 0
    _coords: dict[CoordinateMapKey, torch.Tensor] = field(default_factory=dict)
    _identity_keys: dict[tuple[int, int, Triple], CoordinateMapKey] = field(
        default_factory=dict)
    _default_identity_keys: dict[tuple[int, Triple], CoordinateMapKey] = field(
        default_factory=dict)
    _active_rows: dict[CoordinateMapKey, torch.Tensor] = field(
        default_factory=dict)
    _kernel_relations: dict[
        tuple[CoordinateMapKey, CoordinateMapKey | None, KernelSpec, str],
        KernelRelation] = field(default_factory=dict)
    # The block table of the last submanifold relation built over a key
    # (its buffer only, not the rest of the build's workspace) and the
    # stream it was written on (64 B per bucket, 1.5-3 buckets per row): the
    # next forward relation over the same key takes the entry, and reuses
    # the table when it runs on that stream.
    _block_tables: dict[CoordinateMapKey, tuple[torch.Tensor, object]] = field(
        default_factory=dict)

    def insert_coords(self, coords: torch.Tensor,
                      stride: int | Sequence[int] = 1,
                      active_rows: torch.Tensor | None = None,
                      ) -> CoordinateMapKey:
        """Register a coordinate array by object identity and stride
        (manager.py:71-115)."""
        validate_coords(coords)
        normalized = triple(stride, name='stride')
        if active_rows is None:
            default_key = (id(coords), normalized)
            if default_key in self._default_identity_keys:
                return self._default_identity_keys[default_key]
            # a device fill: no host-to-device copy to wait for
            active = torch.full((1,), coords.shape[0], dtype=torch.int32,
                                device=coords.device)
        else:
            active = active_rows
        cache_key = (id(coords), id(active), normalized)
        if cache_key in self._identity_keys:
            return self._identity_keys[cache_key]
        key = CoordinateMapKey(self._next_id, normalized, self._manager_id)
        self._next_id += 1
        self._coords[key] = coords
        self._active_rows[key] = active
        self._identity_keys[cache_key] = key
        if active_rows is None:
            self._default_identity_keys[(id(coords), normalized)] = key
        return key

    def owns(self, key: CoordinateMapKey) -> bool:
        return key.manager_id == self._manager_id and key in self._coords

    def coords(self, key: CoordinateMapKey) -> torch.Tensor:
        if not self.owns(key):
            raise ValueError('coordinate key does not belong to this manager.')
        return self._coords[key]

    def active_rows(self, key: CoordinateMapKey) -> torch.Tensor:
        if not self.owns(key):
            raise ValueError('coordinate key does not belong to this manager.')
        return self._active_rows[key]

    def kernel_relation(self, key: CoordinateMapKey, *,
                        kernel_size: int | Sequence[int] = 3,
                        stride: int | Sequence[int] = 1,
                        padding: int | Sequence[int] = 0,
                        dilation: int | Sequence[int] = 1) -> KernelRelation:
        """Build or reuse a forward relation (manager.py:142-174)."""
        spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                          dilation=dilation)
        cache_key = (key, None, spec, 'forward')
        if cache_key not in self._kernel_relations:
            self._kernel_relations[cache_key] = build_kernel_relation(
                self.coords(key), active_rows=self.active_rows(key),
                kernel_size=spec.size, stride=spec.stride,
                padding=spec.padding, dilation=spec.dilation,
                table=self._take_block_table(key))
        return self._kernel_relations[cache_key]

    def _take_block_table(self, key: CoordinateMapKey) -> torch.Tensor | None:
        """Pop the key's kept block table; hand it out only when the
        current stream is the one that wrote it (stream order then makes
        the table complete before the new build reads it)."""
        entry = self._block_tables.pop(key, None)
        if entry is None:
            return None
        table, stream = entry
        if table.is_cuda and torch.cuda.current_stream(table.device) != stream:
            return None
        return table

    def generative_relation(self, key: CoordinateMapKey, *,
                            kernel_size: int | Sequence[int] = 2,
                            stride: int | Sequence[int] = 2) -> KernelRelation:
        """Build or reuse a generative transpose-convolution relation
        (manager.py:176-198)."""
        spec = KernelSpec(size=kernel_size, stride=stride)
        cache_key = (key, None, spec, 'generative')
        if cache_key not in self._kernel_relations:
            self._kernel_relations[cache_key] = build_generative_relation(
                self.coords(key), active_rows=self.active_rows(key),
                kernel_size=spec.size, stride=spec.stride)
        return self._kernel_relations[cache_key]

    def transposed_kernel_relation(self, key: CoordinateMapKey, *,
                                   kernel_size: int | Sequence[int] = 2,
                                   stride: int | Sequence[int] = 2,
                                   padding: int | Sequence[int] = 0,
                                   dilation: int | Sequence[int] = 1
                                   ) -> KernelRelation:
        """Build or reuse a transpose-convolution relation
        (manager.py:231-264)."""
        spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                          dilation=dilation)
        cache_key = (key, None, spec, 'transpose')
        if cache_key not in self._kernel_relations:
            self._kernel_relations[cache_key] = (
                build_transposed_kernel_relation(
                    self.coords(key), active_rows=self.active_rows(key),
                    kernel_size=spec.size, stride=spec.stride,
                    padding=spec.padding, dilation=spec.dilation))
        return self._kernel_relations[cache_key]

    def submanifold_kernel_relation(
            self, key: CoordinateMapKey, *,
            kernel_size: int | Sequence[int] = 3,
            dilation: int | Sequence[int] = 1) -> KernelRelation:
        """Build or reuse a submanifold relation (manager.py:200-229)."""
        spec = KernelSpec(size=kernel_size, stride=1, padding=0,
                          dilation=dilation)
        cache_key = (key, key, spec, 'submanifold')
        if cache_key not in self._kernel_relations:
            relation = build_submanifold_kernel_relation(
                self.coords(key), active_rows=self.active_rows(key),
                kernel_size=spec.size, dilation=spec.dilation,
                keep_table=True)
            table = relation.block_table
            if table is not None:
                stream = (torch.cuda.current_stream(table.device)
                          if table.is_cuda else None)
                self._block_tables[key] = (table, stream)
                object.__setattr__(relation, 'block_table', None)
            self._kernel_relations[cache_key] = relation
        return self._kernel_relations[cache_key]

    def target_kernel_relation(
            self, key: CoordinateMapKey, target_key: CoordinateMapKey, *,
            kernel_size: int | Sequence[int] = 3,
            stride: int | Sequence[int] = 1,
            padding: int | Sequence[int] = 0,
            dilation: int | Sequence[int] = 1) -> KernelRelation:
        """Build or reuse a relation to explicit target coords
        (manager.py:266-305)."""
        if not self.owns(key) or not self.owns(target_key):
            raise ValueError(
                'input and target coordinate keys must belong to this manager.')
        spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                          dilation=dilation)
        cache_key = (key, target_key, spec, 'target')
        if cache_key not in self._kernel_relations:
            self._kernel_relations[cache_key] = build_target_kernel_relation(
                self.coords(key), self.coords(target_key),
                active_rows=self.active_rows(key),
                target_active_rows=self.active_rows(target_key),
                kernel_size=spec.size, stride=spec.stride,
                padding=spec.padding, dilation=spec.dilation)
        return self._kernel_relations[cache_key]
