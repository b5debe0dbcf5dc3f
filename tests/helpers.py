"""Shared helpers for the parity tests (test infrastructure)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / 'golden'


def golden(name: str) -> dict:
    with open(GOLDEN / 'reference_known_answers.json') as fh:
        return json.load(fh)[name]


def to_np(t) -> np.ndarray:
    return t.detach().cpu().numpy()


RELATION_FIELDS = ('in_rows', 'out_rows', 'kernel_ids', 'row_offsets',
                   'out_coords', 'counts', 'in_row_offsets', 'in_edge_ids',
                   'kernel_row_offsets', 'kernel_edge_ids')


def native_relation_dict(native) -> dict:
    out = {name: to_np(value) for name, value in zip(RELATION_FIELDS, native)}
    if len(native) > 10:
        out['out_in_map'] = to_np(native[10])
        out['row_masks'] = to_np(native[11])
    return out


def assert_relation_equal(actual: dict, expected: dict, *,
                          check_coords: bool = True) -> None:
    """Bit-exact comparison of the defined parts of two relations: counts,
    full row_offsets / CSR offsets, active prefixes of the edge arrays and
    edge-id views, and the active output coordinates."""
    np.testing.assert_array_equal(actual['counts'], expected['counts'])
    e = int(expected['counts'][0])
    n_out = int(expected['counts'][1])
    for name in ('in_rows', 'out_rows', 'kernel_ids', 'in_edge_ids',
                 'kernel_edge_ids'):
        np.testing.assert_array_equal(actual[name][:e], expected[name][:e],
                                      err_msg=name)
    for name in ('row_offsets', 'in_row_offsets', 'kernel_row_offsets'):
        np.testing.assert_array_equal(actual[name], expected[name],
                                      err_msg=name)
    if check_coords:
        np.testing.assert_array_equal(actual['out_coords'][:n_out],
                                      expected['out_coords'][:n_out])
