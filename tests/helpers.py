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


I32_MIN, I32_MAX = -2**31, 2**31 - 1


def extreme_cloud(seed: int, per_blob: int = 60) -> np.ndarray:
    """Blobs of voxels around anchors across the whole int32 domain: the
    axis limits, large negatives, batch ids above the packed range and
    negative ones, and the edges of the packed range itself, so that
    neighbours, downsampled cells and targets cross every boundary.  Mixed
    with a few in-range rows and repeated coordinates."""
    rng = np.random.default_rng(seed)
    anchors = [
        (0, I32_MAX - 2, I32_MAX - 2, I32_MAX - 2),
        (0, I32_MIN, I32_MIN, I32_MIN),
        (3, I32_MIN + 1, I32_MAX - 1, 0),
        (2**31 - 1, 0, 0, 0),
        (-7, 100, -100, 5),
        (1023, 5, 5, 5),
        (5000, -1_000_000_000, 123_456_789, -42),
        (0, 131070, -131073, 131071),
        (0, -131072, 131071, -5),
        (I32_MIN, I32_MAX - 1, I32_MIN, I32_MAX - 1),
    ]
    rows = []
    for b, x, y, z in anchors:
        d = rng.integers(-2, 3, (per_blob, 3))
        c = np.array([x, y, z], np.int64) + d
        c = np.clip(c, I32_MIN, I32_MAX)
        rows.append(np.concatenate([np.full((per_blob, 1), b, np.int64), c], 1))
    rows.append(np.concatenate([rng.integers(0, 3, (200, 1)),
                                rng.integers(-20, 20, (200, 3))], 1))
    coords = np.concatenate(rows)
    coords = coords[rng.permutation(len(coords))]
    coords[len(coords) // 2] = coords[3]      # repeated coordinates
    coords[len(coords) // 3] = coords[11]
    return coords.astype(np.int32)
