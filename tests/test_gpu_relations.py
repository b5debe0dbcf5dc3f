"""GPU parity of the coordinate hash + kernel-map kernels (bit-exact).

Every case runs the gfx950 relation kernels through the native binding
(which calls the C ABI) and compares with the CPU oracle restating the
reference route (native/features/coordinates/cpu/relation_build_detail.h:
3-80, relation_views_detail.h:15-169).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (assert_relation_equal, extreme_cloud, golden,
                     native_relation_dict, to_np)
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _ext():
    from mlx_lattice_amd._native import ext

    return ext


def _t(a) -> torch.Tensor:
    return torch.as_tensor(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


def _active(n: int) -> torch.Tensor:
    return torch.tensor([n], dtype=torch.int32, device=DEV)


def _triple(v):
    return list(v) if not isinstance(v, int) else [v, v, v]


def _with_grouped_views(native, in_capacity, k):
    """The *_with_view builders skip the grouped CSR views; build them with
    the on-demand entry point, as the Python relation does."""
    views = _ext().build_relation_grouped_views(native[0], native[2], native[5],
                                                in_capacity, k)
    return tuple(native[:6]) + tuple(views) + tuple(native[10:])


def gpu_forward(coords, active=None, kernel_size=3, stride=1, padding=0,
                dilation=1) -> dict:
    c = _t(coords)
    n = c.shape[0] if active is None else active
    native = _ext().build_kernel_relation_with_view(
        c, _active(n), _triple(kernel_size), _triple(stride),
        _triple(padding), _triple(dilation))
    k = len(O.kernel_offsets(kernel_size, dilation))
    native = _with_grouped_views(native, c.shape[0], k)
    torch.cuda.synchronize()
    return native_relation_dict(native)


def gpu_target(coords, target, kernel_size=3, stride=1, padding=0,
               dilation=1, active=None, target_active=None) -> dict:
    c = _t(coords)
    t = _t(target)
    n = c.shape[0] if active is None else active
    tn = t.shape[0] if target_active is None else target_active
    native = _ext().build_target_kernel_relation_with_view(
        c, _active(n), t, _active(tn), _triple(kernel_size),
        _triple(stride), _triple(padding), _triple(dilation))
    k = len(O.kernel_offsets(kernel_size, dilation))
    native = _with_grouped_views(native, c.shape[0], k)
    torch.cuda.synchronize()
    return native_relation_dict(native)


def check_forward(coords, active=None, **geom) -> dict:
    print(f'forward relation rows={len(coords)} active={active} {geom}',
          flush=True)
    actual = gpu_forward(coords, active, **geom)
    expected = O.kernel_relation(coords, active, **geom)
    assert_relation_equal(actual, expected)
    # The dense view produced by the same pass equals the reference view.
    offs = O.kernel_offsets(geom.get('kernel_size', 3),
                            geom.get('dilation', 1))
    n_out = int(expected['counts'][1])
    src_active = len(coords) if active is None else active
    om, rm = O.implicit_gemm_view(coords, src_active, expected['out_coords'],
                                  n_out, offs, geom.get('stride', 1),
                                  geom.get('padding', 0))
    np.testing.assert_array_equal(actual['out_in_map'], om)
    np.testing.assert_array_equal(actual['row_masks'], rm)
    return actual


# ------------------------------------------------------------ golden ----


def test_golden_forward_relation_line():
    g = golden('forward_relation_line')
    actual = gpu_forward(g['coords'], kernel_size=g['kernel_size'])
    e = g['counts'][0]
    assert actual['counts'].tolist() == g['counts']
    assert actual['out_coords'].tolist() == g['out_coords']
    for name in ('in_rows', 'out_rows', 'kernel_ids', 'in_edge_ids',
                 'kernel_edge_ids'):
        assert actual[name][:e].tolist() == g[name], name
    for name in ('row_offsets', 'in_row_offsets', 'kernel_row_offsets'):
        assert actual[name].tolist() == g[name], name


def test_eager_ten_tuple_matches_on_demand_views():
    from mlx_lattice_amd.synthetic import config_rng, uniform_grid_cloud

    coords = uniform_grid_cloud(3000, 20, rng=config_rng(1))
    lazy = gpu_forward(coords, kernel_size=3)
    eager = native_relation_dict(_ext().build_kernel_relation(
        _t(coords), _active(len(coords)), [3, 3, 3], [1, 1, 1], [0, 0, 0],
        [1, 1, 1]))
    assert_relation_equal(eager, lazy)
    expected = O.kernel_relation(coords, kernel_size=3)
    assert_relation_equal(eager, expected)
    assert len(_ext().build_kernel_relation(
        _t(coords), _active(len(coords)), [3, 3, 3], [1, 1, 1], [0, 0, 0],
        [1, 1, 1])) == 10


def test_golden_target_relation_line():
    g = golden('target_relation_line')
    actual = gpu_target(g['coords'], g['target'], kernel_size=g['kernel_size'])
    e = g['counts'][0]
    assert actual['counts'].tolist() == g['counts']
    for name in ('in_rows', 'out_rows', 'kernel_ids'):
        assert actual[name][:e].tolist() == g[name], name
    assert actual['row_offsets'].tolist() == g['row_offsets']


def test_golden_strided_relation():
    g = golden('strided_relation_pointwise')
    actual = gpu_forward(g['coords'], kernel_size=g['kernel_size'],
                         stride=g['stride'])
    assert actual['counts'].tolist() == g['counts']
    assert actual['out_coords'][:2].tolist() == g['out_coords']
    assert actual['in_rows'][:2].tolist() == g['in_rows']


@pytest.mark.parametrize('name', ['downsample_first_seen',
                                  'downsample_negative_duplicates'])
def test_golden_downsample_first_seen(name):
    g = golden(name)
    actual = gpu_forward(g['coords'], kernel_size=1, stride=g['stride'])
    n = int(actual['counts'][1])
    assert actual['out_coords'][:n].tolist() == g['out_coords']


def test_golden_implicit_gemm_views():
    g = golden('implicit_gemm_view_forward')
    actual = gpu_forward(g['coords'], kernel_size=g['kernel_size'])
    assert actual['out_in_map'].tolist() == g['out_in_map']
    assert actual['row_masks'].tolist() == g['row_masks']
    g = golden('implicit_gemm_view_target')
    actual = gpu_target(g['coords'], g['target'], kernel_size=g['kernel_size'])
    assert actual['out_in_map'].tolist() == g['out_in_map']
    assert actual['row_masks'].tolist() == g['row_masks']
    g = golden('implicit_gemm_view_33')
    actual = gpu_forward(g['coords'], kernel_size=g['kernel_size'])
    assert list(actual['out_in_map'].shape) == g['out_in_map_shape']
    assert int(actual['out_in_map'][0, 16]) == g['out_in_map_16']
    assert actual['row_masks'].tolist() == g['row_masks']


def test_golden_standalone_implicit_gemm_view():
    g = golden('implicit_gemm_view_target')
    src = _t(g['coords'])
    dst = _t(g['target'])
    offs = _t(O.kernel_offsets(g['kernel_size']))
    om, rm = _ext().build_relation_implicit_gemm_view(
        src, _active(3), dst, _active(2), offs, [1, 1, 1], [0, 0, 0])
    assert to_np(om).tolist() == g['out_in_map']
    assert to_np(rm).tolist() == g['row_masks']


def test_golden_sorted_view():
    g = golden('sorted_view_line')
    actual = gpu_forward(g['coords'], kernel_size=g['kernel_size'])
    reorder, sorted_map, kv, tiles = _ext().build_sorted_implicit_gemm_view(
        _t(actual['out_in_map']), _t(actual['row_masks']))
    assert to_np(reorder).tolist() == g['reorder_rows']
    assert to_np(sorted_map).tolist() == g['sorted_out_in_map']
    assert to_np(kv).tolist() == g['sorted_kv_out_in_map']
    assert to_np(tiles).tolist() == g['tile_masks']


# ----------------------------------------------------- edge cases ----


def test_empty_and_inactive_rows():
    empty = np.zeros((0, 4), np.int32)
    actual = gpu_forward(empty)
    assert actual['counts'].tolist() == [0, 0]
    assert actual['row_offsets'].tolist() == [0]
    coords = np.array([[0, 0, 0, 0], [0, 1, 0, 0], [0, 2, 0, 0],
                       [0, 3, 0, 0]], np.int32)
    check_forward(coords, active=2, kernel_size=(3, 1, 1))
    check_forward(coords, active=0, kernel_size=(3, 1, 1))
    check_forward(coords, active=3, kernel_size=(3, 1, 1), stride=2)


def test_duplicates_negative_and_batches():
    rng = np.random.default_rng(7)
    coords = rng.integers(-6, 6, size=(600, 4)).astype(np.int32)
    coords[:, 0] = rng.integers(0, 3, size=600)
    check_forward(coords)                                   # duplicates kept
    check_forward(coords, kernel_size=2, stride=2)          # first-seen cells
    check_forward(coords, kernel_size=3, stride=2, padding=1)
    check_forward(coords, kernel_size=3, stride=1, padding=1)
    check_forward(coords, kernel_size=(3, 3, 3), dilation=2)
    check_forward(coords, kernel_size=(5, 5, 5))            # K = 125 > 64
    check_forward(coords, kernel_size=(3, 3, 5))            # K = 45
    tgt = rng.integers(-4, 4, size=(300, 4)).astype(np.int32)
    tgt[:, 0] = rng.integers(0, 3, size=300)
    for geom in (dict(kernel_size=3), dict(kernel_size=2, stride=2),
                 dict(kernel_size=3, stride=2, padding=1)):
        actual = gpu_target(coords, tgt, **geom)
        expected = O.target_kernel_relation(coords, tgt, **geom)
        assert_relation_equal(actual, expected, check_coords=False)


@pytest.mark.parametrize('geom', [
    dict(kernel_size=3),
    dict(kernel_size=2, stride=2),
    dict(kernel_size=3, stride=2, padding=1),
    dict(kernel_size=3, dilation=2),
    dict(kernel_size=(3, 1, 2), stride=(1, 3, 2)),
])
def test_full_int32_domain_forward(geom):
    """Coordinates anywhere in int32 (the reference hashes all four words,
    cpu/common_detail.h:68-107): bit-exact against the oracle."""
    coords = extreme_cloud(71)
    check_forward(coords, **geom)
    check_forward(coords, active=len(coords) - 37, **geom)


@pytest.mark.parametrize('geom', [dict(kernel_size=3),
                                  dict(kernel_size=2, stride=2)])
def test_full_int32_domain_target(geom):
    coords = extreme_cloud(72)
    target = extreme_cloud(73)[:400]
    print(f'target relation extreme domain {geom}', flush=True)
    actual = gpu_target(coords, target, **geom)
    expected = O.target_kernel_relation(coords, target, **geom)
    assert_relation_equal(actual, expected, check_coords=False)


def test_full_int32_domain_through_the_operators():
    """subm_conv3d and a k2s2 conv3d over an extreme-domain cloud: the
    relations behind the operators match the oracle's, and so do the
    features (fp32, rtol 1e-3)."""
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor

    coords = extreme_cloud(74)
    rng = np.random.default_rng(74)
    feats = rng.standard_normal((len(coords), 8)).astype(np.float32)
    w = (rng.standard_normal((16, 3, 3, 3, 8)) * 0.2).astype(np.float32)
    x = SparseTensor(_t(coords), torch.as_tensor(feats).to(DEV))
    out = ops.subm_conv3d(x, torch.as_tensor(w).to(DEV), kernel_size=3)
    rel = O.kernel_relation(coords, kernel_size=3)
    ref = O.conv_features_fp64(feats, O.mapped_weight(w.astype(np.float64)),
                               rel)
    got = out.feats.cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-4)
    w2 = (rng.standard_normal((8, 2, 2, 2, 8)) * 0.2).astype(np.float32)
    down = ops.conv3d(x, torch.as_tensor(w2).to(DEV), kernel_size=2, stride=2)
    rel2 = O.kernel_relation(coords, kernel_size=2, stride=2)
    n = int(rel2['counts'][1])
    assert int(down.active_rows.item()) == n
    np.testing.assert_array_equal(down.coords[:n].cpu().numpy(),
                                  rel2['out_coords'][:n])
    ref2 = O.conv_features_fp64(feats, O.mapped_weight(w2.astype(np.float64)),
                                rel2)
    np.testing.assert_allclose(down.feats[:n].cpu().numpy(), ref2[:n],
                               rtol=1e-3, atol=1e-4)


def test_range_edges_are_exact():
    lo, hi = -131072, 131071
    coords = np.array([[0, lo, lo, lo], [0, hi, hi, hi], [1022, lo, 0, hi],
                       [0, lo + 1, lo, lo], [0, hi - 1, hi, hi]], np.int32)
    check_forward(coords)
    check_forward(coords, kernel_size=2, stride=2)


def test_repeated_builds_are_deterministic():
    from mlx_lattice_amd.synthetic import config_rng, uniform_grid_cloud

    coords = uniform_grid_cloud(5000, 24, rng=config_rng(1))
    first = gpu_forward(coords)
    e = int(first['counts'][0])
    for _ in range(3):
        again = gpu_forward(coords)
        np.testing.assert_array_equal(first['counts'], again['counts'])
        # Edge arrays are defined on their active prefix only.
        for name in ('in_rows', 'in_edge_ids', 'kernel_edge_ids'):
            np.testing.assert_array_equal(first[name][:e], again[name][:e])
        for name in ('row_offsets', 'out_in_map', 'row_masks'):
            np.testing.assert_array_equal(first[name], again[name])


# ------------------------------------------------ benchmark configs ----


def test_config1_submanifold_map():
    from mlx_lattice_amd.synthetic import config_rng, uniform_grid_cloud

    coords = uniform_grid_cloud(20000, 64, rng=config_rng(1))
    check_forward(coords, kernel_size=3)


def test_config2_downsample_map():
    from mlx_lattice_amd.synthetic import config_rng, lidar_cloud

    coords = lidar_cloud(100000, 2, rng=config_rng(2))
    actual = check_forward(coords, kernel_size=2, stride=2)
    # k=2, s=2, p=0: every active input feeds exactly one (out, k) pair.
    assert int(actual['counts'][0]) == len(coords)


def test_config3_submanifold_map_400k():
    from mlx_lattice_amd.synthetic import config_rng, sphere_shell_cloud

    coords = sphere_shell_cloud(400000, 512, rng=config_rng(3))
    actual = check_forward(coords, kernel_size=3)
    # Every active row of a submanifold map has its own centre edge.
    n = len(coords)
    assert (actual['out_in_map'][:n, 13] == np.arange(n)).all()


def test_config5_stage_chain():
    from mlx_lattice_amd.synthetic import config_rng, lidar_cloud

    coords = lidar_cloud(30000, 4, rng=config_rng(5))
    check_forward(coords, kernel_size=3)
    level = coords
    for _ in range(3):
        rel = check_forward(level, kernel_size=2, stride=2)
        n = int(rel['counts'][1])
        level = rel['out_coords'][:n]
        check_forward(level, kernel_size=3)


def test_sorted_view_matches_stable_argsort():
    from mlx_lattice_amd.synthetic import config_rng, sphere_shell_cloud

    coords = sphere_shell_cloud(30000, 160, rng=config_rng(3))
    actual = gpu_forward(coords, kernel_size=3)
    reorder, sorted_map, kv, tiles = _ext().build_sorted_implicit_gemm_view(
        _t(actual['out_in_map']), _t(actual['row_masks']))
    masks = actual['row_masks'][:, 0]
    expect = np.argsort(masks, kind='stable')
    np.testing.assert_array_equal(to_np(reorder), expect)
    smap = actual['out_in_map'][expect]
    np.testing.assert_array_equal(to_np(sorted_map), smap)
    np.testing.assert_array_equal(to_np(kv), smap.T)
    n = len(coords)
    pad = (-n) % 64
    sm = np.concatenate([masks[expect], np.zeros(pad, masks.dtype)])
    quarters = np.bitwise_or.reduce(sm.reshape(-1, 16), axis=1)
    np.testing.assert_array_equal(to_np(tiles), quarters)


@pytest.mark.parametrize('rows,k,seed', [(1, 27, 0), (2047, 27, 1),
                                          (2048, 27, 2), (2049, 27, 3),
                                          (50000, 5, 4), (70001, 32, 5),
                                          (300000, 27, 6)])
def test_sorted_view_sort_edge_cases(rows, k, seed):
    """The device radix sort behind the sorted view, against numpy's stable
    argsort: tile boundaries (2048 items per tile), one-pass keys (K = 5),
    32-bit masks ordered as signed int32 (sign bit set), and many ties."""
    rng = np.random.default_rng(seed)
    if k == 32:
        masks = rng.integers(-2**31, 2**31, size=rows, dtype=np.int64)
    else:
        # few distinct masks -> long runs of ties across tiles
        pool = rng.integers(0, 2**k, size=max(1, rows // 500))
        masks = pool[rng.integers(0, len(pool), size=rows)]
    masks = masks.astype(np.int32).reshape(rows, 1)
    out_in_map = rng.integers(-1, 1000, size=(rows, k)).astype(np.int32)
    reorder, sorted_map, kv, tiles = _ext().build_sorted_implicit_gemm_view(
        _t(out_in_map), _t(masks))
    expect = np.argsort(masks[:, 0], kind='stable')
    np.testing.assert_array_equal(to_np(reorder), expect)
    np.testing.assert_array_equal(to_np(sorted_map), out_in_map[expect])
    np.testing.assert_array_equal(to_np(kv), out_in_map[expect].T)
    pad = (-rows) % 64
    sm = np.concatenate([masks[expect, 0], np.zeros(pad, np.int32)])
    np.testing.assert_array_equal(to_np(tiles),
                                  np.bitwise_or.reduce(sm.reshape(-1, 16),
                                                       axis=1))


def test_python_relation_views_on_demand():
    from mlx_lattice_amd.core.coords.builders import (
        build_kernel_relation,
        build_submanifold_kernel_relation,
    )
    from mlx_lattice_amd.synthetic import config_rng, uniform_grid_cloud

    coords = uniform_grid_cloud(4000, 24, rng=config_rng(1))
    for build, kw, geom in ((build_submanifold_kernel_relation,
                             dict(kernel_size=3), dict(kernel_size=3)),
                            (build_kernel_relation,
                             dict(kernel_size=2, stride=2),
                             dict(kernel_size=2, stride=2))):
        rel = build(_t(coords), **kw)
        assert rel._input_csr is None  # not built by the forward path
        expected = O.kernel_relation(coords, **geom)
        e = int(expected['counts'][0])
        np.testing.assert_array_equal(to_np(rel.in_row_offsets),
                                      expected['in_row_offsets'])
        np.testing.assert_array_equal(to_np(rel.in_edge_ids)[:e],
                                      expected['in_edge_ids'][:e])
        np.testing.assert_array_equal(to_np(rel.kernel_row_offsets),
                                      expected['kernel_row_offsets'])
        np.testing.assert_array_equal(to_np(rel.kernel_edge_ids)[:e],
                                      expected['kernel_edge_ids'][:e])


@pytest.mark.parametrize('n,groups,valid', [(3_000_000, 5000, 2_900_000),
                                            (4_200_000, 2**26, 4_200_000),
                                            (5000, 70000, 4000)])
def test_group_by_key_large_sorts(n, groups, valid):
    """The device radix sort at edge-list sizes (up to 2,051 tiles of 2048
    items, one to three digit passes), through the stable grouping: the ids
    are numpy's stable argsort of the keys, with keys outside [0, groups)
    and positions at or past the count left out (sorted past the groups)."""
    rng = np.random.default_rng(n % 97)
    keys = rng.integers(-3, groups, size=n).astype(np.int32)
    keys[: n // 3] = keys[n // 3: 2 * (n // 3)]   # long runs of equal keys
    print(f'group_by_key n={n} groups={groups}', flush=True)
    offsets, ids = _ext().group_by_key(_t(keys), _active(valid), groups)
    torch.cuda.synchronize()
    k = keys.astype(np.int64).copy()
    k[valid:] = groups
    k[(k < 0) | (k >= groups)] = groups
    expect = np.argsort(k, kind='stable')
    inside = int((k < groups).sum())
    np.testing.assert_array_equal(to_np(ids)[:inside], expect[:inside])
    counts = np.bincount(k[k < groups], minlength=groups)
    np.testing.assert_array_equal(
        to_np(offsets), np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))


@pytest.mark.parametrize('ks,stride', [(2, 2), (3, 2), (3, 1)])
def test_forward_relation_reuses_the_submanifold_block_table(ks, stride):
    """A forward relation built over the block table a submanifold relation
    of the same coordinates left in its workspace
    (LATTICE_RELATION_TABLE_READY) equals one built from scratch, bit for
    bit; the manager hands the table over once."""
    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd.core.coords.builders import build_kernel_relation

    if ks == 3 and stride == 1:
        coords = extreme_cloud(40 + ks)
    else:
        from mlx_lattice_amd.synthetic import lidar_cloud
        coords = lidar_cloud(3000, 2, rng=np.random.default_rng(40 + ks))
    n = len(coords)
    c = _t(coords)
    x = SparseTensor(c, torch.zeros((n, 4), device=DEV))
    mgr = x.coord_manager
    mgr.submanifold_kernel_relation(x.coord_key, kernel_size=3)
    assert x.coord_key in mgr._block_tables
    # only the table is kept: one 64-byte bucket per block-table slot
    # (a power of two above 1.5 n), not the rest of the build's workspace
    kept = mgr._block_tables[x.coord_key][0]
    assert kept.numel() <= 64 * 2 * (n + n // 2 + 1) + 4096
    print(f'table reuse k={ks} s={stride} N={n}', flush=True)
    reused = mgr.kernel_relation(x.coord_key, kernel_size=ks, stride=stride)
    assert x.coord_key not in mgr._block_tables
    fresh = build_kernel_relation(c, _active(n), kernel_size=ks,
                                  stride=stride)
    torch.cuda.synchronize()

    def arrays(rel):
        return {'in_rows': to_np(rel.edges.in_rows),
                'out_rows': to_np(rel.edges.out_rows),
                'kernel_ids': to_np(rel.edges.kernel_ids),
                'counts': to_np(rel.counts),
                'row_offsets': to_np(rel.output_csr.row_offsets),
                'in_row_offsets': to_np(rel.input_csr.row_offsets),
                'in_edge_ids': to_np(rel.input_csr.edge_ids),
                'kernel_row_offsets': to_np(rel.kernel_csr.row_offsets),
                'kernel_edge_ids': to_np(rel.kernel_csr.edge_ids),
                'out_coords': to_np(rel.out_coords)}

    assert_relation_equal(arrays(reused), arrays(fresh))
    n_out = int(fresh.counts[1].item())
    np.testing.assert_array_equal(
        to_np(reused.require_implicit_gemm().out_in_map)[:n_out],
        to_np(fresh.require_implicit_gemm().out_in_map)[:n_out])


def test_block_table_is_not_reused_on_another_stream():
    """The kept block table was written on the stream of its submanifold
    build; a forward relation over the same key built on another stream
    hashes the coordinates again (no cross-stream read) and still matches
    a fresh build."""
    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd.core.coords.builders import build_kernel_relation
    from mlx_lattice_amd.synthetic import lidar_cloud

    coords = lidar_cloud(3000, 2, rng=np.random.default_rng(47))
    n = len(coords)
    c = _t(coords)
    x = SparseTensor(c, torch.zeros((n, 4), device=DEV))
    mgr = x.coord_manager
    mgr.submanifold_kernel_relation(x.coord_key, kernel_size=3)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    kept = mgr._block_tables[x.coord_key]
    print(f'table reuse across streams N={n}', flush=True)
    with torch.cuda.stream(side):
        assert mgr._take_block_table(x.coord_key) is None
        mgr._block_tables[x.coord_key] = kept
        other = mgr.kernel_relation(x.coord_key, kernel_size=2, stride=2)
    assert x.coord_key not in mgr._block_tables
    torch.cuda.current_stream().wait_stream(side)
    fresh = build_kernel_relation(c, _active(n), kernel_size=2, stride=2)
    torch.cuda.synchronize()
    e = int(fresh.counts[0].item())
    np.testing.assert_array_equal(to_np(other.counts), to_np(fresh.counts))
    np.testing.assert_array_equal(to_np(other.edges.in_rows)[:e],
                                  to_np(fresh.edges.in_rows)[:e])
    np.testing.assert_array_equal(to_np(other.edges.out_rows)[:e],
                                  to_np(fresh.edges.out_rows)[:e])
