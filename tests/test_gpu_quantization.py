"""GPU parity of point -> voxel quantization and the point <-> voxel feature
maps (mlx_lattice/core/coords/quantization.py, ops/quantization.py; CPU
routines native/features/coordinates/cpu/quantization_detail.h:66-391).

Integer outputs (voxel coordinates, inverse rows, counts, map rows) are
bit-exact against the oracle.  The float outputs use one IEEE rounding per
operation in the same order as the oracle, so they are compared exactly as
well (the documented tolerance, rtol=1e-6, is only used for the reference's
hand-written known answers, which the reference itself compares with
assert_nested_close).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import golden, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _ops():
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor

    return ops, SparseTensor


def _f(a) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, np.float32)).to(DEV)


def _i(a) -> torch.Tensor:
    return torch.as_tensor(np.asarray(a, np.int32)).to(DEV)


# ------------------------------------------------------------ golden ----


def test_golden_sparse_quantize():
    ops, _ = _ops()
    g = golden('quantize_ordered_metadata')
    q = ops.sparse_quantize(_f(g['points']), tuple(g['voxel_size']),
                            batch_indices=_i(g['batch_indices']))
    n = int(q.active_rows.item())
    assert q.capacity == g['capacity']
    assert q.active_count is q.active_rows
    assert to_np(q.active_rows).tolist() == g['active_rows']
    assert to_np(q.coords[:n]).tolist() == g['coords']
    assert to_np(q.inverse_rows).tolist() == g['inverse_rows']
    assert to_np(q.counts[:n]).tolist() == g['counts']
    g = golden('quantize_origin_active_rows')
    q = ops.sparse_quantize(_f(g['points']), tuple(g['voxel_size']),
                            origin=tuple(g['origin']),
                            active_rows=_i(g['active_rows_in']))
    n = int(q.active_rows.item())
    assert to_np(q.active_rows).tolist() == g['active_rows']
    assert to_np(q.coords[:n]).tolist() == g['coords']
    assert to_np(q.inverse_rows).tolist() == g['inverse_rows']
    assert to_np(q.counts).tolist() == g['counts_full']


def test_golden_voxelize():
    ops, SparseTensor = _ops()
    g = golden('voxelize_mean_sum')
    pts, feats = _f(g['points']), _f(g['feats'])
    mean = ops.voxelize(pts, feats, voxel_size=g['voxel_size'],
                        reduction='mean')
    summed = ops.voxelize(pts, feats, voxel_size=g['voxel_size'],
                          reduction='sum')
    n = int(mean.active_rows.item())
    assert to_np(mean.coords[:n]).tolist() == g['coords']
    np.testing.assert_allclose(to_np(mean.feats[:n]), g['mean'], rtol=1e-6)
    np.testing.assert_allclose(to_np(summed.feats[:n]), g['sum'], rtol=1e-6)
    assert mean.stride == tuple(g['stride'])
    # voxelize_with_quantization with a template
    q = ops.sparse_quantize(pts)
    template = SparseTensor(q.coords, torch.zeros_like(feats),
                            active_rows=q.active_rows)
    mapped = ops.voxelize_with_quantization(q, feats, reduction='mean',
                                            template=template)
    assert mapped.same_coords(template)
    np.testing.assert_allclose(to_np(mapped.feats[:n]), g['mean'],
                               rtol=1e-6)


def test_golden_voxelize_gradient():
    ops, _ = _ops()
    g = golden('voxelize_grad')
    pts = _f(g['points'])
    feats = _f(g['feats']).requires_grad_(True)
    out = ops.voxelize(pts, feats, reduction=g['reduction'])
    n = int(out.active_rows.item())
    np.testing.assert_allclose(to_np(out.feats[:n]), g['features'],
                               rtol=1e-6)
    out.feats[:n].sum().backward()
    np.testing.assert_allclose(to_np(feats.grad), g['grad'], rtol=1e-6)
    with torch.no_grad():
        jvp = ops.voxelize(pts, _f(g['tangent']), reduction=g['reduction'])
    np.testing.assert_allclose(to_np(jvp.feats[:n]), g['jvp'], rtol=1e-6)


def test_golden_devoxelize():
    ops, SparseTensor = _ops()
    g = golden('devoxelize_nearest')
    vox = SparseTensor(_i(g['coords']), _f(g['feats']))
    got = ops.devoxelize(_f(g['points']), vox, interpolation='nearest')
    np.testing.assert_allclose(to_np(got), g['sampled'], rtol=1e-6)
    g = golden('devoxelize_linear')
    vox = SparseTensor(_i(g['coords']), _f(g['feats']))
    got = ops.devoxelize(_f(g['points']), vox, interpolation='linear')
    np.testing.assert_allclose(to_np(got), g['sampled'], rtol=1e-6)
    g = golden('point_voxel_map_reuse')
    vox = SparseTensor(_i(g['coords']), _f(g['feats']),
                       active_rows=_i(g['voxel_active_rows']))
    pmap = ops.build_point_voxel_map(
        _f(g['points']), vox.coords, vox.active_rows,
        point_active_rows=_i(g['point_active_rows']),
        interpolation=g['interpolation'])
    assert pmap.point_count == g['point_count']
    np.testing.assert_allclose(
        to_np(ops.interpolate_point_features(vox.feats, pmap)), g['sampled'],
        rtol=1e-6)


def test_golden_devoxelize_gradient():
    ops, _ = _ops()
    g = golden('devoxelize_grad')
    pmap = ops.build_point_voxel_map(_f(g['points']), _i(g['coords']),
                                     _i(g['voxel_active_rows']),
                                     interpolation=g['interpolation'])
    feats = _f(g['feats']).requires_grad_(True)
    out = ops.interpolate_point_features(feats, pmap)
    np.testing.assert_allclose(to_np(out), g['features'], rtol=1e-6)
    out.sum().backward()
    np.testing.assert_allclose(to_np(feats.grad), g['grad'], rtol=1e-6)
    with torch.no_grad():
        jvp = ops.interpolate_point_features(_f(g['tangent']), pmap)
    np.testing.assert_allclose(to_np(jvp), g['jvp'], rtol=1e-6)


def test_quantization_contract_errors():
    ops, SparseTensor = _ops()
    m = golden('quantization_errors')['messages']
    points = torch.ones((2, 3), device=DEV)
    feats = torch.ones((2, 1), device=DEV)
    with pytest.raises(ValueError, match=m['points_shape']):
        ops.sparse_quantize(torch.ones((2, 4), device=DEV))
    with pytest.raises(ValueError, match=m['points_dtype']):
        ops.sparse_quantize(torch.ones((2, 3), dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError, match=m['batch_indices']):
        ops.sparse_quantize(points, batch_indices=torch.ones(
            (2,), dtype=torch.int64, device=DEV))
    with pytest.raises(ValueError, match=m['voxel_size']):
        ops.sparse_quantize(points, voxel_size=0.0)
    with pytest.raises(ValueError, match=m['reduction']):
        ops.voxelize(points, feats, reduction='max')
    with pytest.raises(ValueError, match=m['rows']):
        ops.voxelize(points, torch.ones((3, 1), device=DEV))
    with pytest.raises(ValueError, match=m['interpolation']):
        ops.devoxelize(points, SparseTensor(
            _i([[0, 0, 0, 0]]), torch.ones((1, 1), device=DEV)),
            interpolation='cubic')


# ------------------------------------------------------ oracle parity ----


def _points(seed, n, batches=3, scale=4.0):
    rng = np.random.default_rng(seed)
    pts = (rng.standard_normal((n, 3)) * scale).astype(np.float32)
    pts[n // 2] = pts[3]
    pts[n // 3] = pts[11]
    return pts, rng.integers(0, batches, n).astype(np.int32), rng


@pytest.mark.parametrize('size,origin,n,active', [
    (0.5, 0.0, 5000, 5000),
    ((0.3, 0.7, 0.25), (0.1, -0.2, 0.05), 20000, 19000),
    (0.05, 0.0, 300000, 300000),
])
def test_sparse_quantize_matches_oracle(size, origin, n, active):
    ops, _ = _ops()
    pts, b, _ = _points(100, n)
    print(f'quantize n={n} size={size}', flush=True)
    q = ops.sparse_quantize(_f(pts), size, batch_indices=_i(b),
                            origin=origin, active_rows=_i([active]))
    torch.cuda.synchronize()
    ref = O.sparse_quantize(pts, size, batch_indices=b, origin=origin,
                            active_rows=active)
    assert to_np(q.active_rows).tolist() == ref['active_rows'].tolist()
    np.testing.assert_array_equal(to_np(q.coords), ref['coords'])
    np.testing.assert_array_equal(to_np(q.inverse_rows), ref['inverse_rows'])
    np.testing.assert_array_equal(to_np(q.counts), ref['counts'])


def test_sparse_quantize_full_domain():
    """Voxels anywhere in int64 and batches anywhere in int32: deduplicated
    on their int64 value, written as int32 (write_coords); the point map
    over those voxels matches the oracle too."""
    ops, _ = _ops()
    rng = np.random.default_rng(107)
    scales = np.array([1e3, 6.5e4, 1e6, 2.1e9, -3e9, 1e12, -5e15],
                      np.float64)
    n = 7000
    # one magnitude per point (so about half the points have voxels inside
    # int32 that the point map can find), a random sign per axis
    centre = (scales[rng.integers(0, len(scales), (n, 1))]
              * rng.choice([-1.0, 1.0], (n, 3)))
    pts = (centre + rng.standard_normal((n, 3)) * 3.0).astype(np.float32)
    b = rng.choice(np.array([0, 1, 1022, 1023, 5000, -3, 2**31 - 1],
                            np.int64), n).astype(np.int32)
    pts[n // 2] = pts[3]
    b[n // 2] = b[3]
    print('quantize full domain', flush=True)
    q = ops.sparse_quantize(_f(pts), 0.5, batch_indices=_i(b))
    torch.cuda.synchronize()
    ref = O.sparse_quantize(pts, 0.5, batch_indices=b)
    assert to_np(q.active_rows).tolist() == ref['active_rows'].tolist()
    np.testing.assert_array_equal(to_np(q.coords), ref['coords'])
    np.testing.assert_array_equal(to_np(q.inverse_rows), ref['inverse_rows'])
    np.testing.assert_array_equal(to_np(q.counts), ref['counts'])
    n_vox = int(ref['active_rows'][0])
    for interpolation in ('nearest', 'linear'):
        pmap = ops.build_point_voxel_map(_f(pts), q.coords, q.active_rows,
                                         0.5, batch_indices=_i(b),
                                         interpolation=interpolation)
        torch.cuda.synchronize()
        rows, w = O.point_voxel_map(pts, ref['coords'], n_vox, 0.5,
                                    batch_indices=b,
                                    interpolation=interpolation)
        np.testing.assert_array_equal(to_np(pmap.rows), rows)
        np.testing.assert_array_equal(to_np(pmap.weights), w)
        # the probes do find voxels (400 nearest, 3062 linear hits)
        assert (rows >= 0).sum() >= (400 if interpolation == 'nearest' else 3000)


def test_point_map_at_the_packed_block_range_edges():
    """Cells whose lower corner sits on either side of the edge of the
    packed block-key range (lower corner in [-2^18, 2^18 - 2] per axis and
    batch in [0, 1022] take the overlapped home-bucket reads, the others
    the full lookup); every corner voxel present, bit-exact against the
    oracle."""
    ops, _ = _ops()
    edges = np.array([-(1 << 18) - 2, -(1 << 18) - 1, -(1 << 18),
                      -(1 << 18) + 1, (1 << 18) - 3, (1 << 18) - 2,
                      (1 << 18) - 1, (1 << 18)], np.int64)
    cells = []
    for bt in (0, 1022, 1023):
        for v in edges:
            for axis in range(3):
                c = np.array([5, -7, 11], np.int64)
                c[axis] = v
                cells.append((bt, c))
    vox, pts, bs = [], [], []
    rng = np.random.default_rng(113)
    for bt, c in cells:
        for corner in range(8):
            d = np.array([corner & 1, (corner >> 1) & 1, (corner >> 2) & 1])
            vox.append(np.concatenate([[bt], c + d]))
        # a point at c + frac (unit voxels, origin 0) has the cell lower
        # corner c; float32 keeps 1/32 at 2^18
        pts.append(c + rng.uniform(0.1, 0.9, 3))
        bs.append(bt)
    vox = np.unique(np.array(vox, np.int64), axis=0).astype(np.int32)
    pts = np.array(pts, np.float64).astype(np.float32)
    bs = np.array(bs, np.int32)
    n_vox = len(vox)
    print(f'point map range edges voxels={n_vox}', flush=True)
    pmap = ops.build_point_voxel_map(
        _f(pts), _i(vox), _i([n_vox]), 1.0, batch_indices=_i(bs),
        interpolation='linear')
    torch.cuda.synchronize()
    rows, w = O.point_voxel_map(pts, vox, n_vox, 1.0, batch_indices=bs,
                                interpolation='linear')
    np.testing.assert_array_equal(to_np(pmap.rows), rows)
    np.testing.assert_array_equal(to_np(pmap.weights), w)
    assert (rows >= 0).all()


@pytest.mark.parametrize('reduction', ['sum', 'mean'])
def test_voxelize_matches_oracle(reduction):
    ops, _ = _ops()
    pts, b, rng = _points(101, 40000)
    feats = rng.standard_normal((40000, 24)).astype(np.float32)
    q = ops.sparse_quantize(_f(pts), 0.25, batch_indices=_i(b))
    ref_q = O.sparse_quantize(pts, 0.25, batch_indices=b)
    t_feats = _f(feats).requires_grad_(True)
    print(f'voxelize {reduction}', flush=True)
    out = ops.voxelize_with_quantization(q, t_feats, reduction=reduction)
    ref = O.voxelize_features(feats, ref_q['inverse_rows'], ref_q['counts'],
                              reduction)
    np.testing.assert_array_equal(to_np(out.feats), ref)
    cot = rng.standard_normal(ref.shape).astype(np.float32)
    (out.feats * _f(cot)).sum().backward()
    ref_g = O.voxelize_features_grad(cot, ref_q['inverse_rows'],
                                     ref_q['counts'], 40000, reduction)
    np.testing.assert_array_equal(to_np(t_feats.grad), ref_g)
    # a separate, smaller active-row count for the features
    with torch.no_grad():
        part = ops.voxelize_with_quantization(q, _f(feats),
                                              active_rows=_i([30000]),
                                              reduction=reduction)
    ref_p = O.voxelize_features(feats, ref_q['inverse_rows'],
                                ref_q['counts'], reduction,
                                active_rows=30000)
    np.testing.assert_array_equal(to_np(part.feats), ref_p)


@pytest.mark.parametrize('interpolation', ['nearest', 'linear'])
def test_point_voxel_map_and_interpolation_match_oracle(interpolation):
    ops, SparseTensor = _ops()
    pts, b, rng = _points(102, 30000)
    q = ops.sparse_quantize(_f(pts), 0.3, batch_indices=_i(b), origin=0.1)
    n_vox = int(q.active_rows.item())
    query, qb, _ = _points(103, 25000)
    print(f'point map {interpolation} voxels={n_vox}', flush=True)
    pmap = ops.build_point_voxel_map(_f(query), q.coords, q.active_rows, 0.3,
                                     batch_indices=_i(qb),
                                     point_active_rows=_i([24000]),
                                     origin=0.1, interpolation=interpolation)
    torch.cuda.synchronize()
    rows, w = O.point_voxel_map(query, to_np(q.coords), n_vox, 0.3,
                                batch_indices=qb, point_active=24000,
                                origin=0.1, interpolation=interpolation)
    np.testing.assert_array_equal(to_np(pmap.rows), rows)
    np.testing.assert_array_equal(to_np(pmap.weights), w)
    assert (rows >= 0).sum() > 1000        # the probes do find voxels
    vals = rng.standard_normal((q.capacity, 16)).astype(np.float32)
    t_vals = _f(vals).requires_grad_(True)
    out = ops.interpolate_point_features(t_vals, pmap)
    np.testing.assert_array_equal(to_np(out), O.point_features(vals, rows, w))
    g = rng.standard_normal((25000, 16)).astype(np.float32)
    (out * _f(g)).sum().backward()
    np.testing.assert_array_equal(
        to_np(t_vals.grad), O.point_features_grad(g, rows, w, q.capacity))


def test_voxelize_devoxelize_round_trip_at_scale():
    """1M points: every point's nearest voxel centre sample of a
    mean-voxelized constant field returns the constant; counts sum to the
    active points; inverse rows index the voxel holding each point."""
    ops, _ = _ops()
    pts, b, _ = _points(104, 1000000, batches=4, scale=20.0)
    t_pts = _f(pts)
    q = ops.sparse_quantize(t_pts, 0.1, batch_indices=_i(b))
    n = int(q.active_rows.item())
    assert int(q.counts.sum().item()) == 1000000
    vox = to_np(q.coords[:n])
    inv = to_np(q.inverse_rows)
    # binary32 division, as numpy computes it (torch may divide by a
    # scalar through its reciprocal)
    own = np.floor(pts / np.float32(0.1)).astype(np.int64)
    np.testing.assert_array_equal(vox[inv, 1:], own)
    np.testing.assert_array_equal(vox[inv, 0], b)
    ones = torch.ones((1000000, 2), device=DEV)
    out = ops.voxelize_with_quantization(q, ones, reduction='mean')
    assert torch.equal(out.feats[:n], torch.ones((n, 2), device=DEV))
    assert not out.feats[n:].any()
