"""GPU parity of sparse pooling (mlx_lattice/ops/pool.py; native/features/
pooling; CPU routines pooling/cpu/algorithms.cpp:180-331).

Known answers transcribed from the reference's tests/ops/test_pool.py, plus
the CPU oracle's restatement on seeded clouds.  Pooling is float32 only; the
forward and the sum/avg gradients are compared with ``rtol=1e-5`` (the
summation order differs), the max forward and the max gradient exactly.
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


def _sparse(coords, feats, stride=1):
    _, SparseTensor = _ops()
    return SparseTensor(torch.as_tensor(coords, dtype=torch.int32).to(DEV),
                        feats, stride=stride)


def _active(out):
    n = int(out.active_rows.item())
    return to_np(out.coords[:n]).tolist(), to_np(out.feats[:n]).tolist()


@pytest.mark.parametrize('mode', ['sum', 'max', 'avg'])
def test_local_pooling_golden(mode):
    ops, _ = _ops()
    g = golden('pool_local_line')
    x = _sparse(g['coords'], torch.tensor(g['feats'], device=DEV))
    fn = {'sum': ops.sum_pool3d, 'max': ops.max_pool3d,
          'avg': ops.avg_pool3d}[mode]
    coords, feats = _active(fn(x, kernel_size=tuple(g['kernel_size']),
                               stride=g['stride']))
    assert coords == g['coords']
    assert feats == g[mode]


@pytest.mark.parametrize('mode', ['sum', 'max', 'avg'])
def test_pooling_gradients_golden(mode):
    ops, _ = _ops()
    g = golden('pool_grad_line')
    feats = torch.tensor(g['feats'], device=DEV, requires_grad=True)
    out = ops.pool3d(_sparse(g['coords'], feats), mode=mode,
                     kernel_size=tuple(g['kernel_size']), stride=g['stride'])
    out.feats.sum().backward()
    np.testing.assert_allclose(to_np(feats.grad), g[mode], rtol=1e-6)


def test_max_pool_tie_policy_golden():
    ops, _ = _ops()
    g = golden('pool_max_ties')
    feats = torch.tensor(g['feats'], device=DEV, requires_grad=True)
    out = ops.max_pool3d(_sparse(g['coords'], feats),
                         kernel_size=tuple(g['kernel_size']), stride=1)
    assert to_np(out.feats).tolist() == g['pooled']
    out.feats.sum().backward()
    assert to_np(feats.grad).tolist() == g['grad']


def test_strided_pooling_golden():
    ops, _ = _ops()
    g = golden('pool_strided_pointwise')
    x = _sparse(g['coords'], torch.tensor(g['feats'], device=DEV))
    out = ops.sum_pool3d(x, kernel_size=g['kernel_size'], stride=g['stride'])
    coords, feats = _active(out)
    assert coords == g['out_coords']
    assert feats == g['sum']
    assert out.stride == (2, 2, 2)
    assert out.coord_manager is x.coord_manager
    assert out.coord_key != x.coord_key
    assert out.coord_manager.owns(out.coord_key)


def _collate(g):
    ops, _ = _ops()
    coords = [torch.tensor(c, dtype=torch.int32, device=DEV).reshape(-1, 3)
              for c in g['coords']]
    feats = [torch.tensor(f, dtype=torch.float32, device=DEV).reshape(-1, 2)
             for f in g['feats']]
    return ops.sparse_collate(coords, feats)


def test_global_pooling_golden():
    ops, _ = _ops()
    x = _collate(golden('pool_global'))
    g = golden('pool_global')
    assert to_np(ops.global_sum_pool(x)).tolist() == g['sum']
    assert to_np(ops.global_avg_pool(x)).tolist() == g['avg']
    assert to_np(ops.global_max_pool(x)).tolist() == g['max']


def test_global_pooling_empty_batch_golden():
    ops, _ = _ops()
    g = golden('pool_global_empty_batch')
    x = _collate(g)
    assert to_np(ops.global_sum_pool(x)).tolist() == g['sum']
    assert to_np(ops.global_avg_pool(x)).tolist() == g['avg']
    with pytest.raises(ValueError, match=g['max_error']):
        ops.global_max_pool(x)


def test_pool_rejects_invalid_mode_and_dtype():
    ops, _ = _ops()
    x = _sparse([[0, 0, 0, 0]], torch.ones((1, 1), device=DEV))
    with pytest.raises(ValueError, match='mode'):
        ops.pool3d(x, mode='median')
    with pytest.raises(ValueError, match='float32'):
        ops.sum_pool3d(x.astype(torch.float16))


@pytest.mark.parametrize('mode', ['sum', 'max', 'avg'])
@pytest.mark.parametrize('ks,stride', [(3, 1), (2, 2), (3, 2)])
def test_pooling_matches_oracle(mode, ks, stride):
    ops, _ = _ops()
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(ks * 10 + stride)
    coords = sphere_shell_cloud(5000, 128, rng=rng)
    feats_np = rng.standard_normal((len(coords), 24)).astype(np.float32)
    if mode == 'max':
        feats_np = np.round(feats_np * 2) / 2  # plenty of ties
    feats = torch.as_tensor(feats_np, device=DEV).requires_grad_(True)
    x = _sparse(coords, feats)
    print(f'case {mode} k{ks} s{stride} N={len(coords)}', flush=True)
    out = ops.pool3d(x, mode=mode, kernel_size=ks, stride=stride)
    rel = x.coord_manager.kernel_relation(x.coord_key, kernel_size=ks,
                                          stride=stride)
    orel = {name: to_np(t) for name, t in (
        ('in_rows', rel.edges.in_rows), ('out_rows', rel.edges.out_rows),
        ('kernel_ids', rel.edges.kernel_ids), ('counts', rel.counts),
        ('row_offsets', rel.output_csr.row_offsets),
        ('in_row_offsets', rel.input_csr.row_offsets),
        ('in_edge_ids', rel.input_csr.edge_ids))}
    ref = O.pool_features(feats_np, orel, mode)
    got = to_np(out.feats.detach())
    if mode == 'max':
        assert np.array_equal(got, ref)
    else:
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)
    cot_np = rng.standard_normal(got.shape).astype(np.float32)
    (out.feats * torch.as_tensor(cot_np, device=DEV)).sum().backward()
    ref_g = O.pool_grad(cot_np, feats_np, ref, orel, mode)
    if mode == 'max':
        np.testing.assert_allclose(to_np(feats.grad), ref_g, rtol=1e-6,
                                   atol=1e-6)
    else:
        np.testing.assert_allclose(to_np(feats.grad), ref_g, rtol=1e-5,
                                   atol=1e-5)
