"""Edge cases of the widened rows on the GPU: empty and fully inactive
inputs (the reference's capacity semantics: zero active rows give zero
edges, zero-filled or identity-filled capacity rows), single rows, and the
maximum-offset kernels.  Expected values follow from the definitions and
the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _ops():
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor

    return ops, SparseTensor


def _i(a):
    return torch.as_tensor(np.asarray(a, np.int32)).to(DEV)


@pytest.mark.parametrize('ks,stride', [(2, 2), (3, 2)])
def test_transposed_conv_with_no_active_rows(ks, stride):
    ops, SparseTensor = _ops()
    coords = _i([[0, 1, 2, 3], [0, 4, 5, 6]])
    feats = torch.ones((2, 32), dtype=torch.float16, device=DEV)
    x = SparseTensor(coords, feats, stride=stride, active_rows=_i([0]))
    w = torch.ones((32, ks, ks, ks, 32), dtype=torch.float16, device=DEV)
    b = torch.full((32,), 0.5, dtype=torch.float16, device=DEV)
    out = ops.conv_transpose3d(x, w, b, kernel_size=ks, stride=stride)
    torch.cuda.synchronize()
    assert int(out.active_rows.item()) == 0
    assert out.feats.shape == (2 * ks ** 3, 32)
    assert torch.equal(out.feats, b.expand_as(out.feats))
    assert not out.coords.any()


def test_generative_conv_single_row_every_offset():
    """One input row: output row k is coord * stride + offset[k] and holds
    feats @ W[k]."""
    ops, SparseTensor = _ops()
    x = SparseTensor(_i([[2, -3, 5, 7]]),
                     torch.arange(32, dtype=torch.float32,
                                  device=DEV).reshape(1, 32).half(),
                     stride=2)
    rng = np.random.default_rng(3)
    w = torch.as_tensor(rng.standard_normal((64, 2, 2, 2, 32)).astype(
        np.float16)).to(DEV)
    out = ops.generative_conv_transpose3d(x, w, kernel_size=2, stride=2)
    torch.cuda.synchronize()
    offs = O.kernel_offsets(2)
    expect = np.concatenate([np.full((8, 1), 2), np.array([-6, 10, 14]) + offs],
                            1)
    assert to_np(out.coords).tolist() == expect.tolist()
    wm = to_np(w.float()).transpose(1, 2, 3, 4, 0).reshape(8, 32, 64)
    ref = np.einsum('c,kco->ko', to_np(x.feats.float())[0], wm)
    np.testing.assert_allclose(to_np(out.feats.float()), ref, rtol=2e-2,
                               atol=5e-2)


def test_quantize_empty_and_inactive_points():
    ops, _ = _ops()
    q = ops.sparse_quantize(torch.zeros((0, 3), device=DEV))
    assert q.capacity == 0 and to_np(q.active_rows).tolist() == [0]
    pts = torch.rand((5, 3), device=DEV)
    q = ops.sparse_quantize(pts, active_rows=_i([0]))
    assert to_np(q.active_rows).tolist() == [0]
    assert to_np(q.inverse_rows).tolist() == [-1] * 5
    assert not q.counts.any() and not q.coords.any()
    v = ops.voxelize_with_quantization(q, torch.ones((5, 3), device=DEV))
    assert not v.feats.any()
    m = ops.build_point_voxel_map(pts, q.coords, q.active_rows)
    assert (to_np(m.rows) == -1).all() and not m.weights.any()


def test_pooling_and_transposed_relations_on_empty_coords():
    ops, SparseTensor = _ops()
    from mlx_lattice_amd.ops import (build_generative_relation,
                                     build_transposed_kernel_relation)

    empty = torch.zeros((0, 4), dtype=torch.int32, device=DEV)
    for rel in (build_generative_relation(empty),
                build_transposed_kernel_relation(empty, kernel_size=3,
                                                 stride=2)):
        torch.cuda.synchronize()
        assert to_np(rel.counts).tolist() == [0, 0]
        assert to_np(rel.output_csr.row_offsets).tolist() == [0]


def test_transposed_relation_at_large_kernel():
    """K = 5^3 = 125 offsets (more than a 64-bit row of masks): the CSR
    route, bit-exact relation and features against the oracle."""
    ops, SparseTensor = _ops()
    rng = np.random.default_rng(7)
    coords = np.unique(np.concatenate([np.zeros((300, 1), np.int64),
                                       rng.integers(0, 12, (300, 3))], 1),
                       axis=0).astype(np.int32)
    feats = rng.standard_normal((len(coords), 8)).astype(np.float32)
    w = rng.standard_normal((4, 5, 5, 5, 8)).astype(np.float32)
    x = SparseTensor(_i(coords), torch.as_tensor(feats).to(DEV), stride=2)
    out = ops.conv_transpose3d(x, torch.as_tensor(w).to(DEV), kernel_size=5,
                               stride=2)
    torch.cuda.synchronize()
    rel = O.transposed_kernel_relation(coords, kernel_size=5, stride=2)
    n = int(rel['counts'][1])
    assert int(out.active_rows.item()) == n
    np.testing.assert_array_equal(to_np(out.coords[:n]),
                                  rel['out_coords'][:n])
    ref = O.conv_features_fp64(feats.astype(np.float64),
                               O.mapped_weight(w.astype(np.float64)), rel)
    np.testing.assert_allclose(to_np(out.feats), ref, rtol=1e-3, atol=1e-4)
