"""GPU parity of the sparse-convolution gradients (the reference conv
primitive's vjp, native/features/convolution/primitive.cpp:137-176;
cpu/algorithms.cpp:355-481).

Every route is checked against the CPU oracle's restatement of
eval_input_grad_typed / eval_weight_grad_typed on the same relation, plus the
reference's own gradient known answers and torch autograd of the dense conv3d
on a fully occupied box.  Tolerances (written in each test): fp32
``rtol=1e-3``; fp16 / bf16 ``rtol=2e-2`` with an ``atol`` scaled to the
gradient's magnitude, since both sides accumulate in fp32 and round once but
sum the edges in a different order.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import golden, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'


def _imports():
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor

    return ops, SparseTensor


def _sparse(coords, feats, stride=1):
    _, SparseTensor = _imports()
    return SparseTensor(torch.as_tensor(coords, dtype=torch.int32).to(DEV),
                        feats, stride=stride)


# ------------------------------------------------------------ golden ----


@pytest.mark.parametrize('name,mode', [
    ('grad_conv3d_generic_line', 'conv3d'),
    ('grad_subm_conv3d_line', 'subm'),
    ('grad_conv3d_target_line', 'target'),
])
def test_golden_gradients(name, mode):
    ops, _ = _imports()
    g = golden(name)
    feats = torch.tensor(g['feats'], device=DEV, requires_grad=True)
    weight = torch.tensor(g['weight'], device=DEV, requires_grad=True)
    x = _sparse(g['coords'], feats)
    if mode == 'conv3d':
        out = ops.conv3d(x, weight, kernel_size=tuple(g['kernel_size']))
    elif mode == 'subm':
        out = ops.subm_conv3d(x, weight, kernel_size=tuple(g['kernel_size']))
    else:
        target = torch.tensor(g['target'], dtype=torch.int32, device=DEV)
        out = ops.conv3d(x, weight, kernel_size=tuple(g['kernel_size']),
                         coordinates=target)
    out.feats.sum().backward()
    assert to_np(feats.grad).tolist() == g['grad_feats']
    assert to_np(weight.grad).tolist() == g['grad_weight']


# ------------------------------------------------- oracle parity ----


def _cloud(n, grid, seed):
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    return sphere_shell_cloud(n, grid, rng=np.random.default_rng(seed))


def _relation(x, kind, ks, stride):
    mgr = x.coord_manager
    if kind == 'subm':
        return mgr.submanifold_kernel_relation(x.coord_key, kernel_size=ks)
    return mgr.kernel_relation(x.coord_key, kernel_size=ks, stride=stride)


def _oracle_relation(rel):
    """The device relation as numpy, with its grouped CSR views."""
    out = {name: to_np(t) for name, t in (
        ('in_rows', rel.edges.in_rows), ('out_rows', rel.edges.out_rows),
        ('kernel_ids', rel.edges.kernel_ids), ('counts', rel.counts),
        ('row_offsets', rel.output_csr.row_offsets),
        ('in_row_offsets', rel.input_csr.row_offsets),
        ('in_edge_ids', rel.input_csr.edge_ids),
        ('kernel_row_offsets', rel.kernel_csr.row_offsets),
        ('kernel_edge_ids', rel.kernel_csr.edge_ids))}
    return out


def _close(got, ref, rtol, scale_atol):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    atol = scale_atol * max(1.0, float(np.abs(ref).max()))
    err = np.abs(got - ref) - (atol + rtol * np.abs(ref))
    assert (err <= 0).all(), f'max excess {err.max():.3e}'


CASES = [
    # kind, ks, stride, c_in, c_out, dtype, mapped weight
    ('subm', 3, 1, 64, 64, torch.float16, False),      # matrix-core input grad, MFMA weight grad
    ('subm', 3, 1, 32, 128, torch.bfloat16, False),
    ('subm', 3, 1, 64, 32, torch.float16, True),       # mapped (K, C_in, C_out) weight
    ('forward', 2, 2, 64, 128, torch.float16, False),  # k2s2 downsample
    ('subm', 3, 1, 16, 32, torch.float32, False),      # CSR input grad, simple weight grad
    ('subm', 3, 1, 24, 40, torch.float16, False),      # CSR input grad (C_out % 32), MFMA weight grad
    ('forward', 2, 2, 8, 16, torch.float32, True),
    ('subm', 3, 1, 128, 128, torch.float16, False),    # 128 x 128 weight-grad tiles
    ('subm', 3, 1, 96, 136, torch.bfloat16, False),    # ragged 128-channel tiles
    ('subm', 5, 1, 16, 64, torch.float16, False),      # 125 offsets, fewer edges than block slots
]


@pytest.mark.parametrize('kind,ks,stride,c_in,c_out,dtype,mapped', CASES)
def test_gradients_match_oracle(kind, ks, stride, c_in, c_out, dtype, mapped):
    from mlx_lattice_amd.ops._relation_exec import (
        sparse_conv_input_grad_from_relation,
        sparse_conv_weight_grad_from_relation,
    )

    rng = np.random.default_rng(c_in * 7 + c_out)
    coords = _cloud(3000, 128, c_in + c_out)
    n = len(coords)
    feats_np = rng.standard_normal((n, c_in)).astype(np.float32)
    k3 = ks ** 3
    if mapped:
        w_np = (rng.standard_normal((k3, c_in, c_out)) /
                np.sqrt(k3 * c_in)).astype(np.float32)
    else:
        w_np = (rng.standard_normal((c_out, ks, ks, ks, c_in)) /
                np.sqrt(k3 * c_in)).astype(np.float32)
    feats = torch.as_tensor(feats_np).to(DEV, dtype)
    weight = torch.as_tensor(w_np).to(DEV, dtype)
    x = _sparse(coords, feats)
    rel = _relation(x, kind, ks, stride)
    cot_np = rng.standard_normal((n, c_out)).astype(np.float32)
    n_out = int(rel.counts[1].item())
    cot_np[n_out:] = 0.0
    cot = torch.as_tensor(cot_np).to(DEV, dtype)
    print(f'case {kind} k{ks}s{stride} {c_in}->{c_out} {dtype} mapped={mapped}'
          f' N={n} E={int(rel.counts[0].item())}', flush=True)
    gin = sparse_conv_input_grad_from_relation(cot, weight, rel, n)
    gw = sparse_conv_weight_grad_from_relation(feats, cot, weight, rel)
    torch.cuda.synchronize()
    assert gin.shape == (n, c_in) and gin.dtype == dtype
    assert gw.shape == weight.shape and gw.dtype == dtype
    orel = _oracle_relation(rel)
    # The oracle computes in fp32 from the same (rounded) operands.
    f32 = lambda t: to_np(t.float())  # noqa: E731
    ref_in = O.conv_input_grad(f32(cot), f32(weight), orel, n)
    ref_w = O.conv_weight_grad(f32(feats), f32(cot), tuple(weight.shape), orel)
    if dtype == torch.float32:
        _close(to_np(gin), ref_in, 1e-3, 1e-5)
        _close(to_np(gw), ref_w, 1e-3, 1e-5)
    else:
        _close(to_np(gin.float()), ref_in, 2e-2, 1e-2)
        _close(to_np(gw.float()), ref_w, 2e-2, 1e-2)


def test_input_grad_routes_agree():
    """The matrix-core routes (the forward sorted view with the mirrored
    weight, which a submanifold relation takes, and the transposed sorted
    view) and the CSR route of the input gradient give the same numbers to
    fp16 rounding."""
    from mlx_lattice_amd._native import ext
    from mlx_lattice_amd.ops._relation_exec import (
        _transposed_weight,
        sparse_conv_input_grad_from_relation,
    )

    rng = np.random.default_rng(3)
    coords = _cloud(20000, 256, 5)
    n = len(coords)
    feats = torch.as_tensor(rng.standard_normal((n, 64))).to(DEV, torch.float16)
    weight = torch.as_tensor(rng.standard_normal((128, 3, 3, 3, 64)) * 0.02
                             ).to(DEV, torch.float16)
    x = _sparse(coords, feats)
    rel = _relation(x, 'subm', 3, 1)
    cot = torch.as_tensor(rng.standard_normal((n, 128))).to(DEV, torch.float16)
    fast = sparse_conv_input_grad_from_relation(cot, weight, rel, n)
    csr = ext.sparse_conv_input_grad(
        cot, weight, rel.edges.out_rows, rel.edges.kernel_ids, rel.counts,
        rel.input_csr.row_offsets, rel.input_csr.edge_ids, n, 27)
    # the transposed sorted view, which the submanifold route skips
    tview = rel.require_transposed_sorted_implicit_gemm()
    transposed = ext.sparse_conv_features_sorted_implicit_gemm(
        cot, _transposed_weight(weight), tview.sorted_out_in_map,
        tview.sorted_kv_out_in_map, tview.reorder_rows, tview.tile_masks,
        None, None, None, None, None, None, None, None, None, n, 27)
    torch.cuda.synchronize()
    _close(to_np(fast.float()), to_np(csr.float()), 2e-2, 1e-2)
    _close(to_np(transposed.float()), to_np(csr.float()), 2e-2, 1e-2)


def test_weight_grad_is_deterministic():
    from mlx_lattice_amd.ops._relation_exec import (
        sparse_conv_weight_grad_from_relation,
    )

    rng = np.random.default_rng(4)
    coords = _cloud(20000, 256, 6)
    n = len(coords)
    feats = torch.as_tensor(rng.standard_normal((n, 64))).to(DEV, torch.float16)
    weight = torch.zeros((64, 3, 3, 3, 64), dtype=torch.float16, device=DEV)
    x = _sparse(coords, feats)
    rel = _relation(x, 'subm', 3, 1)
    cot = torch.as_tensor(rng.standard_normal((n, 64))).to(DEV, torch.float16)
    a = sparse_conv_weight_grad_from_relation(feats, cot, weight, rel)
    b = sparse_conv_weight_grad_from_relation(feats, cot, weight, rel)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize('ks', [3, 5])
def test_gradients_with_repeated_coordinates(ks):
    """A submanifold relation over repeated coordinates: every copy of a
    coordinate is an output row with the same neighbours (first-row
    lookups), so an input row has several output rows at one offset.  The
    relation build flags it, the input gradient leaves the dense transposed
    map for the input-grouped CSR, and both gradients match the oracle."""
    from mlx_lattice_amd._native import ext
    from mlx_lattice_amd.ops._relation_exec import (
        sparse_conv_input_grad_from_relation,
        sparse_conv_weight_grad_from_relation,
    )

    rng = np.random.default_rng(17 + ks)
    base = _cloud(4000, 128, 23 + ks)
    repeats = base[rng.choice(len(base), 300, replace=False)]
    coords = np.concatenate([base, repeats, repeats[:50]])
    coords = coords[rng.permutation(len(coords))]
    n = len(coords)
    k3 = ks ** 3
    feats = torch.as_tensor(rng.standard_normal((n, 64)).astype(np.float32)
                            ).to(DEV, torch.float16)
    weight = torch.as_tensor((rng.standard_normal((64, ks, ks, ks, 64))
                              / np.sqrt(k3 * 64)).astype(np.float32)
                             ).to(DEV, torch.float16)
    cot = torch.as_tensor(rng.standard_normal((n, 64)).astype(np.float32)
                          ).to(DEV, torch.float16)
    x = _sparse(coords, feats)
    rel = _relation(x, 'subm', ks, 1)
    print(f'repeated coordinates k={ks} N={n}', flush=True)
    assert not rel.transposed_map_exact
    _, _, status = ext.build_transposed_implicit_gemm_map(
        rel.edges.in_rows, rel.edges.out_rows, rel.edges.kernel_ids,
        rel.counts, n, k3)
    gin = sparse_conv_input_grad_from_relation(cot, weight, rel, n)
    gw = sparse_conv_weight_grad_from_relation(feats, cot, weight, rel)
    torch.cuda.synchronize()
    assert int(status.item()) & 4  # LATTICE_STATUS_REPEATED_PAIR
    orel = _oracle_relation(rel)
    f32 = lambda t: to_np(t.float())  # noqa: E731
    _close(to_np(gin.float()),
           O.conv_input_grad(f32(cot), f32(weight), orel, n), 2e-2, 1e-2)
    _close(to_np(gw.float()),
           O.conv_weight_grad(f32(feats), f32(cot), tuple(weight.shape), orel),
           2e-2, 1e-2)
    # the same cloud without the copies keeps the matrix-core route
    y = _sparse(base, feats[:len(base)])
    assert _relation(y, 'subm', ks, 1).transposed_map_exact


def test_weight_grad_with_no_edges():
    """An empty relation gives a zero weight gradient on every route."""
    from mlx_lattice_amd.ops._relation_exec import (
        sparse_conv_weight_grad_from_relation,
    )

    for c_in, c_out, dtype in ((128, 128, torch.float16), (16, 24, torch.float32)):
        feats = torch.zeros((0, c_in), dtype=dtype, device=DEV)
        x = _sparse(np.zeros((0, 4), np.int32), feats)
        rel = _relation(x, 'subm', 3, 1)
        cot = torch.zeros((0, c_out), dtype=dtype, device=DEV)
        weight = torch.ones((c_out, 3, 3, 3, c_in), dtype=dtype, device=DEV)
        print(f'empty weight grad {c_in}->{c_out} {dtype}', flush=True)
        gw = sparse_conv_weight_grad_from_relation(feats, cot, weight, rel)
        torch.cuda.synchronize()
        assert gw.shape == weight.shape
        assert not gw.any()


# ------------------------------------------------------ dense box ----


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_autograd_matches_dense_conv3d_on_a_full_box(dtype):
    """On a fully occupied box subm_conv3d is a zero-padded dense
    cross-correlation, so torch's conv3d autograd gives its gradients."""
    ops, _ = _imports()
    rng = np.random.default_rng(12)
    size, c_in, c_out = 8, 32, 64
    grid = np.stack(np.meshgrid(np.arange(size), np.arange(size),
                                np.arange(size), indexing='ij'), -1)
    coords = np.concatenate([np.zeros((size ** 3, 1), np.int64),
                             grid.reshape(-1, 3)], 1).astype(np.int32)
    coords = coords[rng.permutation(len(coords))]
    feats_np = rng.standard_normal((len(coords), c_in))
    w_np = rng.standard_normal((c_out, 3, 3, 3, c_in)) / np.sqrt(27 * c_in)
    cot_np = rng.standard_normal((len(coords), c_out))
    feats = torch.as_tensor(feats_np).to(DEV, dtype).requires_grad_(True)
    weight = torch.as_tensor(w_np).to(DEV, dtype).requires_grad_(True)
    out = ops.subm_conv3d(_sparse(coords, feats), weight, kernel_size=3)
    (out.feats.float() * torch.as_tensor(cot_np, device=DEV,
                                         dtype=dtype).float()).sum().backward()
    # fp64 dense reference
    xd = torch.zeros((1, c_in, size, size, size), dtype=torch.float64)
    xd[0, :, coords[:, 1], coords[:, 2], coords[:, 3]] = torch.as_tensor(
        feats.detach().double().cpu().numpy()).T
    xd.requires_grad_(True)
    wd = torch.as_tensor(weight.detach().double().cpu().numpy().transpose(
        0, 4, 1, 2, 3).copy()).requires_grad_(True)
    y = torch.nn.functional.conv3d(xd, wd, padding=1)
    gd = torch.zeros_like(y)
    gd[0, :, coords[:, 1], coords[:, 2], coords[:, 3]] = torch.as_tensor(
        torch.as_tensor(cot_np).to(dtype).double().numpy()).T
    (y * gd).sum().backward()
    ref_in = xd.grad[0].numpy()[:, coords[:, 1], coords[:, 2], coords[:, 3]].T
    ref_w = wd.grad.numpy().transpose(0, 2, 3, 4, 1)
    rtol, atol = (1e-3, 1e-5) if dtype == torch.float32 else (2e-2, 1e-2)
    _close(to_np(feats.grad.float()), ref_in, rtol, atol)
    _close(to_np(weight.grad.float()), ref_w, rtol, atol)
