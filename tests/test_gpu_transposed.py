"""GPU parity of the generative and transposed relations and of the
transposed convolutions over them (relation_build_detail.h:82-196;
relations.cpp:599-670; ops/conv.py:153-214).

Relations are bit-exact against the oracle's restatement (all ten tuple
entries: counts, full row offsets, active edge prefixes, grouped views, the
whole out_coords array including its zero tail).  Features are compared
with the north-star tolerances against an fp64 edge sum over the oracle's
relation: fp32 ``rtol=1e-3, atol=1e-5``; fp16 ``rtol=2e-2, atol=1e-2``.
Gradients follow tests/test_gpu_grad.py's tolerances.
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


def _ops():
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor

    return ops, SparseTensor


def _t(a) -> torch.Tensor:
    return torch.as_tensor(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


def _active(n: int) -> torch.Tensor:
    return torch.tensor([n], dtype=torch.int32, device=DEV)


def _triple(v):
    return list(v) if not isinstance(v, int) else [v, v, v]


def _sparse(coords, feats, stride=1):
    _, SparseTensor = _ops()
    return SparseTensor(torch.as_tensor(coords, dtype=torch.int32).to(DEV),
                        feats, stride=stride)


def _close(actual, ref, rtol, atol, what):
    actual = np.asarray(actual, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(actual - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (f'{what}: {bad.sum()} of {bad.size} outside '
                           f'tolerance; max err {err.max():.3e}')


# ------------------------------------------------------------ golden ----


def test_golden_relation_policy():
    g = golden('transposed_relation_policy')
    c = _t(g['coords'])
    gen = native_relation_dict(_ext().build_generative_relation(
        c, _active(1), g['kernel_size'], g['stride']))
    tr = native_relation_dict(_ext().build_transposed_kernel_relation(
        c, _active(1), g['kernel_size'], g['stride'], [0], [1]))
    assert gen['counts'].tolist() == g['generative_counts']
    assert gen['out_coords'][:2].tolist() == g['generative_out_coords']
    n = int(tr['counts'][1])
    assert tr['out_coords'][:n].tolist() == g['transposed_out_coords']


@pytest.mark.parametrize('op', ['conv_transpose3d',
                                'generative_conv_transpose3d'])
def test_golden_conv_transpose_contract(op):
    ops, _ = _ops()
    g = golden('conv_transpose_contract')
    x = _sparse(g['coords'], torch.tensor(g['feats'], device=DEV),
                stride=tuple(g['in_stride']))
    w = torch.tensor(g['weight'], device=DEV)
    out = getattr(ops, op)(x, w, kernel_size=tuple(g['kernel_size']),
                           stride=tuple(g['stride']))
    n = int(out.active_rows.item())
    assert to_np(out.coords[:n]).tolist() == g['out_coords']
    assert to_np(out.feats[:n]).tolist() == g['out_feats']
    assert out.stride == tuple(g['out_stride'])
    assert out.coord_manager is x.coord_manager


@pytest.mark.parametrize('op', ['conv_transpose3d',
                                'generative_conv_transpose3d'])
def test_golden_conv_transpose_gradients(op):
    ops, _ = _ops()
    g = golden('grad_conv_transpose_line')
    feats = torch.tensor(g['feats'], device=DEV, requires_grad=True)
    w = torch.tensor(g['weight'], device=DEV, requires_grad=True)
    x = _sparse(g['coords'], feats, stride=tuple(g['in_stride']))
    out = getattr(ops, op)(x, w, kernel_size=tuple(g['kernel_size']),
                           stride=tuple(g['stride']))
    out.feats.sum().backward()
    assert to_np(feats.grad).tolist() == g['grad_feats']
    assert to_np(w.grad).tolist() == g['grad_weight']


def test_stride_must_divide():
    ops, _ = _ops()
    g = golden('conv_transpose_stride_error')
    x = _sparse(g['coords'], torch.ones((1, 1), device=DEV))
    with pytest.raises(ValueError, match=g['message']):
        ops.conv_transpose3d(x, torch.ones((1, 2, 2, 2, 1), device=DEV))
    with pytest.raises(ValueError, match=g['message']):
        ops.generative_conv_transpose3d(x, torch.ones((1, 2, 2, 2, 1),
                                                      device=DEV))


# -------------------------------------------------- relation parity ----


def _cloud(rng, n, extent, dup=True):
    coords = np.concatenate([rng.integers(0, 3, (n, 1)),
                             rng.integers(-extent, extent, (n, 3))], 1)
    if dup:
        coords[n // 2] = coords[5]
        coords[n // 3] = coords[7]
    return coords.astype(np.int32)


GEOMS = [
    # kernel, stride, padding, dilation
    (2, 2, 0, 1),          # direct (decoder k2s2)
    (3, 3, 0, 1),          # direct, odd kernel
    ((2, 1, 3), (2, 1, 3), (0, 0, 1), 1),
    (3, 2, 0, 1),          # overlapping candidates
    (3, 1, 1, 1),
    (2, 1, 0, 1),
    (3, 2, 1, 2),          # dilated (neighbourhood of 125 cells: per-candidate lookups)
    (3, 4, 0, 2),          # dilated, offset period 2 (tiled neighbourhood)
    ((5, 3, 2), (3, 2, 1), (1, 0, 0), 1),  # anisotropic 3x3x3 neighbourhood
    (4, 2, 0, 1),          # even kernel, two preimages per axis
    ((3, 2, 2), 1, 0, 1),  # 45-cell neighbourhood, 12 candidates per output row (ranked, not listed)
]


@pytest.mark.parametrize('ks,stride,pad,dil', GEOMS)
@pytest.mark.parametrize('dup', [False, True])
def test_transposed_relation_matches_oracle(ks, stride, pad, dil, dup):
    rng = np.random.default_rng(50 + dup)
    coords = _cloud(rng, 2000, 40, dup)
    active = 1950
    print(f'transposed k{ks} s{stride} p{pad} d{dil} dup={dup}', flush=True)
    native = _ext().build_transposed_kernel_relation(
        _t(coords), _active(active), _triple(ks), _triple(stride),
        _triple(pad), _triple(dil))
    torch.cuda.synchronize()
    got = native_relation_dict(native)
    ref = O.transposed_kernel_relation(coords, active, kernel_size=ks,
                                       stride=stride, padding=pad,
                                       dilation=dil)
    assert_relation_equal(got, ref)
    np.testing.assert_array_equal(got['out_coords'], ref['out_coords'])


@pytest.mark.parametrize('ks,stride,pad,dil', [(3, 2, 0, 1), (4, 2, 0, 1),
                                               (2, 1, 0, 1)])
def test_transposed_relation_wide_coordinates_match_oracle(ks, stride, pad,
                                                           dil):
    """A dense cloud moved to coordinates beyond the packed key range
    (|v| around 2^29, odd and even): the unit-reach resolve looks its blocks
    up by full keys."""
    rng = np.random.default_rng(250)
    coords = _cloud(rng, 2000, 7, True)
    coords[:, 1:] += np.array([(1 << 29) + 1, -(1 << 29), 3 << 20],
                              dtype=np.int32)
    active = len(coords) - 40
    print(f'transposed wide k{ks} s{stride}', flush=True)
    native = _ext().build_transposed_kernel_relation(
        _t(coords), _active(active), _triple(ks), _triple(stride),
        _triple(pad), _triple(dil))
    torch.cuda.synchronize()
    got = native_relation_dict(native)
    ref = O.transposed_kernel_relation(coords, active, kernel_size=ks,
                                       stride=stride, padding=pad,
                                       dilation=dil)
    assert_relation_equal(got, ref)
    np.testing.assert_array_equal(got['out_coords'], ref['out_coords'])


@pytest.mark.parametrize('ks,stride,pad,dil', GEOMS)
@pytest.mark.parametrize('dup', [False, True])
def test_transposed_relation_dense_cloud_matches_oracle(ks, stride, pad, dil,
                                                        dup):
    """The same geometries on a dense cloud (2000 rows in 3 x 14^3 cells):
    most candidates coincide with another row's, so the cross-row part of
    the tiled resolve (representative minimum, member counts, ranks) is
    exercised on nearly every output row."""
    rng = np.random.default_rng(150 + dup)
    coords = _cloud(rng, 2000, 7, dup)
    if not dup:
        coords = np.unique(coords, axis=0)
        coords = coords[rng.permutation(len(coords))]
    active = len(coords) - 40
    print(f'transposed dense k{ks} s{stride} p{pad} d{dil} dup={dup}',
          flush=True)
    native = _ext().build_transposed_kernel_relation(
        _t(coords), _active(active), _triple(ks), _triple(stride),
        _triple(pad), _triple(dil))
    torch.cuda.synchronize()
    got = native_relation_dict(native)
    ref = O.transposed_kernel_relation(coords, active, kernel_size=ks,
                                       stride=stride, padding=pad,
                                       dilation=dil)
    assert_relation_equal(got, ref)
    np.testing.assert_array_equal(got['out_coords'], ref['out_coords'])
    # dense: candidates of different rows share output rows (except in the
    # direct layout, one output row per candidate)
    k3, s3, d3 = _triple(ks), _triple(stride), _triple(dil)
    direct = all(s3[a] > (k3[a] - 1) * d3[a] for a in range(3))
    assert direct or int(ref['counts'][1]) < int(ref['counts'][0])


@pytest.mark.parametrize('ks,stride,pad,dil', [(2, 2, 0, 1), (3, 2, 0, 1),
                                                (3, 1, 1, 1), (3, 4, 0, 2)])
@pytest.mark.parametrize('unique', [False, True])
def test_transposed_relation_full_int32_domain(ks, stride, pad, dil, unique):
    """Inputs anywhere in int32; candidates coord * stride + offset leave
    int32 and are written as int32 (low 32 bits), as the reference's
    write_coords does with its int64 candidates."""
    coords = extreme_cloud(81)
    if unique:
        coords = np.unique(coords, axis=0)
        coords = coords[np.random.default_rng(82).permutation(len(coords))]
    active = len(coords) - 9
    print(f'transposed extreme k{ks} s{stride} p{pad} d{dil} unique={unique}',
          flush=True)
    native = _ext().build_transposed_kernel_relation(
        _t(coords), _active(active), _triple(ks), _triple(stride),
        _triple(pad), _triple(dil))
    torch.cuda.synchronize()
    got = native_relation_dict(native)
    ref = O.transposed_kernel_relation(coords, active, kernel_size=ks,
                                       stride=stride, padding=pad,
                                       dilation=dil)
    assert_relation_equal(got, ref)
    np.testing.assert_array_equal(got['out_coords'], ref['out_coords'])


@pytest.mark.parametrize('ks,stride', [(2, 2), (3, 2), ((1, 2, 3), 1)])
def test_generative_relation_matches_oracle(ks, stride):
    rng = np.random.default_rng(60)
    coords = _cloud(rng, 1500, 50)
    print(f'generative k{ks} s{stride}', flush=True)
    native = _ext().build_generative_relation(_t(coords), _active(1400),
                                              _triple(ks), _triple(stride))
    torch.cuda.synchronize()
    got = native_relation_dict(native)
    ref = O.generative_relation(coords, 1400, kernel_size=ks, stride=stride)
    assert_relation_equal(got, ref)
    np.testing.assert_array_equal(got['out_coords'], ref['out_coords'])


def test_empty_and_repeated_edge_flag():
    from mlx_lattice_amd.ops import build_transposed_kernel_relation

    rng = np.random.default_rng(61)
    coords = _cloud(rng, 500, 20, dup=False)
    coords = np.unique(coords, axis=0)
    rel = build_transposed_kernel_relation(_t(coords), kernel_size=3,
                                           stride=2)
    assert rel.dense_map_exact and rel.repeated_edges is False
    dup = np.concatenate([coords, coords[:1]])
    rel = build_transposed_kernel_relation(_t(dup), kernel_size=3, stride=2)
    assert not rel.dense_map_exact and rel.repeated_edges is True
    rel = build_transposed_kernel_relation(_t(dup), kernel_size=2, stride=2)
    assert not rel.repeated_edges   # direct: one output row per candidate
    empty = build_transposed_kernel_relation(
        _t(np.zeros((4, 4), np.int32)), _active(0), kernel_size=3, stride=2)
    assert to_np(empty.counts).tolist() == [0, 0]
    assert to_np(empty.output_csr.row_offsets).tolist() == [0] * (4 * 27 + 1)


def test_decoder_scale_relation_properties():
    """At a decoder's real size (400k rows, k3s2 overlapping and k2s2
    direct) against the oracle, bit for bit."""
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    coords = sphere_shell_cloud(400000, 512, rng=np.random.default_rng(62))
    for ks, stride in ((2, 2), (3, 2)):
        print(f'decoder k{ks} s{stride}', flush=True)
        native = _ext().build_transposed_kernel_relation(
            _t(coords), _active(len(coords)), _triple(ks), _triple(stride),
            [0, 0, 0], [1, 1, 1])
        torch.cuda.synchronize()
        got = native_relation_dict(native)
        ref = O.transposed_kernel_relation(coords, kernel_size=ks,
                                           stride=stride)
        assert_relation_equal(got, ref)


# ------------------------------------------------------ conv parity ----


def _fp64_conv(feats, w5d, rel):
    return O.conv_features_fp64(feats.astype(np.float64),
                                O.mapped_weight(w5d.astype(np.float64)), rel)


CONV_CASES = [
    # op, kernel, stride, c_in, c_out, dtype, repeated coordinate
    ('conv_transpose3d', 2, 2, 128, 128, torch.float16, False),   # direct MFMA
    ('conv_transpose3d', 3, 2, 64, 64, torch.float16, False),     # overlap MFMA
    ('conv_transpose3d', 3, 2, 64, 32, torch.float16, True),      # CSR (repeats)
    ('conv_transpose3d', 2, 2, 16, 32, torch.float32, False),     # CSR fp32
    ('generative_conv_transpose3d', 2, 2, 64, 128, torch.bfloat16, False),
    ('generative_conv_transpose3d', 3, 2, 32, 64, torch.float16, True),
]


@pytest.mark.parametrize('op,ks,stride,c_in,c_out,dtype,dup', CONV_CASES)
def test_conv_transpose_matches_oracle(op, ks, stride, c_in, c_out, dtype,
                                       dup):
    ops, _ = _ops()
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(c_in + c_out + ks)
    coords = sphere_shell_cloud(6000, 128, rng=rng)
    if dup:
        coords = np.concatenate([coords, coords[:3]])
    n = len(coords)
    feats_np = rng.standard_normal((n, c_in)).astype(np.float32)
    w_np = (rng.standard_normal((c_out, ks, ks, ks, c_in))
            / np.sqrt(ks ** 3 * c_in)).astype(np.float32)
    feats = torch.as_tensor(feats_np).to(DEV, dtype)
    w = torch.as_tensor(w_np).to(DEV, dtype)
    x = _sparse(coords, feats, stride=stride)
    print(f'{op} k{ks}s{stride} {c_in}->{c_out} {dtype} dup={dup}',
          flush=True)
    out = getattr(ops, op)(x, w, kernel_size=ks, stride=stride)
    torch.cuda.synchronize()
    if op == 'conv_transpose3d':
        rel = O.transposed_kernel_relation(coords, kernel_size=ks,
                                           stride=stride)
    else:
        rel = O.generative_relation(coords, kernel_size=ks, stride=stride)
    n_out = int(rel['counts'][1])
    assert int(out.active_rows.item()) == n_out
    np.testing.assert_array_equal(to_np(out.coords[:n_out]),
                                  rel['out_coords'][:n_out])
    assert out.stride == (1, 1, 1)
    f32 = lambda t: to_np(t.float())  # noqa: E731
    ref = _fp64_conv(f32(feats), f32(w), rel)
    rtol, atol = (1e-3, 1e-5) if dtype == torch.float32 else (2e-2, 1e-2)
    _close(f32(out.feats), ref, rtol, atol, f'{op} features')
    # the route taken: matrix cores unless fp32 or a repeated coordinate
    relation = (x.coord_manager.transposed_kernel_relation(
        x.coord_key, kernel_size=ks, stride=stride)
        if op == 'conv_transpose3d' else
        x.coord_manager.generative_relation(x.coord_key, kernel_size=ks,
                                            stride=stride))
    direct = op == 'generative_conv_transpose3d' or O.direct_transposed(
        ks, stride)
    expand = (direct and dtype != torch.float32
              and c_in in (32, 64, 128, 256) and c_out in (32, 64, 128, 256)
              and c_in * c_out <= 16384)
    mfma = (dtype != torch.float32 and not expand
            and (op != 'conv_transpose3d' or not dup))
    assert relation.direct_expansion == direct
    assert (relation.sorted_implicit_gemm is not None) == mfma


@pytest.mark.parametrize('op,ks,stride,c_in,c_out,dtype', [
    ('conv_transpose3d', 2, 2, 64, 64, torch.float16),
    ('conv_transpose3d', 3, 2, 32, 64, torch.float16),
    ('conv_transpose3d', 3, 2, 16, 8, torch.float32),
    ('generative_conv_transpose3d', 2, 2, 32, 32, torch.bfloat16),
])
def test_conv_transpose_gradients_match_oracle(op, ks, stride, c_in, c_out,
                                               dtype):
    ops, _ = _ops()
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(70 + c_in)
    coords = sphere_shell_cloud(4000, 128, rng=rng)
    n = len(coords)
    feats_np = rng.standard_normal((n, c_in)).astype(np.float32)
    w_np = (rng.standard_normal((c_out, ks, ks, ks, c_in))
            / np.sqrt(ks ** 3 * c_in)).astype(np.float32)
    feats = torch.as_tensor(feats_np).to(DEV, dtype).requires_grad_(True)
    w = torch.as_tensor(w_np).to(DEV, dtype).requires_grad_(True)
    x = _sparse(coords, feats, stride=stride)
    print(f'grad {op} k{ks}s{stride} {c_in}->{c_out} {dtype}', flush=True)
    out = getattr(ops, op)(x, w, kernel_size=ks, stride=stride)
    cot_np = rng.standard_normal(tuple(out.feats.shape)).astype(np.float32)
    n_out = int(out.active_rows.item())
    cot_np[n_out:] = 0.0
    cot = torch.as_tensor(cot_np).to(DEV, dtype)
    (out.feats.float() * cot.float()).sum().backward()
    torch.cuda.synchronize()
    if op == 'conv_transpose3d':
        rel = O.transposed_kernel_relation(coords, kernel_size=ks,
                                           stride=stride)
    else:
        rel = O.generative_relation(coords, kernel_size=ks, stride=stride)
    f32 = lambda t: to_np(t.detach().float())  # noqa: E731
    ref_in = O.conv_input_grad(f32(cot), f32(w), rel, n)
    ref_w = O.conv_weight_grad(f32(feats), f32(cot), tuple(w.shape), rel)
    rtol, atol = (1e-3, 1e-5) if dtype == torch.float32 else (2e-2, 1e-2)
    scale_in = max(1.0, float(np.abs(ref_in).max()))
    scale_w = max(1.0, float(np.abs(ref_w).max()))
    _close(f32(feats.grad), ref_in, rtol, atol * scale_in, 'input grad')
    _close(f32(w.grad), ref_w, rtol, atol * scale_w, 'weight grad')


def test_modules_and_quantized_transpose():
    """ConvTranspose3d / GenerativeConvTranspose3d modules and their int8
    versions, against the float op on the dequantized weight."""
    from mlx_lattice_amd import nn as lnn
    from mlx_lattice_amd.core import dequantize_weight
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    ops, _ = _ops()
    torch.manual_seed(0)
    coords = sphere_shell_cloud(3000, 96, rng=np.random.default_rng(80))
    feats = torch.randn((len(coords), 64), device=DEV, dtype=torch.float16)
    x = _sparse(coords, feats, stride=2)
    for cls in (lnn.ConvTranspose3d, lnn.GenerativeConvTranspose3d):
        m = cls(64, 32, kernel_size=2, stride=2, device=DEV,
                dtype=torch.float16)
        out = m(x)
        assert out.stride == (1, 1, 1)
        q = m.to_quantized(group_size=32, bits=8)
        qout = q(x)
        dq = dequantize_weight(q._quantized_weight()).to(DEV, torch.float16)
        ref = (ops.conv_transpose3d(x, dq, m.bias, kernel_size=2, stride=2)
               if cls is lnn.ConvTranspose3d else
               ops.generative_conv_transpose3d(x, dq, m.bias, kernel_size=2,
                                               stride=2))
        torch.cuda.synchronize()
        n = int(ref.active_rows.item())
        _close(to_np(qout.feats[:n].float()), to_np(ref.feats[:n].float()),
               2e-2, 1e-2, f'{cls.__name__} int8')


@pytest.mark.parametrize('c_in,c_out,dtype', [
    (128, 128, torch.float16), (64, 256, torch.bfloat16), (32, 32, torch.float16),
    (256, 64, torch.float16)])
def test_expansion_conv_matches_sorted_route_and_oracle(c_in, c_out, dtype):
    """The dense expansion kernel of a direct relation against the generic
    matrix-core route over the same relation (same fp32 MFMA sums) and the
    oracle; rows past the active count hold the bias."""
    ops, _ = _ops()
    from mlx_lattice_amd.ops._relation_exec import (
        sparse_conv_features_sorted_from_relation,
    )
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(90 + c_in + c_out)
    coords = sphere_shell_cloud(5000, 128, rng=rng)
    n = len(coords)
    active = n - 37
    feats_np = rng.standard_normal((n, c_in)).astype(np.float32)
    w_np = (rng.standard_normal((c_out, 2, 2, 2, c_in))
            / np.sqrt(8 * c_in)).astype(np.float32)
    feats = torch.as_tensor(feats_np).to(DEV, dtype)
    w = torch.as_tensor(w_np).to(DEV, dtype)
    bias = torch.as_tensor(rng.standard_normal(c_out).astype(np.float32)
                           ).to(DEV, dtype)
    from mlx_lattice_amd import SparseTensor
    x = SparseTensor(_t(coords), feats, stride=2, active_rows=_active(active))
    print(f'expand {c_in}->{c_out} {dtype}', flush=True)
    out = ops.conv_transpose3d(x, w, bias, kernel_size=2, stride=2)
    rel = x.coord_manager.transposed_kernel_relation(x.coord_key,
                                                     kernel_size=2, stride=2)
    assert rel.direct_expansion and rel.sorted_implicit_gemm is None
    generic = sparse_conv_features_sorted_from_relation(feats, w, rel)
    torch.cuda.synchronize()
    assert torch.equal(out.feats, generic + bias)
    ref_rel = O.transposed_kernel_relation(coords, active, kernel_size=2,
                                           stride=2)
    f32 = lambda t: to_np(t.float())  # noqa: E731
    ref = O.conv_features_fp64(f32(feats).astype(np.float64),
                               O.mapped_weight(f32(w).astype(np.float64)),
                               ref_rel)
    _close(f32(generic), ref, 2e-2, 1e-2, 'expansion vs oracle')
    assert torch.equal(out.feats[active * 8:],
                       bias.expand(n * 8 - active * 8, c_out))
