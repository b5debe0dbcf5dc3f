"""Pins the CPU oracle (no GPU needed).

The oracle restates the reference CPU route; these tests check it against
(a) the known answers transcribed from the reference's own tests
(tests/golden/reference_known_answers.json), (b) an independent numpy
brute force written from the relation definition (dict lookups, no shared
code with the C restatement), and (c) closed forms: a dense-box
submanifold conv equals a zero-padded dense 3D cross-correlation, k=2 s=2
gives E = N_in, the grouped views are stable partitions.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import golden
from oracle import oracle as O


# ------------------------------------------------------------ golden ----


def test_kernel_offsets_golden():
    g = golden('kernel_offsets_3x1x1')
    assert O.kernel_offsets(g['kernel_size']).tolist() == g['expected']
    offs = O.kernel_offsets(3)
    assert offs.shape == (27, 3)
    assert offs[13].tolist() == [0, 0, 0]
    assert O.kernel_offsets(2).tolist()[:3] == [[0, 0, 0], [0, 0, 1],
                                                [0, 1, 0]]


def test_forward_relation_golden():
    g = golden('forward_relation_line')
    r = O.kernel_relation(np.array(g['coords']), kernel_size=g['kernel_size'])
    e = g['counts'][0]
    assert r['counts'].tolist() == g['counts']
    assert r['out_coords'].tolist() == g['out_coords']
    for name in ('in_rows', 'out_rows', 'kernel_ids', 'in_edge_ids',
                 'kernel_edge_ids'):
        assert r[name][:e].tolist() == g[name], name
    for name in ('row_offsets', 'in_row_offsets', 'kernel_row_offsets'):
        assert r[name].tolist() == g[name], name


def test_target_relation_golden():
    g = golden('target_relation_line')
    r = O.target_kernel_relation(np.array(g['coords']), np.array(g['target']),
                                 kernel_size=g['kernel_size'])
    e = g['counts'][0]
    assert r['counts'].tolist() == g['counts']
    for name in ('in_rows', 'out_rows', 'kernel_ids'):
        assert r[name][:e].tolist() == g[name]
    assert r['row_offsets'].tolist() == g['row_offsets']


def test_strided_and_downsample_golden():
    g = golden('strided_relation_pointwise')
    r = O.kernel_relation(np.array(g['coords']), kernel_size=1,
                          stride=g['stride'])
    assert r['counts'].tolist() == g['counts']
    assert r['out_coords'][:2].tolist() == g['out_coords']
    assert r['in_rows'][:2].tolist() == g['in_rows']
    for name in ('downsample_first_seen', 'downsample_negative_duplicates'):
        g = golden(name)
        r = O.kernel_relation(np.array(g['coords']), kernel_size=1,
                              stride=g['stride'])
        n = int(r['counts'][1])
        assert r['out_coords'][:n].tolist() == g['out_coords']


def test_implicit_gemm_view_golden():
    g = golden('implicit_gemm_view_forward')
    c = np.array(g['coords'])
    om, rm = O.implicit_gemm_view(c, 3, c, 3,
                                  O.kernel_offsets(g['kernel_size']))
    assert om.tolist() == g['out_in_map']
    assert rm.tolist() == g['row_masks']
    g = golden('implicit_gemm_view_target')
    om, rm = O.implicit_gemm_view(np.array(g['coords']), 3,
                                  np.array(g['target']), 2,
                                  O.kernel_offsets(g['kernel_size']))
    assert om.tolist() == g['out_in_map']
    assert rm.tolist() == g['row_masks']
    g = golden('implicit_gemm_view_33')
    c = np.array(g['coords'])
    om, rm = O.implicit_gemm_view(c, 1, c, 1,
                                  O.kernel_offsets(g['kernel_size']))
    assert list(om.shape) == g['out_in_map_shape']
    assert int(om[0, 16]) == g['out_in_map_16']
    assert rm.tolist() == g['row_masks']


def _conv_golden(name, **kw):
    g = golden(name)
    coords = np.array(g['coords'])
    rel = O.kernel_relation(coords, **kw)
    w = np.array(g['weight'], np.float32).reshape(g['weight_5d_shape'])
    out = O.conv_features(np.array(g['feats'], np.float32), w, rel)
    n = int(rel['counts'][1])
    return out[:n].tolist(), g


def test_conv_golden():
    out, g = _conv_golden('conv3d_generic_line', kernel_size=(3, 1, 1))
    assert out == g['expected']
    out, g = _conv_golden('subm_conv3d_line', kernel_size=(3, 1, 1))
    assert out == g['expected']
    out, g = _conv_golden('conv3d_strided_pointwise', kernel_size=1, stride=2)
    assert out == g['expected']
    g = golden('conv3d_target_line')
    rel = O.target_kernel_relation(np.array(g['coords']),
                                   np.array(g['target']), kernel_size=(3, 1, 1))
    w = np.array(g['weight'], np.float32).reshape(g['weight_5d_shape'])
    out = O.conv_features(np.array(g['feats'], np.float32), w, rel)
    assert out.tolist() == g['expected']


# ------------------------------------------------------- brute force ----


def _floor_div(v, s):
    return v // s  # python floor division


def brute_forward(coords, kernel_size=3, stride=1, padding=0, dilation=1,
                  active=None):
    coords = [tuple(int(v) for v in row) for row in np.asarray(coords)]
    if active is not None:
        coords = coords[:active]
    first = {}
    for i, c in enumerate(coords):
        first.setdefault(c, i)
    s = (stride,) * 3 if isinstance(stride, int) else tuple(stride)
    p = (padding,) * 3 if isinstance(padding, int) else tuple(padding)
    if s == (1, 1, 1) and p == (0, 0, 0):
        outs = list(coords)
    else:
        seen = {}
        for c in coords:
            q = (c[0], _floor_div(c[1], s[0]), _floor_div(c[2], s[1]),
                 _floor_div(c[3], s[2]))
            seen.setdefault(q, len(seen))
        outs = list(seen)
    ks = (kernel_size,) * 3 if isinstance(kernel_size, int) else kernel_size
    d = (dilation,) * 3 if isinstance(dilation, int) else dilation
    axes = [list(range(-(k // 2), k // 2 + 1)) if k % 2 else list(range(k))
            for k in ks]
    offs = [(x * d[0], y * d[1], z * d[2]) for x in axes[0] for y in axes[1]
            for z in axes[2]]
    edges = []
    for o, c in enumerate(outs):
        for k, off in enumerate(offs):
            cand = (c[0], c[1] * s[0] + off[0] - p[0],
                    c[2] * s[1] + off[1] - p[1], c[3] * s[2] + off[2] - p[2])
            if cand in first:
                edges.append((first[cand], o, k))
    return outs, edges, len(offs)


def _check_against_brute(coords, active=None, **geom):
    r = O.kernel_relation(coords, active, **geom)
    outs, edges, k = brute_forward(coords, active=active, **geom)
    e = len(edges)
    assert r['counts'].tolist() == [e, len(outs)]
    assert r['out_coords'][:len(outs)].tolist() == [list(c) for c in outs]
    got = list(zip(r['in_rows'][:e].tolist(), r['out_rows'][:e].tolist(),
                   r['kernel_ids'][:e].tolist()))
    assert got == edges
    # Output CSR: monotone, last = E, rows own contiguous edge ranges.
    ro = r['row_offsets']
    assert (np.diff(ro) >= 0).all() and ro[-1] == e
    outs_arr = np.array([x[1] for x in edges], np.int64)
    for o in range(len(outs)):
        assert (outs_arr[ro[o]:ro[o + 1]] == o).all()
    # Grouped views are stable partitions of the edge ids.
    for key, groups, name in ((0, r['in_row_offsets'].shape[0] - 1, 'in'),
                              (2, k, 'kernel')):
        ids = r[f'{name}_edge_ids'][:e]
        offs = r[f'{name}_row_offsets' if name == 'kernel' else
                 'in_row_offsets']
        expect = sorted(range(e), key=lambda i: (edges[i][key], i))
        assert ids.tolist() == expect
        counts = np.bincount([edges[i][key] for i in range(e)],
                             minlength=groups)
        assert offs.tolist() == [0] + np.cumsum(counts).tolist()


def test_brute_force_small_clouds():
    rng = np.random.default_rng(3)
    coords = rng.integers(-5, 5, size=(300, 4)).astype(np.int32)
    coords[:, 0] = rng.integers(0, 2, size=300)
    _check_against_brute(coords, kernel_size=3)
    _check_against_brute(coords, kernel_size=2, stride=2)
    _check_against_brute(coords, kernel_size=3, stride=2, padding=1)
    _check_against_brute(coords, kernel_size=(3, 1, 5), dilation=(1, 1, 2))
    _check_against_brute(coords, active=120, kernel_size=3)


def test_k2s2_edge_count_closed_form():
    rng = np.random.default_rng(4)
    coords = np.unique(rng.integers(-20, 20, size=(2000, 4)), axis=0)
    coords[:, 0] = 0
    coords = np.unique(coords, axis=0).astype(np.int32)
    r = O.kernel_relation(coords, kernel_size=2, stride=2)
    assert int(r['counts'][0]) == len(coords)


def test_submanifold_self_edge_invariant():
    rng = np.random.default_rng(5)
    coords = np.unique(rng.integers(0, 12, size=(500, 4)), axis=0)
    coords[:, 0] = 0
    coords = np.unique(coords, axis=0).astype(np.int32)
    r = O.kernel_relation(coords, kernel_size=3)
    om, _ = O.implicit_gemm_view(coords, len(coords), coords, len(coords),
                                 O.kernel_offsets(3))
    assert (om[:, 13] == np.arange(len(coords))).all()
    # Symmetry of unique-coordinate submanifold maps: o->i at k  iff
    # i->o at 26-k.
    rows, ks = np.nonzero(om >= 0)
    assert (om[om[rows, ks], 26 - ks] == rows).all()
    assert int(r['counts'][0]) == int((om >= 0).sum())


# ------------------------------------------------------ conv closed form --


def test_dense_box_matches_dense_cross_correlation():
    torch = pytest.importorskip('torch')
    rng = np.random.default_rng(6)
    size = 5
    grid = np.stack(np.meshgrid(np.arange(size), np.arange(size),
                                np.arange(size), indexing='ij'), -1)
    coords = np.concatenate([np.zeros((size ** 3, 1), np.int64),
                             grid.reshape(-1, 3)], 1).astype(np.int32)
    perm = rng.permutation(len(coords))
    coords = coords[perm]
    c_in, c_out = 4, 3
    feats = rng.standard_normal((len(coords), c_in)).astype(np.float32)
    w = rng.standard_normal((c_out, 3, 3, 3, c_in)).astype(np.float32)
    rel = O.kernel_relation(coords, kernel_size=3)
    got = O.conv_features(feats, w, rel)
    dense = np.zeros((1, c_in, size, size, size), np.float64)
    dense[0, :, coords[:, 1], coords[:, 2], coords[:, 3]] = feats
    ref = torch.nn.functional.conv3d(
        torch.from_numpy(dense), torch.from_numpy(
            w.transpose(0, 4, 1, 2, 3).astype(np.float64)), padding=1)
    ref = ref[0].numpy()[:, coords[:, 1], coords[:, 2], coords[:, 3]].T
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    f64 = O.conv_features_fp64(feats, O.mapped_weight(w.astype(np.float64)),
                               rel)
    np.testing.assert_allclose(f64, ref, rtol=1e-12, atol=1e-12)


def test_k2s2_matches_strided_dense_conv():
    torch = pytest.importorskip('torch')
    rng = np.random.default_rng(8)
    size = 6
    grid = np.stack(np.meshgrid(np.arange(size), np.arange(size),
                                np.arange(size), indexing='ij'), -1)
    coords = np.concatenate([np.zeros((size ** 3, 1), np.int64),
                             grid.reshape(-1, 3)], 1).astype(np.int32)
    coords = coords[rng.permutation(len(coords))]
    feats = rng.standard_normal((len(coords), 2)).astype(np.float32)
    w = rng.standard_normal((3, 2, 2, 2, 2)).astype(np.float32)
    rel = O.kernel_relation(coords, kernel_size=2, stride=2)
    got = O.conv_features(feats, w, rel)
    n = int(rel['counts'][1])
    dense = np.zeros((1, 2, size, size, size), np.float64)
    dense[0, :, coords[:, 1], coords[:, 2], coords[:, 3]] = feats
    ref = torch.nn.functional.conv3d(
        torch.from_numpy(dense),
        torch.from_numpy(w.transpose(0, 4, 1, 2, 3).astype(np.float64)),
        stride=2)[0].numpy()
    oc = rel['out_coords'][:n]
    np.testing.assert_allclose(got[:n], ref[:, oc[:, 1], oc[:, 2], oc[:, 3]].T,
                               rtol=1e-5, atol=1e-5)


def per_fma_fp16_bound(feats, weight5d, rel) -> np.ndarray:
    """Elementwise error bound of the reference's per-FMA fp16 route
    (cpu/algorithms.cpp:180-239) against the exact sum: recursive summation
    over L = edges(row) * c_in steps, each rounded to fp16 (u = 2^-11):
    ((1 + u)^L - 1) * sum over the row's terms of |f * w|, plus 2^-25
    absolute per rounding (fp16 subnormal spacing)."""
    u = 2.0 ** -11
    e = int(rel['counts'][0])
    n_out = rel['row_offsets'].shape[0] - 1
    c_in = feats.shape[1]
    absw = np.abs(O.mapped_weight(weight5d.astype(np.float64)))
    absf = np.abs(feats.astype(np.float64))
    s = np.zeros((n_out, absw.shape[2]))
    ins, outs, ks = (rel[k][:e] for k in ('in_rows', 'out_rows', 'kernel_ids'))
    for k in range(absw.shape[0]):
        sel = ks == k
        if sel.any():
            np.add.at(s, outs[sel], absf[ins[sel]] @ absw[k])
    steps = np.diff(rel['row_offsets']).astype(np.float64)[:, None] * c_in
    grow = np.expm1(steps * np.log1p(u))  # (1 + u)^L - 1, valid for any L
    return grow * s + (steps + 1) * 2.0 ** -25


def test_fp16_routes_rounding_semantics():
    rng = np.random.default_rng(9)
    coords = np.unique(rng.integers(0, 10, size=(400, 4)), axis=0)
    coords[:, 0] = 0
    coords = np.unique(coords, axis=0).astype(np.int32)
    rel = O.kernel_relation(coords, kernel_size=3)
    for c_in, c_out, square in ((32, 32, True), (24, 40, False)):
        f = rng.standard_normal((len(coords), c_in)).astype(np.float16)
        w = (rng.standard_normal((c_out, 3, 3, 3, c_in)) * 0.05).astype(
            np.float16)
        got = O.conv_features(f, w, rel).astype(np.float64)
        ref = O.conv_features_fp64(f.astype(np.float64),
                                   O.mapped_weight(w.astype(np.float64)), rel)
        err = np.abs(got - ref).max()
        if square:
            # fp32 accumulator, single rounding (eval_dense_channels_typed).
            assert err <= np.abs(ref).max() * 2 ** -10
        else:
            # per-FMA fp16 rounding (eval_typed) is measurably worse, and
            # bounded by recursive summation with a rounding to fp16 after
            # each of the L = edges(row) * c_in steps:
            # |err| <= ((1 + u)^L - 1) * sum |f * w|, u = 2^-11, plus
            # 2^-25 absolute per rounding in the fp16 subnormal range.
            assert err > 0
            bound = per_fma_fp16_bound(f, w, rel)
            assert (np.abs(got - ref) <= bound).all()


# ---------------------------------------------------------- quantized ----


def test_unpack_formula_on_hand_built_words():
    # int4: word 0x76543210 holds codes 0..7 for ci 0..7 (LSB first).
    words = np.zeros((1, 1, 1), np.uint32)
    words[0, 0, 0] = 0x76543210
    scales = np.full((1, 1, 1), 0.5, np.float32)
    biases = np.full((1, 1, 1), -1.0, np.float32)
    deq = O.dequantize_mapped(words, scales, biases, in_channels=8,
                              out_channels=1, storage_in_channels=8,
                              group_size=8, bits=4)
    assert deq[0, :, 0].tolist() == [0.5 * q - 1.0 for q in range(8)]
    words = np.zeros((1, 2, 1), np.uint32)
    words[0, 0, 0] = 0x04030201
    words[0, 1, 0] = 0xFF000005
    deq = O.dequantize_mapped(words, np.ones((1, 1, 1), np.float32),
                              np.zeros((1, 1, 1), np.float32), in_channels=8,
                              out_channels=1, storage_in_channels=8,
                              group_size=8, bits=8)
    assert deq[0, :, 0].tolist() == [1, 2, 3, 4, 5, 0, 0, 255]


@pytest.mark.parametrize('bits', [4, 8])
def test_quantized_route_matches_dequantized_float_route(bits):
    rng = np.random.default_rng(10 + bits)
    coords = np.unique(rng.integers(0, 8, size=(200, 4)), axis=0)
    coords[:, 0] = 0
    coords = np.unique(coords, axis=0).astype(np.int32)
    rel = O.kernel_relation(coords, kernel_size=3)
    k, c_in, c_out, g = 27, 40, 8, 32
    storage = 64
    words = rng.integers(0, 2 ** 32, size=(k, storage * bits // 32, c_out),
                         dtype=np.uint64).astype(np.uint32)
    scales = (rng.random((k, storage // g, c_out)) * 0.01).astype(np.float32)
    biases = (rng.standard_normal((k, storage // g, c_out)) * 0.01).astype(
        np.float32)
    feats = rng.standard_normal((len(coords), c_in)).astype(np.float32)
    got = O.quantized_conv_features(feats, words, scales, biases, rel,
                                    in_channels=c_in, out_channels=c_out,
                                    storage_in_channels=storage,
                                    group_size=g, bits=bits)
    deq = O.dequantize_mapped(words, scales, biases, in_channels=c_in,
                              out_channels=c_out,
                              storage_in_channels=storage, group_size=g,
                              bits=bits)
    ref = O.conv_features_fp64(feats, deq.astype(np.float64), rel)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------ gradients --


@pytest.mark.parametrize('name', ['grad_conv3d_generic_line',
                                  'grad_subm_conv3d_line',
                                  'grad_conv3d_target_line'])
def test_gradients_golden(name):
    g = golden(name)
    coords = np.array(g['coords'], np.int32)
    feats = np.array(g['feats'], np.float32)
    weight = np.array(g['weight'], np.float32)
    if 'target' in g:
        rel = O.target_kernel_relation(coords, np.array(g['target'], np.int32),
                                       kernel_size=g['kernel_size'])
        n_out = len(g['target'])
    else:
        rel = O.kernel_relation(coords, kernel_size=g['kernel_size'])
        n_out = len(coords)
    cot = np.ones((n_out, weight.shape[0]), np.float32)
    assert O.conv_input_grad(cot, weight, rel, len(coords)).tolist() == \
        g['grad_feats']
    assert O.conv_weight_grad(feats, cot, weight.shape, rel).tolist() == \
        g['grad_weight']


def _box(size, rng):
    grid = np.stack(np.meshgrid(np.arange(size), np.arange(size),
                                np.arange(size), indexing='ij'), -1)
    coords = np.concatenate([np.zeros((size ** 3, 1), np.int64),
                             grid.reshape(-1, 3)], 1).astype(np.int32)
    return coords[rng.permutation(len(coords))]


def test_gradients_match_dense_autograd_on_a_full_box():
    """On a fully occupied box the submanifold conv is a zero-padded dense
    cross-correlation, so its gradients are torch's conv3d gradients."""
    torch = pytest.importorskip('torch')
    rng = np.random.default_rng(9)
    size, c_in, c_out = 5, 3, 4
    coords = _box(size, rng)
    feats = rng.standard_normal((len(coords), c_in))
    w = rng.standard_normal((c_out, 3, 3, 3, c_in))
    cot = rng.standard_normal((len(coords), c_out))
    rel = O.kernel_relation(coords, kernel_size=3)
    x = torch.zeros((1, c_in, size, size, size), dtype=torch.float64,
                    requires_grad=True)
    dense_feats = torch.zeros((1, c_in, size, size, size), dtype=torch.float64)
    dense_feats[0, :, coords[:, 1], coords[:, 2], coords[:, 3]] = \
        torch.from_numpy(feats).T
    x = dense_feats.clone().requires_grad_(True)
    wt = torch.from_numpy(w.transpose(0, 4, 1, 2, 3).copy()).requires_grad_(True)
    y = torch.nn.functional.conv3d(x, wt, padding=1)
    g = torch.zeros_like(y)
    g[0, :, coords[:, 1], coords[:, 2], coords[:, 3]] = torch.from_numpy(cot).T
    (y * g).sum().backward()
    ref_in = x.grad[0].numpy()[:, coords[:, 1], coords[:, 2], coords[:, 3]].T
    ref_w = wt.grad.numpy().transpose(0, 2, 3, 4, 1)
    got_in = O.conv_input_grad(cot.astype(np.float32), w.astype(np.float32),
                               rel, len(coords))
    got_w = O.conv_weight_grad(feats.astype(np.float32),
                               cot.astype(np.float32), w.shape, rel)
    np.testing.assert_allclose(got_in, ref_in, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(got_w, ref_w, rtol=1e-4, atol=1e-4)


def test_gradients_adjoint_to_the_forward_conv():
    """<conv(x, W), g> = <x, input_grad(g)> = <W, weight_grad(x, g)> on a
    strided (k2s2) and a submanifold relation over a sparse cloud."""
    rng = np.random.default_rng(10)
    coords = np.unique(rng.integers(0, 12, (300, 3)), axis=0)
    coords = np.concatenate([rng.integers(0, 2, (len(coords), 1)), coords],
                            1).astype(np.int32)
    coords = coords[rng.permutation(len(coords))]
    for ks, stride in ((3, 1), (2, 2)):
        rel = O.kernel_relation(coords, kernel_size=ks, stride=stride)
        c_in, c_out = 5, 3
        feats = rng.standard_normal((len(coords), c_in)).astype(np.float32)
        w = rng.standard_normal((c_out, ks, ks, ks, c_in)).astype(np.float32)
        n_out = int(rel['counts'][1])
        y = O.conv_features_fp64(feats, O.mapped_weight(w.astype(np.float64)),
                                 rel)
        g = np.zeros((len(coords), c_out), np.float32)
        g[:n_out] = rng.standard_normal((n_out, c_out))
        lhs = float((y * g).sum())
        gin = O.conv_input_grad(g, w, rel, len(coords)).astype(np.float64)
        gw = O.conv_weight_grad(feats, g, w.shape, rel).astype(np.float64)
        assert abs(lhs - float((feats * gin).sum())) < 1e-3 * (1 + abs(lhs))
        assert abs(lhs - float((w * gw).sum())) < 1e-3 * (1 + abs(lhs))
        # the mapped layout gives the same numbers, transposed
        gw_mapped = O.conv_weight_grad(feats, g, (ks ** 3, c_in, c_out), rel)
        np.testing.assert_allclose(O.mapped_weight(gw), gw_mapped, rtol=1e-6)


# -------------------------------------------------------------- pooling --


@pytest.mark.parametrize('mode', ['sum', 'max', 'avg'])
def test_pool_golden(mode):
    g = golden('pool_local_line')
    rel = O.kernel_relation(np.array(g['coords'], np.int32),
                            kernel_size=g['kernel_size'], stride=g['stride'])
    feats = np.array(g['feats'], np.float32)
    assert O.pool_features(feats, rel, mode).tolist() == g[mode]
    gg = golden('pool_grad_line')
    feats = np.array(gg['feats'], np.float32)
    pooled = O.pool_features(feats, rel, mode)
    got = O.pool_grad(np.ones_like(pooled), feats, pooled, rel, mode)
    np.testing.assert_allclose(got, gg[mode], rtol=1e-6)


def test_pool_max_tie_policy_golden():
    g = golden('pool_max_ties')
    rel = O.kernel_relation(np.array(g['coords'], np.int32),
                            kernel_size=g['kernel_size'])
    feats = np.array(g['feats'], np.float32)
    pooled = O.pool_features(feats, rel, 'max')
    assert pooled.tolist() == g['pooled']
    assert O.pool_grad(np.ones_like(pooled), feats, pooled, rel,
                       'max').tolist() == g['grad']


def test_pool_strided_golden():
    g = golden('pool_strided_pointwise')
    rel = O.kernel_relation(np.array(g['coords'], np.int32),
                            kernel_size=g['kernel_size'], stride=g['stride'])
    n = int(rel['counts'][1])
    assert rel['out_coords'][:n].tolist() == g['out_coords']
    got = O.pool_features(np.array(g['feats'], np.float32), rel, 'sum')
    assert got[:n].tolist() == g['sum']


def _pool_brute(coords, feats, ks, stride, mode):
    """Brute force from the definition: every output cell's reduction over
    the active inputs inside its kernel window."""
    rel = O.kernel_relation(coords, kernel_size=ks, stride=stride)
    n_out = int(rel['counts'][1])
    outs = rel['out_coords'][:n_out]
    index = {tuple(c): i for i, c in enumerate(coords.tolist())}
    offs = O.kernel_offsets(ks)
    res = np.full((n_out, feats.shape[1]), -np.inf if mode == 'max' else 0.0)
    deg = np.zeros(n_out)
    for o, (b, x, y, z) in enumerate(outs.tolist()):
        for dx, dy, dz in offs.tolist():
            i = index.get((b, x * stride + dx, y * stride + dy, z * stride + dz))
            if i is None:
                continue
            deg[o] += 1
            res[o] = np.maximum(res[o], feats[i]) if mode == 'max' else res[o] + feats[i]
    if mode == 'avg':
        res /= np.maximum(deg, 1)[:, None]
    return rel, res


@pytest.mark.parametrize('mode', ['sum', 'max', 'avg'])
@pytest.mark.parametrize('ks,stride', [(3, 1), (2, 2)])
def test_pool_brute_force(mode, ks, stride):
    rng = np.random.default_rng(20 + ks)
    coords = np.unique(rng.integers(0, 10, (400, 3)), axis=0)
    coords = np.concatenate([rng.integers(0, 2, (len(coords), 1)), coords],
                            1).astype(np.int32)
    coords = coords[rng.permutation(len(coords))]
    feats = rng.standard_normal((len(coords), 3)).astype(np.float32)
    rel, ref = _pool_brute(coords, feats, ks, stride, mode)
    got = O.pool_features(feats, rel, mode)
    n_out = ref.shape[0]
    np.testing.assert_allclose(got[:n_out], ref, rtol=1e-5, atol=1e-6)
    # gradient of sum/avg pooling is the adjoint of the forward
    if mode != 'max':
        g = rng.standard_normal(got.shape).astype(np.float32)
        g[n_out:] = 0
        gin = O.pool_grad(g, feats, got, rel, mode)
        lhs = float((got[:n_out].astype(np.float64) * g[:n_out]).sum())
        assert abs(lhs - float((feats.astype(np.float64) * gin).sum())) < 1e-3 * (1 + abs(lhs))


# ------------------------------------- transposed / generative relations --


def test_transposed_relation_policy_golden():
    g = golden('transposed_relation_policy')
    gen = O.generative_relation(g['coords'], kernel_size=g['kernel_size'],
                                stride=g['stride'])
    tr = O.transposed_kernel_relation(g['coords'],
                                      kernel_size=g['kernel_size'],
                                      stride=g['stride'])
    assert gen['counts'].tolist() == g['generative_counts']
    n = int(gen['counts'][1])
    assert gen['out_coords'][:n].tolist() == g['generative_out_coords']
    m = int(tr['counts'][1])
    assert tr['out_coords'][:m].tolist() == g['transposed_out_coords']


def test_conv_transpose_contract_golden():
    g = golden('conv_transpose_contract')
    feats = np.asarray(g['feats'], np.float32)
    w = np.asarray(g['weight'], np.float32)
    for rel in (O.generative_relation(g['coords'], kernel_size=g['kernel_size'],
                                      stride=g['stride']),
                O.transposed_kernel_relation(g['coords'],
                                             kernel_size=g['kernel_size'],
                                             stride=g['stride'])):
        n = int(rel['counts'][1])
        assert rel['out_coords'][:n].tolist() == g['out_coords']
        assert O.conv_features(feats, w, rel)[:n].tolist() == g['out_feats']


def test_conv_transpose_gradients_golden():
    g = golden('grad_conv_transpose_line')
    feats = np.asarray(g['feats'], np.float32)
    w = np.asarray(g['weight'], np.float32)
    for rel in (O.generative_relation(g['coords'], kernel_size=g['kernel_size'],
                                      stride=g['stride']),
                O.transposed_kernel_relation(g['coords'],
                                             kernel_size=g['kernel_size'],
                                             stride=g['stride'])):
        n_out = rel['row_offsets'].shape[0] - 1
        cot = np.zeros((n_out, 1), np.float32)
        cot[:int(rel['counts'][1])] = 1.0
        assert O.conv_input_grad(cot, w, rel, 1).tolist() == g['grad_feats']
        assert O.conv_weight_grad(feats, cot, w.shape, rel).tolist() == \
            g['grad_weight']


def test_direct_transposed_rule():
    """relations.cpp:107-127: direct when every stride exceeds the offsets'
    extent on its axis."""
    assert O.direct_transposed(2, 2)
    assert O.direct_transposed(3, 3)
    assert O.direct_transposed((2, 1, 3), (2, 1, 3))
    assert not O.direct_transposed(3, 2)
    assert not O.direct_transposed(2, 1)
    assert not O.direct_transposed(2, 2, dilation=2)


def _cloud_with_duplicates(rng, n, extent, batches=2):
    coords = np.concatenate([rng.integers(0, batches, (n, 1)),
                             rng.integers(-extent, extent, (n, 3))], 1)
    coords[n // 2] = coords[3]          # a repeated coordinate
    return coords.astype(np.int32)


@pytest.mark.parametrize('ks,stride,pad,dil', [
    (2, 2, 0, 1), (3, 2, 0, 1), (3, 1, 1, 1), (2, 1, 0, 1), (3, 2, 1, 2),
    ((2, 3, 1), (2, 1, 1), (0, 1, 0), 1)])
def test_transposed_relation_structure(ks, stride, pad, dil):
    """Every (input row, offset) lands on the output row whose coordinate is
    coord * stride + offset - padding; output rows are the distinct
    candidates in first-seen order (or one per candidate when direct);
    edges run in (out_row, kernel_id, in_row) order; the CSR rows cover
    them."""
    rng = np.random.default_rng(40)
    coords = _cloud_with_duplicates(rng, 300, 6)
    active = 290
    rel = O.transposed_kernel_relation(coords, active, kernel_size=ks,
                                       stride=stride, padding=pad,
                                       dilation=dil)
    offs = O.kernel_offsets(ks, dil).astype(np.int64)
    s = np.asarray(stride if isinstance(stride, tuple) else (stride,) * 3)
    p = np.asarray(pad if isinstance(pad, tuple) else (pad,) * 3)
    K = len(offs)
    E, n_out = int(rel['counts'][0]), int(rel['counts'][1])
    assert E == active * K
    c = coords[:active].astype(np.int64)
    cand = np.concatenate([np.repeat(c[:, :1], K, 0),
                           (c[:, None, 1:] * s + offs[None] - p).reshape(-1, 3)],
                          1)  # candidate j = in*K + k
    oc = rel['out_coords'][:n_out].astype(np.int64)
    if O.direct_transposed(ks, stride, dil):
        assert n_out == active * K
        assert np.array_equal(oc, cand)
    else:
        _, first = np.unique(cand, axis=0, return_index=True)
        assert np.array_equal(oc, cand[np.sort(first)])
    in_r = rel['in_rows'][:E]
    out_r = rel['out_rows'][:E]
    k_r = rel['kernel_ids'][:E]
    assert np.array_equal(oc[out_r], cand[in_r * K + k_r])
    # every (in, k) exactly once
    assert np.array_equal(np.sort(in_r.astype(np.int64) * K + k_r),
                          np.arange(active * K))
    order = np.lexsort((in_r, k_r, out_r))
    assert np.array_equal(order, np.arange(E))
    ro = rel['row_offsets']
    assert ro[0] == 0 and np.all(np.diff(ro) >= 0) and ro[-1] == E
    assert np.array_equal(np.diff(ro[:n_out + 1]),
                          np.bincount(out_r, minlength=n_out))


@pytest.mark.parametrize('ks,stride,pad', [(2, 2, 0), (3, 2, 1), (3, 1, 0)])
def test_transposed_relation_is_the_forward_relation_reversed(ks, stride, pad):
    """A target relation from the transposed relation's output coordinates
    to its input coordinates (same kernel, stride, padding) holds exactly the
    transposed edges with input and output swapped (unique coordinates)."""
    rng = np.random.default_rng(41)
    coords = np.unique(_cloud_with_duplicates(rng, 400, 5), axis=0)
    coords = coords[rng.permutation(len(coords))]
    tr = O.transposed_kernel_relation(coords, kernel_size=ks, stride=stride,
                                      padding=pad)
    n_out = int(tr['counts'][1])
    fwd = O.target_kernel_relation(tr['out_coords'][:n_out], coords,
                                   kernel_size=ks, stride=stride,
                                   padding=pad)
    E = int(tr['counts'][0])
    assert int(fwd['counts'][0]) == E
    a = set(zip(tr['in_rows'][:E].tolist(), tr['out_rows'][:E].tolist(),
                tr['kernel_ids'][:E].tolist()))
    b = set(zip(fwd['out_rows'][:E].tolist(), fwd['in_rows'][:E].tolist(),
                fwd['kernel_ids'][:E].tolist()))
    assert a == b


def test_generative_relation_structure():
    rng = np.random.default_rng(42)
    coords = _cloud_with_duplicates(rng, 200, 6)
    rel = O.generative_relation(coords, 150, kernel_size=3, stride=2)
    offs = O.kernel_offsets(3).astype(np.int64)
    K = len(offs)
    assert rel['counts'].tolist() == [150 * K, 150 * K]
    c = coords[:150].astype(np.int64)
    oc = rel['out_coords'][:150 * K].reshape(150, K, 4)
    assert np.array_equal(oc[..., 0], np.repeat(c[:, :1], K, 1))
    assert np.array_equal(oc[..., 1:], c[:, None, 1:] * 2 + offs[None])
    assert np.array_equal(rel['in_rows'][:150 * K], np.repeat(np.arange(150), K))
    assert np.array_equal(rel['kernel_ids'][:150 * K], np.tile(np.arange(K), 150))
    assert np.array_equal(rel['row_offsets'][:150 * K + 1], np.arange(150 * K + 1))
    assert not rel['out_coords'][150 * K:].any()


@pytest.mark.parametrize('ks,stride,pad,dil', [(2, 2, 0, 1), (3, 1, 0, 1),
                                               (3, 2, 1, 1), (2, 1, 0, 2)])
def test_conv_transpose_matches_dense_conv_transpose3d(ks, stride, pad, dil):
    """On a fully occupied box the sparse transposed conv is torch's dense
    conv_transpose3d, read at coordinate + centre offset + padding."""
    torch = pytest.importorskip('torch')
    rng = np.random.default_rng(43)
    size, c_in, c_out = 4, 3, 2
    coords = _box(size, rng)
    feats = rng.standard_normal((len(coords), c_in)).astype(np.float32)
    w = rng.standard_normal((c_out, ks, ks, ks, c_in)).astype(np.float32)
    rel = O.transposed_kernel_relation(coords, kernel_size=ks, stride=stride,
                                       padding=pad, dilation=dil)
    got = O.conv_features(feats, w, rel)
    n = int(rel['counts'][1])
    dense = np.zeros((1, c_in, size, size, size), np.float64)
    dense[0, :, coords[:, 1], coords[:, 2], coords[:, 3]] = feats
    ref = torch.nn.functional.conv_transpose3d(
        torch.from_numpy(dense),
        torch.from_numpy(w.transpose(4, 0, 1, 2, 3).astype(np.float64)),
        stride=stride, dilation=dil)[0].numpy()
    shift = (ks // 2) * dil if ks % 2 else 0
    idx = rel['out_coords'][:n, 1:] + shift + pad
    assert (idx >= 0).all() and (idx < ref.shape[1]).all()
    np.testing.assert_allclose(got[:n],
                               ref[:, idx[:, 0], idx[:, 1], idx[:, 2]].T,
                               rtol=1e-5, atol=1e-5)
    # the sparse rows are exactly the dense positions that receive an edge
    assert n == len(np.unique(idx, axis=0))
    assert int((np.abs(ref).sum(0) > 0).sum()) == n


# ------------------------------------------------- point quantization ----


def test_sparse_quantize_golden():
    g = golden('quantize_ordered_metadata')
    q = O.sparse_quantize(g['points'], g['voxel_size'],
                          batch_indices=g['batch_indices'])
    n = int(q['active_rows'][0])
    assert q['coords'].shape[0] == g['capacity']
    assert q['active_rows'].tolist() == g['active_rows']
    assert q['coords'][:n].tolist() == g['coords']
    assert q['inverse_rows'].tolist() == g['inverse_rows']
    assert q['counts'][:n].tolist() == g['counts']
    g = golden('quantize_origin_active_rows')
    q = O.sparse_quantize(g['points'], g['voxel_size'], origin=g['origin'],
                          active_rows=g['active_rows_in'][0])
    n = int(q['active_rows'][0])
    assert q['active_rows'].tolist() == g['active_rows']
    assert q['coords'][:n].tolist() == g['coords']
    assert q['inverse_rows'].tolist() == g['inverse_rows']
    assert q['counts'].tolist() == g['counts_full']


def test_voxelize_golden():
    g = golden('voxelize_mean_sum')
    q = O.sparse_quantize(g['points'], g['voxel_size'])
    n = int(q['active_rows'][0])
    assert q['coords'][:n].tolist() == g['coords']
    for mode in ('mean', 'sum'):
        out = O.voxelize_features(g['feats'], q['inverse_rows'], q['counts'],
                                  mode)
        np.testing.assert_allclose(out[:n], g[mode], rtol=1e-6)
    g = golden('voxelize_grad')
    q = O.sparse_quantize(g['points'])
    n = int(q['active_rows'][0])
    out = O.voxelize_features(g['feats'], q['inverse_rows'], q['counts'],
                              g['reduction'])
    np.testing.assert_allclose(out[:n], g['features'], rtol=1e-6)
    cot = np.zeros_like(out)
    cot[:n] = 1.0
    grad = O.voxelize_features_grad(cot, q['inverse_rows'], q['counts'], 3,
                                    g['reduction'])
    np.testing.assert_allclose(grad, g['grad'], rtol=1e-6)
    # the forward is linear, so its jvp is the forward of the tangent
    jvp = O.voxelize_features(g['tangent'], q['inverse_rows'], q['counts'],
                              g['reduction'])
    np.testing.assert_allclose(jvp[:n], g['jvp'], rtol=1e-6)


def test_point_voxel_map_golden():
    g = golden('devoxelize_nearest')
    rows, w = O.point_voxel_map(g['points'], g['coords'],
                                interpolation='nearest')
    np.testing.assert_allclose(O.point_features(g['feats'], rows, w),
                               g['sampled'], rtol=1e-6)
    g = golden('devoxelize_linear')
    rows, w = O.point_voxel_map(g['points'], g['coords'],
                                interpolation='linear')
    np.testing.assert_allclose(O.point_features(g['feats'], rows, w),
                               g['sampled'], rtol=1e-6)
    g = golden('point_voxel_map_reuse')
    rows, w = O.point_voxel_map(g['points'], g['coords'],
                                g['voxel_active_rows'][0],
                                point_active=g['point_active_rows'][0],
                                interpolation=g['interpolation'])
    assert rows.shape[0] == g['point_count']
    np.testing.assert_allclose(O.point_features(g['feats'], rows, w),
                               g['sampled'], rtol=1e-6)
    g = golden('devoxelize_grad')
    rows, w = O.point_voxel_map(g['points'], g['coords'],
                                g['voxel_active_rows'][0],
                                interpolation=g['interpolation'])
    np.testing.assert_allclose(O.point_features(g['feats'], rows, w),
                               g['features'], rtol=1e-6)
    grad = O.point_features_grad(np.ones((1, 1), np.float32), rows, w, 2)
    np.testing.assert_allclose(grad, g['grad'], rtol=1e-6)
    np.testing.assert_allclose(O.point_features(g['tangent'], rows, w),
                               g['jvp'], rtol=1e-6)


def _points(rng, n, batches=2):
    pts = (rng.standard_normal((n, 3)) * 3.0).astype(np.float32)
    pts[n // 2] = pts[3]                          # a repeated point
    return pts, rng.integers(0, batches, n).astype(np.int32)


@pytest.mark.parametrize('size,origin', [(0.5, 0.0), ((0.3, 0.7, 0.25),
                                                      (0.1, -0.2, 0.05))])
def test_sparse_quantize_brute_force(size, origin):
    """numpy restatement from the definition: voxel = floor((p - o) / s) in
    float32, voxels in first-seen order (np.unique's first index, sorted),
    inverse by lookup, counts by bincount."""
    rng = np.random.default_rng(90)
    pts, b = _points(rng, 3000)
    active = 2900
    q = O.sparse_quantize(pts, size, batch_indices=b, origin=origin,
                          active_rows=active)
    s = np.asarray(size if isinstance(size, tuple) else (size,) * 3,
                   np.float32)
    o = np.asarray(origin if isinstance(origin, tuple) else (origin,) * 3,
                   np.float32)
    vox = np.floor((pts[:active] - o) / s).astype(np.int64)
    keys = np.concatenate([b[:active, None].astype(np.int64), vox], 1)
    uniq, first, inv = np.unique(keys, axis=0, return_index=True,
                                 return_inverse=True)
    order = np.argsort(first)
    rank = np.empty_like(order)
    rank[order] = np.arange(len(order))
    n = int(q['active_rows'][0])
    assert n == len(uniq)
    assert np.array_equal(q['coords'][:n], uniq[order])
    assert not q['coords'][n:].any()
    assert np.array_equal(q['inverse_rows'][:active], rank[inv.ravel()])
    assert (q['inverse_rows'][active:] == -1).all()
    assert np.array_equal(q['counts'][:n],
                          np.bincount(rank[inv.ravel()], minlength=n))
    assert not q['counts'][n:].any()


def test_voxelize_brute_force_and_adjoint():
    rng = np.random.default_rng(91)
    pts, b = _points(rng, 2000)
    feats = rng.standard_normal((2000, 5)).astype(np.float32)
    q = O.sparse_quantize(pts, 0.4, batch_indices=b)
    n = int(q['active_rows'][0])
    inv = q['inverse_rows']
    sums = np.zeros((2000, 5))
    np.add.at(sums, inv, feats.astype(np.float64))
    for mode in ('sum', 'mean'):
        out = O.voxelize_features(feats, inv, q['counts'], mode)
        ref = sums if mode == 'sum' else (
            sums / np.maximum(q['counts'], 1)[:, None])
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
        cot = rng.standard_normal(out.shape).astype(np.float32)
        grad = O.voxelize_features_grad(cot, inv, q['counts'], 2000, mode)
        lhs = float((out[:n].astype(np.float64) * cot[:n]).sum())
        rhs = float((feats.astype(np.float64) * grad).sum())
        assert abs(lhs - rhs) <= 1e-4 * max(1.0, abs(lhs))


def test_linear_map_reproduces_affine_fields():
    """Trilinear weights sum to one and reproduce an affine function of the
    voxel centres exactly wherever all eight corners exist."""
    rng = np.random.default_rng(92)
    grid = np.stack(np.meshgrid(np.arange(6), np.arange(6), np.arange(6),
                                indexing='ij'), -1).reshape(-1, 3)
    coords = np.concatenate([np.zeros((len(grid), 1), np.int64), grid], 1
                            ).astype(np.int32)
    coords = coords[rng.permutation(len(coords))]
    size, origin = 0.5, (0.25, -0.5, 1.0)
    pts = (rng.uniform(0.0, 5.0, (400, 3)) * size
           + np.asarray(origin)).astype(np.float32)
    rows, w = O.point_voxel_map(pts, coords, voxel_size=size, origin=origin)
    assert (rows >= 0).all()
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    a = np.array([0.3, -1.2, 2.0])
    field = (coords[:, 1:] @ a + 0.7).astype(np.float32)[:, None]
    got = O.point_features(field, rows, w)[:, 0]
    pos = (pts.astype(np.float64) - origin) / size
    np.testing.assert_allclose(got, pos @ a + 0.7, rtol=1e-5, atol=1e-5)
    # nearest == the voxel containing the rounded position
    rows_n, w_n = O.point_voxel_map(pts, coords, voxel_size=size,
                                    origin=origin, interpolation='nearest')
    near = np.floor(((pts - np.float32(origin)) / np.float32(size))
                    + np.float32(0.5)).astype(np.int64)
    lookup = {tuple(c[1:]): i for i, c in enumerate(coords)}
    expect = [lookup.get(tuple(v), -1) for v in near]
    assert rows_n[:, 0].tolist() == expect
    assert (rows_n[:, 1:] == -1).all() and (w_n[:, 1:] == 0).all()


def test_point_features_adjoint():
    rng = np.random.default_rng(93)
    pts, b = _points(rng, 1500)
    q = O.sparse_quantize(pts, 0.6, batch_indices=b)
    n = int(q['active_rows'][0])
    rows, w = O.point_voxel_map(pts, q['coords'], n, voxel_size=0.6,
                                batch_indices=b)
    vals = rng.standard_normal((len(pts), 3)).astype(np.float32)
    out = O.point_features(vals, rows, w)
    g = rng.standard_normal(out.shape).astype(np.float32)
    grad = O.point_features_grad(g, rows, w, len(pts))
    lhs = float((out.astype(np.float64) * g).sum())
    rhs = float((vals.astype(np.float64) * grad).sum())
    assert abs(lhs - rhs) <= 1e-4 * max(1.0, abs(lhs))
