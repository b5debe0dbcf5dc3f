"""GPU parity of the sparse-convolution feature kernels.

Features are held to the north-star tolerances against an fp64 edge-sum
restatement built from the oracle's relation: fp32 ``rtol=1e-3``, fp16 /
bf16 ``rtol=2e-2`` (each with the small ``atol`` written in the test).  The
reference CPU route (per-FMA fp16 rounding for non-square channels,
cpu/algorithms.cpp:180-239) is checked against the same fp64 anchor with its
own, looser bound, because it is less accurate than an fp32-accumulating
kernel.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import golden, to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'
ROOT_LIB = (Path(__file__).resolve().parent.parent / 'mlx-lattice_amd' /
            'mlx_lattice_amd' / 'liblattice_hip.so')
RTOL_F32, ATOL_F32 = 1e-3, 1e-5
RTOL_F16, ATOL_F16 = 2e-2, 1e-2


def _imports():
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor

    return ops, SparseTensor


def _tensor(coords, feats, stride=1):
    _, SparseTensor = _imports()
    return SparseTensor(torch.as_tensor(coords, dtype=torch.int32).to(DEV),
                        torch.as_tensor(feats).to(DEV), stride=stride)


def _w(values, shape, dtype=torch.float32):
    return torch.tensor(values, dtype=dtype, device=DEV).reshape(shape)


def _active(out):
    n = int(out.active_rows.item())
    return to_np(out.coords[:n]), to_np(out.feats[:n].float())


# ------------------------------------------------------------ golden ----


def test_golden_conv3d_generic_and_fp16():
    ops, _ = _imports()
    g = golden('conv3d_generic_line')
    for dtype in (torch.float32, torch.float16):
        x = _tensor(g['coords'], np.array(g['feats'], np.float32))
        x = x.astype(dtype)
        w = _w(g['weight'], g['weight_5d_shape'], dtype)
        out = ops.conv3d(x, w, kernel_size=g['kernel_size'])
        coords, feats = _active(out)
        assert coords.tolist() == g['coords']
        assert feats.tolist() == g['expected']
        assert out.stride == (1, 1, 1)
        assert out.coord_manager is x.coord_manager
        assert out.coord_key != x.coord_key


def test_golden_target_and_pointwise_target():
    ops, SparseTensor = _imports()
    g = golden('conv3d_target_line')
    x = _tensor(g['coords'], np.array(g['feats'], np.float32))
    tgt = SparseTensor(torch.tensor(g['target'], dtype=torch.int32, device=DEV),
                       torch.zeros((2, 1), device=DEV),
                       coord_manager=x.coord_manager)
    out = ops.conv3d(x, _w(g['weight'], g['weight_5d_shape']),
                     kernel_size=g['kernel_size'], coordinates=tgt)
    coords, feats = _active(out)
    assert coords.tolist() == g['target']
    assert feats.tolist() == g['expected']
    assert out.coord_key == tgt.coord_key
    g = golden('conv3d_pointwise_target')
    x = _tensor(g['coords'], np.array(g['feats'], np.float32))
    out = ops.conv3d(x, _w(g['weight_2d'], (1, 1)), kernel_size=1,
                     coordinates=torch.tensor(g['target'], dtype=torch.int32,
                                              device=DEV))
    assert _active(out)[1].tolist() == g['expected']


def test_golden_strided_subm_pointwise():
    ops, _ = _imports()
    g = golden('conv3d_strided_pointwise')
    x = _tensor(g['coords'], np.array(g['feats'], np.float32))
    out = ops.conv3d(x, _w(g['weight'], g['weight_5d_shape']), kernel_size=1,
                     stride=2)
    coords, feats = _active(out)
    assert coords.tolist() == g['out_coords']
    assert feats.tolist() == g['expected']
    assert out.stride == (2, 2, 2)
    g = golden('subm_conv3d_line')
    x = _tensor(g['coords'], np.array(g['feats'], np.float32))
    out = ops.subm_conv3d(x, _w(g['weight'], g['weight_5d_shape']),
                          kernel_size=g['kernel_size'])
    assert to_np(out.feats).tolist() == g['expected']
    assert out.coord_key == x.coord_key
    g = golden('conv3d_pointwise_linear')
    x = _tensor(g['coords'], np.array(g['feats'], np.float32))
    out = ops.conv3d(x, _w(g['weight_2d'], (2, 2)),
                     torch.tensor(g['bias'], device=DEV), kernel_size=1)
    assert to_np(out.feats).tolist() == g['expected']


def test_contract_errors():
    ops, _ = _imports()
    x = _tensor([[0, 0, 0, 0]], np.ones((1, 1), np.float32))
    with pytest.raises(ValueError, match='odd kernel_size'):
        ops.subm_conv3d(x, torch.ones((2, 1, 1), device=DEV), kernel_size=2)
    with pytest.raises(ValueError, match='must divide'):
        ops.conv_transpose3d(x, torch.ones((2, 1, 1), device=DEV), stride=3)
    with pytest.raises(ValueError, match='match feature dtype'):
        ops.subm_conv3d(x, torch.ones((1, 3, 3, 3, 1), device=DEV,
                                      dtype=torch.float16))
    with pytest.raises(ValueError, match='kernel rows'):
        ops.subm_conv3d(x, torch.ones((1, 2, 3, 3, 1), device=DEV))


# --------------------------------------------------- seeded clouds ----


def _reference(coords, feats, weight5d, relation_kwargs):
    rel = O.kernel_relation(coords, **relation_kwargs)
    ref = O.conv_features_fp64(feats.astype(np.float64),
                               O.mapped_weight(weight5d.astype(np.float64)),
                               rel)
    return rel, ref


def _run_conv(coords, feats, weight5d, dtype, *, subm, **geom):
    ops, _ = _imports()
    x = _tensor(coords, feats).astype(dtype)
    w = torch.as_tensor(weight5d).to(device=DEV, dtype=dtype)
    if subm:
        out = ops.subm_conv3d(x, w, **geom)
    else:
        out = ops.conv3d(x, w, **geom)
    torch.cuda.synchronize()
    return out


def _shell(rows, grid, seed):
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(seed)
    return sphere_shell_cloud(rows, grid, rng=rng), rng


def _close(actual, ref, rtol, atol, what):
    err = np.abs(actual - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    assert not bad.any(), (
        f'{what}: {bad.sum()} of {bad.size} outside tolerance; max err '
        f'{err.max():.3e}')


def test_config1_fp32_subm_16_to_32():
    from mlx_lattice_amd.synthetic import config_rng, uniform_grid_cloud

    rng = config_rng(1)
    coords = uniform_grid_cloud(20000, 64, rng=rng)
    feats = rng.standard_normal((len(coords), 16)).astype(np.float32)
    w = (rng.standard_normal((32, 3, 3, 3, 16))
         / np.sqrt(27 * 16)).astype(np.float32)
    out = _run_conv(coords, feats, w, torch.float32, subm=True, kernel_size=3)
    rel, ref = _reference(coords, feats, w, dict(kernel_size=3))
    _close(to_np(out.feats), ref, RTOL_F32, ATOL_F32, 'config1 vs fp64')
    cpu = O.conv_features(feats, w, rel)
    _close(cpu, ref, RTOL_F32, ATOL_F32, 'reference CPU route vs fp64')


@pytest.mark.parametrize('c_in,c_out', [(32, 32), (64, 64), (128, 128),
                                        (64, 128), (128, 256), (32, 16),
                                        (256, 64)])
def test_matrix_core_subm_shapes(c_in, c_out):
    coords, rng = _shell(30000, 160, 11 + c_in + c_out)
    feats = rng.standard_normal((len(coords), c_in)).astype(np.float16)
    w = (rng.standard_normal((c_out, 3, 3, 3, c_in))
         * np.sqrt(2.0 / (27 * c_in))).astype(np.float16)
    print(f'mfma subm c_in={c_in} c_out={c_out}', flush=True)
    out = _run_conv(coords, feats, w, torch.float16, subm=True, kernel_size=3)
    _, ref = _reference(coords, feats, w, dict(kernel_size=3))
    _close(to_np(out.feats.float()), ref, RTOL_F16, ATOL_F16,
           f'fp16 {c_in}->{c_out}')


def test_matrix_core_bf16():
    coords, rng = _shell(20000, 128, 5)
    feats = rng.standard_normal((len(coords), 64)).astype(np.float32)
    w = (rng.standard_normal((64, 3, 3, 3, 64))
         * np.sqrt(2.0 / (27 * 64))).astype(np.float32)
    fb = torch.as_tensor(feats).to(torch.bfloat16).float().numpy()
    wb = torch.as_tensor(w).to(torch.bfloat16).float().numpy()
    out = _run_conv(coords, fb, wb, torch.bfloat16, subm=True, kernel_size=3)
    _, ref = _reference(coords, fb, wb, dict(kernel_size=3))
    _close(to_np(out.feats.float()), ref, 2e-2, 3e-2, 'bf16 64->64')


def test_csr_route_fp16_matches():
    # Channel counts the matrix cores do not tile take the CSR route.
    coords, rng = _shell(8000, 160, 3)
    feats = rng.standard_normal((len(coords), 24)).astype(np.float16)
    w = (rng.standard_normal((40, 3, 3, 3, 24)) * 0.05).astype(np.float16)
    out = _run_conv(coords, feats, w, torch.float16, subm=True, kernel_size=3)
    _, ref = _reference(coords, feats, w, dict(kernel_size=3))
    _close(to_np(out.feats.float()), ref, RTOL_F16, ATOL_F16, 'csr fp16')


def test_config2_downsample_fp16():
    from mlx_lattice_amd.synthetic import config_rng, lidar_cloud

    rng = config_rng(2)
    coords = lidar_cloud(100000, 2, rng=rng)
    feats = rng.standard_normal((len(coords), 64)).astype(np.float16)
    w = (rng.standard_normal((128, 2, 2, 2, 64))
         * np.sqrt(2.0 / (8 * 64))).astype(np.float16)
    out = _run_conv(coords, feats, w, torch.float16, subm=False,
                    kernel_size=2, stride=2)
    rel, ref = _reference(coords, feats, w, dict(kernel_size=2, stride=2))
    n = int(rel['counts'][1])
    assert int(out.active_rows.item()) == n
    np.testing.assert_array_equal(to_np(out.coords[:n]),
                                  rel['out_coords'][:n])
    _close(to_np(out.feats.float())[:n], ref[:n], RTOL_F16, ATOL_F16,
           'config2')


def test_config3_headline_fp16_400k():
    from mlx_lattice_amd.synthetic import config_rng, kaiming_weight, sphere_shell_cloud

    rng = config_rng(3)
    coords = sphere_shell_cloud(400000, 512, rng=rng)
    feats = rng.standard_normal((len(coords), 128)).astype(np.float16)
    w = kaiming_weight((128, 3, 3, 3, 128), rng=rng).astype(np.float16)
    out = _run_conv(coords, feats, w, torch.float16, subm=True, kernel_size=3)
    _, ref = _reference(coords, feats, w, dict(kernel_size=3))
    _close(to_np(out.feats.float()), ref, RTOL_F16, ATOL_F16, 'config3')


def _route_bound(feats, w, rel, n):
    """Bound on |GPU - reference fp16 route| over output rows [0, n): the
    reference route (eval_typed, cpu/algorithms.cpp:180-239) rounds its
    running sum to fp16 after each of the L = edges(row) * c_in steps,
    error <= ((1 + u)^L - 1) * S with u = 2^-11 and S the sum of |f * w|
    over the row's terms; the GPU accumulates in fp32 (the same with
    u = 2^-24) and rounds once to fp16 (<= 2^-11 |exact| <= 2^-11 S)."""
    e = int(rel['row_offsets'][n])
    absw = np.abs(O.mapped_weight(w.astype(np.float64)))
    absf = np.abs(feats.astype(np.float64))
    s = np.zeros((n, absw.shape[2]))
    ins, outs, ks = (rel[k][:e] for k in ('in_rows', 'out_rows', 'kernel_ids'))
    for k in range(absw.shape[0]):
        sel = ks == k
        if sel.any():
            np.add.at(s, outs[sel], absf[ins[sel]] @ absw[k])
    steps = np.diff(rel['row_offsets'][:n + 1]).astype(np.float64)[:, None] * feats.shape[1]
    # (1 + u)^L - 1 bounds the relative growth of L roundings whatever L
    # (gamma_L = L u / (1 - L u) needs L u < 1); fp16 subnormals add up to
    # 2^-25 absolute per rounding.
    grow16 = np.expm1(steps * np.log1p(2.0 ** -11))
    grow32 = np.expm1(steps * np.log1p(2.0 ** -24))
    return grow16 * s + grow32 * s + 2.0 ** -11 * s + (steps + 1) * 2.0 ** -25


@pytest.mark.parametrize('config', [2, 3])
def test_fp16_distance_to_the_reference_route(config):
    """The GPU output against the reference's own fp16 CPU route (per-FMA
    fp16 rounding, the route the reference takes for 64->128 and 128->128)
    on the first output rows of configs 2 and 3: every element within the
    derived rounding bound, the distance reported, and at least 99.9% of
    elements within rtol 2e-2 (atol 1e-2) of the reference route."""
    from mlx_lattice_amd.synthetic import (config_rng, kaiming_weight,
                                           lidar_cloud, sphere_shell_cloud)

    rng = config_rng(config)
    if config == 2:
        coords = lidar_cloud(100000, 2, rng=rng)
        feats = rng.standard_normal((len(coords), 64)).astype(np.float16)
        w = kaiming_weight((128, 2, 2, 2, 64), rng=rng).astype(np.float16)
        geom = dict(kernel_size=2, stride=2)
    else:
        coords = sphere_shell_cloud(400000, 512, rng=rng)
        feats = rng.standard_normal((len(coords), 128)).astype(np.float16)
        w = kaiming_weight((128, 3, 3, 3, 128), rng=rng).astype(np.float16)
        geom = dict(kernel_size=3)
    print(f'fp16 distance to the reference route, config {config}', flush=True)
    out = _run_conv(coords, feats, w, torch.float16, subm=config == 3, **geom)
    rel = O.kernel_relation(coords, **geom)
    n = min(16384, int(rel['counts'][1]))
    sample = dict(rel)
    sample['counts'] = np.array([rel['counts'][0], n], np.int32)
    route = O.conv_features(feats, w, sample, out_capacity=n).astype(np.float64)
    got = to_np(out.feats[:n].float()).astype(np.float64)
    diff = np.abs(got - route)
    assert (diff <= _route_bound(feats, w, rel, n)).all()
    rel_err = diff / np.maximum(np.abs(route), 1e-2)
    within = float((diff <= ATOL_F16 + RTOL_F16 * np.abs(route)).mean())
    print(f'config {config}: {n} rows x {got.shape[1]} channels, max |gpu - '
          f'route| {diff.max():.3e}, max relative {rel_err.max():.3e}, '
          f'within rtol 2e-2: {within:.6f}', flush=True)
    assert within >= 0.999


# ------------------------------------------------------- quantized ----


@pytest.mark.parametrize('bits', [4, 8])
def test_quantized_dequantized_contract(bits):
    from mlx_lattice_amd import dequantize_weight, quantize_weight

    ops, _ = _imports()
    coords, rng = _shell(20000, 128, 21 + bits)
    feats = rng.standard_normal((len(coords), 64)).astype(np.float16)
    w = torch.as_tensor((rng.standard_normal((64, 3, 3, 3, 64))
                         * np.sqrt(2.0 / (27 * 64))).astype(np.float16)).to(DEV)
    q = quantize_weight(w, group_size=32, bits=bits)
    deq = dequantize_weight(q)
    x = _tensor(coords, feats)
    actual = ops.subm_conv3d(x, q, kernel_size=3)
    expected = ops.subm_conv3d(x, deq, kernel_size=3)
    _, ref = _reference(coords, feats.astype(np.float32),
                        to_np(deq.float()), dict(kernel_size=3))
    a = to_np(actual.feats.float())
    _close(a, ref, RTOL_F16, ATOL_F16, f'int{bits} fused vs fp64(dequant)')
    _close(a, to_np(expected.feats.float()), 3e-2, 2e-2,
           f'int{bits} fused vs float route')


@pytest.mark.parametrize('bits', [4, 8])
def test_quantized_csr_route_matches_oracle(bits):
    from mlx_lattice_amd import quantize_weight

    ops, _ = _imports()
    rng = np.random.default_rng(31)
    coords = np.array([[0, i, 0, 0] for i in range(12)], np.int32)
    feats = np.array([[((r + 1) * (c + 3) % 19) / 19 for c in range(16)]
                      for r in range(12)], np.float16)
    w = torch.tensor([((i % 37) - 18) / 37 for i in range(12 * 3 * 16)],
                     dtype=torch.float16, device=DEV).reshape(12, 3, 1, 1, 16)
    q = quantize_weight(w, bits=bits)
    assert q.storage_in_channels == 32 and q.in_channels == 16
    x = _tensor(coords, feats)
    out = ops.conv3d(x, q, kernel_size=(3, 1, 1))
    rel = O.kernel_relation(coords, kernel_size=(3, 1, 1))
    expected = O.quantized_conv_features(
        feats, to_np(q.weight), to_np(q.scales), to_np(q.biases), rel,
        in_channels=16, out_channels=12, storage_in_channels=32,
        group_size=q.group_size, bits=bits)
    _close(to_np(out.feats.float()), expected.astype(np.float32), 2e-3, 2e-3,
           'quantized CSR vs oracle')
    del rng


@pytest.mark.parametrize('dtype,bits,c_in,c_out', [
    (torch.float16, 4, 64, 128),
    (torch.float16, 8, 128, 128),
    (torch.float16, 8, 256, 64),     # four 64-channel chunks per offset
    (torch.float16, 4, 96, 64),      # a 32-channel last chunk
    (torch.bfloat16, 4, 64, 64),
    (torch.bfloat16, 8, 128, 256),   # two column halves
])
def test_quantized_streamed_route(dtype, bits, c_in, c_out):
    """The quantized conv on the streamed matrix-core kernel (packed
    fragments dequantised in registers) against the fp64 sum over the
    dequantised weight, fp16/bf16 features, int4/int8, and through the C ABI
    entry of the route itself (no silent fallback)."""
    import ctypes

    from mlx_lattice_amd import dequantize_weight, quantize_weight
    from mlx_lattice_amd._native import ext

    coords, rng = _shell(20000, 128, 61 + bits + c_in + c_out)
    n = len(coords)
    feats = rng.standard_normal((n, c_in)).astype(np.float32)
    w = torch.as_tensor((rng.standard_normal((c_out, 3, 3, 3, c_in))
                         * np.sqrt(2.0 / (27 * c_in))).astype(np.float32)).to(DEV, dtype)
    q = quantize_weight(w, group_size=32, bits=bits)
    f = torch.as_tensor(feats).to(DEV, dtype)
    print(f'quantized streamed {dtype} int{bits} {c_in}->{c_out}', flush=True)
    c = torch.as_tensor(coords, dtype=torch.int32).to(DEV)
    active = torch.tensor([n], dtype=torch.int32, device=DEV)
    rel = ext.build_submanifold_kernel_relation_with_view(c, active, [3, 3, 3],
                                                          [1, 1, 1])
    reorder, _, kv, tiles = ext.build_sorted_implicit_gemm_view(rel[10], rel[11])
    frag = ext.quantized_weight_fragments(q.weight, q.scales, q.biases, q.in_channels,
                                          q.out_channels, q.storage_in_channels,
                                          q.group_size, q.bits)
    assert frag.numel() > 0
    lib = ctypes.CDLL(str(ROOT_LIB))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.lattice_hip_conv_workspace_bytes.restype = ctypes.c_size_t
    entry = lib.lattice_hip_sparse_quantized_conv_features_sorted_fragments
    entry.argtypes = [I, P, I, I, P, I, I, I, P, P, P, I, P, P, I, P, ctypes.c_size_t, P]
    lib.lattice_hip_last_error.restype = ctypes.c_char_p
    wsb = lib.lattice_hip_conv_workspace_bytes(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    out = torch.empty((n, c_out), dtype=dtype, device=DEV)
    code = 1 if dtype == torch.float16 else 2
    rc = entry(code, f.data_ptr(), n, c_in, frag.data_ptr(), bits, 27, c_out,
               kv.data_ptr(), tiles.data_ptr(), reorder.data_ptr(), n, out.data_ptr(),
               None, 0, ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.lattice_hip_last_error()
    torch.cuda.synchronize()
    fin = to_np(f.float())
    _, ref = _reference(coords, fin, to_np(dequantize_weight(q).float()),
                        dict(kernel_size=3))
    tol = (RTOL_F16, ATOL_F16) if dtype == torch.float16 else (2e-2, 3e-2)
    _close(to_np(out.float()), ref, *tol, f'streamed int{bits} {dtype} {c_in}->{c_out}')
    # the operator path takes the same route
    x = _tensor(coords, feats).astype(dtype)
    ops, _ = _imports()
    ops_out = ops.subm_conv3d(x, q, kernel_size=3)
    _close(to_np(ops_out.feats.float()), ref, *tol, 'operator path')


def test_config4_int4_fused_200k():
    from mlx_lattice_amd import dequantize_weight, quantize_weight
    from mlx_lattice_amd.synthetic import config_rng, kaiming_weight, sphere_shell_cloud

    ops, _ = _imports()
    rng = config_rng(4)
    coords = sphere_shell_cloud(200000, 256, rng=rng)
    w = torch.as_tensor(kaiming_weight((64, 3, 3, 3, 64), rng=rng)).to(
        DEV, torch.float16)
    feats = rng.standard_normal((len(coords), 64)).astype(np.float16)
    q = quantize_weight(w, group_size=32, bits=4)
    x = _tensor(coords, feats)
    out = ops.subm_conv3d(x, q, kernel_size=3)
    _, ref = _reference(coords, feats.astype(np.float32),
                        to_np(dequantize_weight(q).float()), dict(kernel_size=3))
    _close(to_np(out.feats.float()), ref, RTOL_F16, ATOL_F16, 'config4')


def test_tile_schedule_does_not_change_results():
    """The longest-first tile schedule (conv workspace) only reorders row
    tiles: through the C ABI, the matrix-core conv with a workspace and
    with none (tiles in order) must agree bit for bit, for float and packed
    weights, and for C_out 16 (128-channel stages) and 128."""
    import ctypes

    from mlx_lattice_amd import quantize_weight
    from mlx_lattice_amd._native import ext

    lib = ctypes.CDLL(str(ROOT_LIB))
    lib.lattice_hip_conv_workspace_bytes.restype = ctypes.c_size_t
    P, I = ctypes.c_void_p, ctypes.c_int
    sorted_conv = lib.lattice_hip_sparse_conv_features_sorted_implicit_gemm
    sorted_conv.argtypes = [I, P, I, I, P, I, I, I, P, P, P, I, P, P, I, P,
                            ctypes.c_size_t, P]
    quant_conv = lib.lattice_hip_sparse_quantized_conv_features
    quant_conv.argtypes = [I, P, I, I, P, P, P, I, I, I, I, I, P, P, P, I, P,
                           P, P, P, I, P, P, I, P, ctypes.c_size_t, P]
    coords, rng = _shell(30000, 128, 31)
    n = len(coords)
    c = torch.as_tensor(coords, dtype=torch.int32).to(DEV)
    active = torch.tensor([n], dtype=torch.int32, device=DEV)
    rel = ext.build_submanifold_kernel_relation_with_view(c, active, [3, 3, 3],
                                                          [1, 1, 1])
    reorder, _, kv, tiles = ext.build_sorted_implicit_gemm_view(rel[10],
                                                                rel[11])
    stream = torch.cuda.current_stream().cuda_stream
    wsb = lib.lattice_hip_conv_workspace_bytes(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    feats = torch.as_tensor(rng.standard_normal((n, 64)).astype(
        np.float16)).to(DEV)
    for c_out in (16, 128):
        w = torch.as_tensor((rng.standard_normal((c_out, 3, 3, 3, 64)) * 0.05)
                            .astype(np.float16)).to(DEV)
        outs = []
        for workspace, nbytes in ((ws.data_ptr(), wsb), (None, 0)):
            out = torch.empty((n, c_out), dtype=torch.float16, device=DEV)
            assert sorted_conv(1, feats.data_ptr(), n, 64, w.data_ptr(), 1,
                               27, c_out, kv.data_ptr(), tiles.data_ptr(),
                               reorder.data_ptr(), n, out.data_ptr(), None,
                               0, workspace, nbytes, stream) == 0
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), c_out
        q = quantize_weight(w, group_size=32, bits=4)
        qouts = []
        for workspace, nbytes in ((ws.data_ptr(), wsb), (None, 0)):
            out = torch.empty((n, c_out), dtype=torch.float16, device=DEV)
            assert quant_conv(1, feats.data_ptr(), n, 64, q.weight.data_ptr(),
                              q.scales.data_ptr(), q.biases.data_ptr(), 27,
                              c_out, q.storage_in_channels, 32, 4,
                              rel[0].data_ptr(), rel[2].data_ptr(),
                              rel[5].data_ptr(), int(rel[0].shape[0]),
                              rel[3].data_ptr(), kv.data_ptr(),
                              tiles.data_ptr(), reorder.data_ptr(), n,
                              out.data_ptr(), None, 0, workspace, nbytes,
                              stream) == 0
            qouts.append(out)
        torch.cuda.synchronize()
        assert torch.equal(qouts[0], qouts[1]), c_out
        # A tile order computed once (lattice_hip_conv_tile_order) and passed
        # back with LATTICE_CONV_ORDER_READY gives the same bits.
        order = ext.conv_tile_order(tiles, n)
        ready = ctypes.c_size_t(wsb | (1 << 63)).value
        out = torch.empty((n, c_out), dtype=torch.float16, device=DEV)
        assert sorted_conv(1, feats.data_ptr(), n, 64, w.data_ptr(), 1, 27,
                           c_out, kv.data_ptr(), tiles.data_ptr(),
                           reorder.data_ptr(), n, out.data_ptr(), None, 0,
                           order.data_ptr(), ready, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, outs[0]), c_out
    # a workspace that is too small is an argument error, not a fault
    out = torch.empty((n, 128), dtype=torch.float16, device=DEV)
    assert sorted_conv(1, feats.data_ptr(), n, 64, w.data_ptr(), 1, 27, 128,
                       kv.data_ptr(), tiles.data_ptr(), reorder.data_ptr(), n,
                       out.data_ptr(), None, 0, ws.data_ptr(), 4, stream) == 1


# -------------------------------------------------------- fused bias ----


@pytest.mark.parametrize('dtype,c_in,c_out,quant,kind', [
    (torch.float16, 64, 64, None, 'subm'),       # matrix cores
    (torch.bfloat16, 128, 256, None, 'subm'),    # 8-wave C_out = 256 shape
    (torch.float16, 32, 16, None, 'subm'),       # C_out = 16 shape
    (torch.float16, 64, 128, None, 'down'),      # k2s2: bias on rows past the active count too
    (torch.float32, 16, 32, None, 'subm'),       # CSR fp32
    (torch.float16, 24, 40, None, 'subm'),       # CSR fp16
    (torch.float16, 64, 64, 8, 'subm'),          # quantized, matrix cores
    (torch.float16, 4, 32, 8, 'subm'),           # quantized CSR (staged weights)
])
def test_fused_bias_equals_separate_add(dtype, c_in, c_out, quant, kind):
    """The bias added in the conv store equals conv + bias done as a
    separate torch add, bit for bit, on every capacity row."""
    from mlx_lattice_amd import quantize_weight

    ops, _ = _imports()
    coords, rng = _shell(20000, 128, 41 + c_in + c_out)
    feats = rng.standard_normal((len(coords), c_in)).astype(np.float32)
    ks = 3 if kind == 'subm' else 2
    w = (rng.standard_normal((c_out, ks, ks, ks, c_in))
         / np.sqrt(ks ** 3 * c_in)).astype(np.float32)
    b = torch.as_tensor(rng.standard_normal(c_out).astype(np.float32)).to(
        DEV, dtype)
    x = _tensor(coords, feats).astype(dtype)
    wt = torch.as_tensor(w).to(DEV, dtype)
    if quant:
        wt = quantize_weight(wt, group_size=32, bits=quant)
    print(f'fused bias {dtype} {c_in}->{c_out} quant={quant} {kind}',
          flush=True)
    if kind == 'subm':
        fused = ops.subm_conv3d(x, wt, b, kernel_size=3)
        plain = ops.subm_conv3d(x, wt, kernel_size=3)
    else:
        fused = ops.conv3d(x, wt, b, kernel_size=2, stride=2)
        plain = ops.conv3d(x, wt, kernel_size=2, stride=2)
    torch.cuda.synchronize()
    assert torch.equal(fused.feats, plain.feats + b)


# -------------------------------------------------------- fused ReLU ----


def _bits(t):
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16)


@pytest.mark.parametrize('dtype,c_in,c_out,quant,kind', [
    (torch.float16, 64, 128, None, 'subm'),      # matrix cores
    (torch.bfloat16, 128, 256, None, 'subm'),    # C_out = 256: two column halves
    (torch.float16, 32, 16, None, 'subm'),       # C_out = 16 shape
    (torch.float16, 64, 128, None, 'down'),      # k2s2: rows past the active count hold relu(bias)
    (torch.float32, 16, 32, None, 'subm'),       # CSR rows (staged weights)
    (torch.float16, 24, 40, None, 'subm'),       # CSR fp16
    (torch.float16, 64, 64, 8, 'subm'),          # quantized, matrix cores
    (torch.float16, 4, 32, 8, 'subm'),           # quantized CSR (staged weights)
    (torch.float16, 64, 64, None, 'expand'),     # generative transposed: dense expansion
])
def test_fused_relu_equals_separate_relu(dtype, c_in, c_out, quant, kind):
    """activation='relu' in the conv store equals the reference's
    maximum(feats, 0) over the stored conv + bias, bit for bit on every
    capacity row: NaN kept, negatives and -0 stored as +0."""
    from mlx_lattice_amd import quantize_weight
    from mlx_lattice_amd.ops.conv import _activate

    ops, _ = _imports()
    coords, rng = _shell(20000, 128, 57 + c_in + c_out)
    feats = rng.standard_normal((len(coords), c_in)).astype(np.float32)
    feats[::997, 0] = np.nan
    ks = 3 if kind == 'subm' else 2
    w = (rng.standard_normal((c_out, ks, ks, ks, c_in))
         / np.sqrt(ks ** 3 * c_in)).astype(np.float32)
    b = torch.as_tensor(rng.standard_normal(c_out).astype(np.float32)).to(
        DEV, dtype)
    x = _tensor(coords, feats, stride=2 if kind == 'expand' else 1).astype(
        dtype)
    wt = torch.as_tensor(w).to(DEV, dtype)
    if quant:
        wt = quantize_weight(wt, group_size=32, bits=quant)
    print(f'fused relu {dtype} {c_in}->{c_out} quant={quant} {kind}',
          flush=True)
    if kind == 'subm':
        run = lambda **kw: ops.subm_conv3d(x, wt, b, kernel_size=3, **kw)  # noqa: E731
    elif kind == 'down':
        run = lambda **kw: ops.conv3d(x, wt, b, kernel_size=2, stride=2, **kw)  # noqa: E731
    else:
        run = lambda **kw: ops.generative_conv_transpose3d(  # noqa: E731
            x, wt, b, kernel_size=2, stride=2, **kw)
    fused = run(activation='relu').feats
    plain = run().feats
    torch.cuda.synchronize()
    assert torch.equal(_bits(fused), _bits(_activate(plain, True)))
    assert torch.isnan(plain).any() and torch.equal(torch.isnan(fused),
                                                    torch.isnan(plain))
    finite = fused[~torch.isnan(fused)]
    assert not (finite < 0).any() and not torch.signbit(finite).any()


def test_relu_activation_under_autograd():
    """With gradients needed the ReLU runs separately (autograd sees it) and
    gives the fused store's values."""
    ops, _ = _imports()
    coords, rng = _shell(8000, 96, 61)
    feats = rng.standard_normal((len(coords), 32)).astype(np.float32)
    w = torch.as_tensor((rng.standard_normal((32, 3, 3, 3, 32)) * 0.05)
                        .astype(np.float32)).to(DEV, torch.float16)
    b = torch.linspace(-1, 1, 32, device=DEV, dtype=torch.float16)
    x = _tensor(coords, feats).astype(torch.float16)
    with torch.no_grad():
        ref = ops.subm_conv3d(x, w, b, kernel_size=3, activation='relu').feats
    xg = x.replace(feats=x.feats.clone().requires_grad_())
    wg = w.clone().requires_grad_()
    out = ops.subm_conv3d(xg, wg, b, kernel_size=3, activation='relu').feats
    out.float().sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(_bits(out.detach()), _bits(ref))
    assert xg.feats.grad is not None and wg.grad is not None
    with pytest.raises(ValueError, match='activation'):
        ops.subm_conv3d(x, w, b, kernel_size=3, activation='gelu')
