"""The dense-map conv for few input channels (C_in 4 or 8, e.g. an
encoder's 4-channel stem): a row's whole neighbourhood, 27 offsets x C_in
channels, contracted on the matrix cores over the relation's dense map
(lattice_hip_sparse_conv_features_dense_map and its quantized twin).

Checked through the C ABI entries themselves (no silent fallback) against
the fp64 edge sum of the oracle (the float and the dequantised weight), and
against the CSR route of the same relation; the operator path must take
the same route (its output equals the entry's bit for bit); rows past the
relation's active count hold the bias alone."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'
ROOT_LIB = (Path(__file__).resolve().parent.parent / 'mlx-lattice_amd' /
            'mlx_lattice_amd' / 'liblattice_hip.so')
RTOL_F16, ATOL_F16 = 2e-2, 1e-2
RTOL_BF16, ATOL_BF16 = 2e-2, 3e-2


def _lib():
    lib = ctypes.CDLL(str(ROOT_LIB))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.lattice_hip_sparse_conv_features_dense_map.argtypes = [
        I, P, I, I, P, I, I, I, P, P, I, P, P, I, P]
    lib.lattice_hip_sparse_quantized_conv_features_dense_map.argtypes = [
        I, P, I, I, P, P, P, I, I, I, I, I, P, P, I, P, P, I, P]
    lib.lattice_hip_last_error.restype = ctypes.c_char_p
    return lib


def _close(actual, ref, rtol, atol, what):
    err = np.abs(actual - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (f'{what}: {bad.sum()} of {bad.size} outside '
                           f'tolerance; max err {err.max():.3e}')


def _cloud(n, grid, seed):
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(seed)
    return sphere_shell_cloud(n, grid, rng=rng), rng


def _relation(coords, n_active):
    from mlx_lattice_amd._native import ext

    c = torch.as_tensor(coords, dtype=torch.int32).to(DEV)
    active = torch.tensor([n_active], dtype=torch.int32, device=DEV)
    return ext.build_submanifold_kernel_relation_with_view(c, active, [3, 3, 3], [1, 1, 1])


def _fp64(coords, feats, w5, n_active):
    rel = O.kernel_relation(coords[:n_active], kernel_size=3)
    return O.conv_features_fp64(feats[:n_active].astype(np.float64),
                                O.mapped_weight(w5.astype(np.float64)), rel)


@pytest.mark.parametrize('dtype,c_in,c_out,epilogue', [
    (torch.float16, 4, 32, 0),
    (torch.float16, 4, 16, 1),
    (torch.float16, 8, 32, 0),
    (torch.bfloat16, 4, 32, 1),
    (torch.bfloat16, 8, 16, 0),
])
def test_dense_map_entry_matches_fp64_and_csr(dtype, c_in, c_out, epilogue):
    from mlx_lattice_amd._native import ext

    coords, rng = _cloud(30000, 160, 7 + c_in + c_out + epilogue)
    n = len(coords)
    n_active = n - 123   # rows past the active count hold the bias alone
    print(f'dense map {dtype} {c_in}->{c_out} epilogue={epilogue}', flush=True)
    feats = rng.standard_normal((n, c_in)).astype(np.float32)
    w = (rng.standard_normal((c_out, 3, 3, 3, c_in)) * np.sqrt(2.0 / (27 * c_in))).astype(np.float32)
    f = torch.as_tensor(feats).to(DEV, dtype)
    wt = torch.as_tensor(w).to(DEV, dtype)
    bias = torch.linspace(-0.5, 0.5, c_out, device=DEV).to(dtype)
    rel = _relation(coords, n_active)
    lib = _lib()
    out = torch.full((n, c_out), float('nan'), dtype=dtype, device=DEV)
    code = 1 if dtype == torch.float16 else 2
    rc = lib.lattice_hip_sparse_conv_features_dense_map(
        code, f.data_ptr(), n, c_in, wt.data_ptr(), 1, 27, c_out, rel[10].data_ptr(),
        rel[5].data_ptr(), n, out.data_ptr(), bias.data_ptr(), epilogue,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.lattice_hip_last_error()
    csr = ext.sparse_conv_features_csr(f, wt, rel[0], rel[2], rel[5], rel[3], n, 27,
                                       bias=bias, relu=bool(epilogue))
    torch.cuda.synchronize()
    got = to_np(out.float())
    assert not np.isnan(got).any()
    # rows past the active count: the bias (after ReLU), as on the CSR route
    assert torch.equal(out[n_active:], csr[n_active:])
    fin = to_np(f.float())
    ref = _fp64(coords, fin, to_np(wt.float()), n_active) + to_np(bias.float())[None, :]
    if epilogue:
        ref = np.maximum(ref, 0.0)
    tol = (RTOL_F16, ATOL_F16) if dtype == torch.float16 else (RTOL_BF16, ATOL_BF16)
    _close(got[:n_active], ref, *tol, 'dense map vs fp64')
    # both routes accumulate in fp32 and round once: they agree to a few ulps
    _close(got, to_np(csr.float()), 4e-3 if dtype == torch.float16 else 3e-2, 2e-3,
           'dense map vs CSR route')
    # the native CSR function takes the dense map when given it
    via = ext.sparse_conv_features_csr(f, wt, rel[0], rel[2], rel[5], rel[3], n, 27,
                                       bias=bias, relu=bool(epilogue), out_in_map=rel[10])
    assert torch.equal(via, out)


@pytest.mark.parametrize('bits', [4, 8])
def test_quantized_dense_map_entry(bits):
    from mlx_lattice_amd import dequantize_weight, quantize_weight

    coords, rng = _cloud(30000, 160, 40 + bits)
    n = len(coords)
    c_in, c_out = 4, 32
    feats = rng.standard_normal((n, c_in)).astype(np.float32)
    w = torch.as_tensor((rng.standard_normal((c_out, 3, 3, 3, c_in))
                         * np.sqrt(2.0 / (27 * c_in))).astype(np.float32)).to(DEV, torch.float16)
    q = quantize_weight(w, group_size=32, bits=bits)
    assert q.storage_in_channels == 32
    f = torch.as_tensor(feats).to(DEV, torch.float16)
    rel = _relation(coords, n)
    print(f'quantized dense map int{bits}', flush=True)
    lib = _lib()
    out = torch.full((n, c_out), float('nan'), dtype=torch.float16, device=DEV)
    rc = lib.lattice_hip_sparse_quantized_conv_features_dense_map(
        1, f.data_ptr(), n, c_in, q.weight.data_ptr(), q.scales.data_ptr(), q.biases.data_ptr(),
        27, c_out, q.storage_in_channels, q.group_size, bits, rel[10].data_ptr(),
        rel[5].data_ptr(), n, out.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.lattice_hip_last_error()
    torch.cuda.synchronize()
    fin = to_np(f.float())
    ref = _fp64(coords, fin, to_np(dequantize_weight(q).float()), n)
    _close(to_np(out.float()), ref, RTOL_F16, ATOL_F16, f'int{bits} dense map vs fp64')
    # the reference's quantized CPU route over the same relation, in fp32 on
    # the same (fp16-representable) feature values
    orel = O.kernel_relation(coords, kernel_size=3)
    cpu = O.quantized_conv_features(
        fin, to_np(q.weight), to_np(q.scales.float()), to_np(q.biases.float()), orel,
        in_channels=c_in, out_channels=c_out, storage_in_channels=q.storage_in_channels,
        group_size=q.group_size, bits=bits)
    _close(to_np(out.float()), cpu.astype(np.float32), RTOL_F16, ATOL_F16,
           f'int{bits} dense map vs reference CPU route')


def test_operator_path_takes_the_dense_map_route():
    """subm_conv3d and QuantizedSubmConv3d with 4 input channels run the
    dense-map kernel (their outputs equal the C entry's bit for bit)."""
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor, quantize_weight
    from mlx_lattice_amd._native import ext

    coords, rng = _cloud(20000, 128, 3)
    n = len(coords)
    feats = rng.standard_normal((n, 4)).astype(np.float16)
    w = torch.as_tensor((rng.standard_normal((32, 3, 3, 3, 4)) * 0.3).astype(np.float16)).to(DEV)
    x = SparseTensor(torch.as_tensor(coords, dtype=torch.int32).to(DEV), torch.as_tensor(feats).to(DEV))
    y = ops.subm_conv3d(x, w, kernel_size=3)
    rel = _relation(coords, n)
    direct = ext.sparse_conv_features_csr(x.feats, w, rel[0], rel[2], rel[5], rel[3], n, 27,
                                          out_in_map=rel[10])
    assert torch.equal(y.feats, direct)
    q = quantize_weight(w, group_size=32, bits=8)
    yq = ops.subm_conv3d(x, q, kernel_size=3)
    lib = _lib()
    out = torch.empty((n, 32), dtype=torch.float16, device=DEV)
    rc = lib.lattice_hip_sparse_quantized_conv_features_dense_map(
        1, x.feats.data_ptr(), n, 4, q.weight.data_ptr(), q.scales.data_ptr(), q.biases.data_ptr(),
        27, 32, q.storage_in_channels, q.group_size, 8, rel[10].data_ptr(), rel[5].data_ptr(), n,
        out.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.lattice_hip_last_error()
    torch.cuda.synchronize()
    assert torch.equal(yq.feats, out)


def test_other_shapes_keep_the_csr_route():
    """A dense map passed with a shape the kernel does not take (16 input
    channels) leaves the CSR route's result unchanged."""
    from mlx_lattice_amd._native import ext

    coords, rng = _cloud(5000, 128, 9)
    n = len(coords)
    f = torch.as_tensor(rng.standard_normal((n, 16)).astype(np.float16)).to(DEV)
    w = torch.as_tensor((rng.standard_normal((32, 3, 3, 3, 16)) * 0.1).astype(np.float16)).to(DEV)
    rel = _relation(coords, n)
    a = ext.sparse_conv_features_csr(f, w, rel[0], rel[2], rel[5], rel[3], n, 27)
    b = ext.sparse_conv_features_csr(f, w, rel[0], rel[2], rel[5], rel[3], n, 27, out_in_map=rel[10])
    torch.cuda.synchronize()
    assert torch.equal(a, b)
