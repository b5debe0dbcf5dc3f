"""The operator path never waits for the device.

The reference builds relations and convolutions lazily on the device
(native/features/convolution/streams.cpp:19-26): nothing in ``conv3d`` or
``subm_conv3d`` reads device memory back.  Here each operator call runs
under ``torch.cuda.set_sync_debug_mode('error')``, which raises on any
host wait torch issues (``.item()``, device-to-host copies, blocking
host-to-device copies).  The results are then checked against the oracle
(fp16 ``rtol=2e-2, atol=1e-2`` against the fp64 edge sum; coordinates
bit-exact).
"""

from __future__ import annotations

import contextlib

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'


@contextlib.contextmanager
def no_host_waits():
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode('error')
    try:
        yield
    finally:
        torch.cuda.set_sync_debug_mode(0)


def _close(got, ref, what):
    err = np.abs(got - ref)
    bad = err > 1e-2 + 2e-2 * np.abs(ref)
    assert not bad.any(), f'{what}: {bad.sum()} outside, max {err.max():.3e}'


def test_subm_and_downsample_convs_run_without_host_waits():
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(91)
    coords = sphere_shell_cloud(20000, 128, rng=rng)
    feats = rng.standard_normal((len(coords), 64)).astype(np.float16)
    w_subm = (rng.standard_normal((64, 3, 3, 3, 64)) * 0.03).astype(np.float16)
    w_down = (rng.standard_normal((32, 2, 2, 2, 64)) * 0.05).astype(np.float16)
    w_next = (rng.standard_normal((32, 3, 3, 3, 32)) * 0.05).astype(np.float16)
    c = torch.as_tensor(coords).to(DEV)
    f = torch.as_tensor(feats).to(DEV)
    ws, wd, wn = (torch.as_tensor(w).to(DEV) for w in (w_subm, w_down, w_next))
    bias = torch.linspace(-1, 1, 32, device=DEV, dtype=torch.float16)
    print(f'async operators N={len(coords)}', flush=True)
    with no_host_waits():
        x = SparseTensor(c, f)
        y = ops.subm_conv3d(x, ws, kernel_size=3)
        d = ops.conv3d(x, wd, kernel_size=2, stride=2, bias=bias)
        z = ops.subm_conv3d(d, wn, kernel_size=3)
    torch.cuda.synchronize()

    rel = O.kernel_relation(coords, kernel_size=3)
    ref = O.conv_features_fp64(feats, O.mapped_weight(w_subm.astype(np.float64)), rel)
    _close(to_np(y.feats.float()), ref, 'subm')

    down = O.kernel_relation(coords, kernel_size=2, stride=2)
    n = int(down['counts'][1])
    assert int(d.active_rows.item()) == n
    np.testing.assert_array_equal(to_np(d.coords[:n]), down['out_coords'][:n])
    ref_d = O.conv_features_fp64(feats, O.mapped_weight(w_down.astype(np.float64)), down)
    ref_d[:n] += to_np(bias.float())
    _close(to_np(d.feats[:n].float()), ref_d[:n], 'k2s2')

    sub2 = O.kernel_relation(down['out_coords'][:n], kernel_size=3)
    in2 = to_np(d.feats[:n])
    ref_z = O.conv_features_fp64(in2, O.mapped_weight(w_next.astype(np.float64)), sub2)
    _close(to_np(z.feats[:n].float()), ref_z, 'subm on the downsampled level')


def test_quantized_layers_run_without_host_waits():
    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd.nn import Conv3d, SubmConv3d
    from mlx_lattice_amd.nn.quantized_conv import (QuantizedConv3d,
                                                   QuantizedSubmConv3d)
    from mlx_lattice_amd.synthetic import config_rng, lidar_cloud

    rng = config_rng(5)
    coords = lidar_cloud(20000, 2, rng=rng)
    feats = rng.random((len(coords), 32)).astype(np.float16)
    dense_s = SubmConv3d(32, 64, kernel_size=3, device=DEV, dtype=torch.float16)
    dense_d = Conv3d(64, 64, kernel_size=2, stride=2, device=DEV, dtype=torch.float16)
    qs = QuantizedSubmConv3d.from_conv(dense_s, group_size=32, bits=8)
    qd = QuantizedConv3d.from_conv(dense_d, group_size=32, bits=4)
    c = torch.as_tensor(coords).to(DEV)
    f = torch.as_tensor(feats).to(DEV)
    print(f'async quantized layers N={len(coords)}', flush=True)
    with no_host_waits():
        x = SparseTensor(c, f)
        y = qs(x)
        z = qd(y)
    torch.cuda.synchronize()
    for mod, inp_coords, inp_feats, out, geom in (
            (qs, coords, feats, y, dict(kernel_size=3)),
            (qd, coords, to_np(y.feats), z, dict(kernel_size=2, stride=2))):
        rel = O.kernel_relation(inp_coords, **geom)
        n = int(rel['counts'][1])
        np.testing.assert_array_equal(to_np(out.coords[:n]), rel['out_coords'][:n])
        ref = O.quantized_conv_features(
            inp_feats, to_np(mod.weight), to_np(mod.scales), to_np(mod.biases),
            rel, in_channels=mod.in_channels, out_channels=mod.out_channels,
            storage_in_channels=to_np(mod.weight).shape[1] * 32 // mod.bits,
            group_size=mod.group_size, bits=mod.bits)[:n]
        ref = ref.astype(np.float32) + to_np(mod.bias).astype(np.float32)
        _close(to_np(out.feats[:n].float()), ref, f'quantized {geom}')


@pytest.mark.parametrize('ks', [2, 3])
def test_conv_transpose_runs_without_host_waits(ks):
    """Decoder step: conv_transpose3d from a stride-2 level back to stride
    1.  k=2 takes the direct expansion; k=3 the deduplicating transposed
    relation, whose repeated-edge flag is copied to pinned memory at build
    time instead of read back with ``.item()``."""
    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(92 + ks)
    fine = sphere_shell_cloud(20000, 128, rng=rng)
    down = O.kernel_relation(fine, kernel_size=2, stride=2)
    coarse = down['out_coords'][:int(down['counts'][1])]
    feats = rng.standard_normal((len(coarse), 64)).astype(np.float16)
    w = (rng.standard_normal((32, ks, ks, ks, 64)) * 0.03).astype(np.float16)
    c = torch.as_tensor(coarse).to(DEV)
    f = torch.as_tensor(feats).to(DEV)
    wt = torch.as_tensor(w).to(DEV)
    print(f'async conv_transpose3d k={ks} N={len(coarse)}', flush=True)
    with no_host_waits():
        x = SparseTensor(c, f, stride=2)
        y = ops.conv_transpose3d(x, wt, kernel_size=ks, stride=2)
    torch.cuda.synchronize()
    rel = O.transposed_kernel_relation(coarse, kernel_size=ks, stride=2)
    n = int(rel['counts'][1])
    assert int(y.active_rows.item()) == n
    np.testing.assert_array_equal(to_np(y.coords[:n]), rel['out_coords'][:n])
    ref = O.conv_features_fp64(feats, O.mapped_weight(w.astype(np.float64)), rel)
    _close(to_np(y.feats[:n].float()), ref[:n], f'conv_transpose3d k={ks}')
