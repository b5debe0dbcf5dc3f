"""Config 5: the int8-quantized four-stage sparse encoder on the GPU.

Each layer is checked on its own against the oracle: the oracle's quantized
CPU route (cpu/quantized.cpp:64-141, fp32 accumulation) runs on the very
fp16 input the GPU layer received, over the oracle's own relation, then adds
the folded-BatchNorm bias and applies ReLU in float32.  The GPU output must
match within the fp16 tolerance ``rtol=2e-2, atol=1e-2``.  Output
coordinates of every downsample must equal the oracle's bit for bit.
Checking layer by layer keeps one layer's rounding from being amplified by
the next, so the bar stays the per-conv one.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_np
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'
RTOL_F16, ATOL_F16 = 2e-2, 1e-2


def _modules(layers):
    from mlx_lattice_amd.nn import Conv3d, SubmConv3d
    from mlx_lattice_amd.nn.quantized_conv import (QuantizedConv3d,
                                                   QuantizedSubmConv3d)

    mods = []
    for spec in layers:
        c_out, *_, c_in = spec['weight'].shape
        if spec['kind'] == 'subm':
            dense = SubmConv3d(c_in, c_out, kernel_size=3, device=DEV,
                               dtype=torch.float16)
            cls = QuantizedSubmConv3d
        else:
            dense = Conv3d(c_in, c_out, kernel_size=2, stride=2, device=DEV,
                           dtype=torch.float16)
            cls = QuantizedConv3d
        dense.weight.data.copy_(torch.as_tensor(spec['weight']))
        dense.bias.data.copy_(torch.as_tensor(spec['bias']))
        mods.append(cls.from_conv(dense, group_size=32, bits=8))
    return mods


def _run_encoder(rows_per_batch: int, batches: int):
    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd.synthetic import (config_rng, encoder_layers,
                                           lidar_cloud)

    rng = config_rng(5)
    coords = lidar_cloud(rows_per_batch, batches, rng=rng)
    feats = rng.random((len(coords), 4)).astype(np.float16)
    layers = encoder_layers(rng)
    mods = _modules(layers)
    x = SparseTensor(torch.as_tensor(coords).to(DEV),
                     torch.as_tensor(feats).to(DEV))
    for i, (spec, mod) in enumerate(zip(layers, mods)):
        n_in = int(x.active_rows.item()) if x.active_rows is not None \
            else x.coords.shape[0]
        in_coords = to_np(x.coords[:n_in])
        in_feats = to_np(x.feats[:n_in])
        y = mod(x)
        y = y.replace(feats=torch.relu(y.feats))
        torch.cuda.synchronize()
        geom = dict(kernel_size=spec['kernel_size'], stride=spec['stride'])
        rel = O.kernel_relation(in_coords, **geom)
        n_out = int(rel['counts'][1])
        got_n = (int(y.active_rows.item()) if y.active_rows is not None
                 else y.coords.shape[0])
        assert got_n == n_out, f'layer {i}: {got_n} rows vs {n_out}'
        np.testing.assert_array_equal(to_np(y.coords[:n_out]),
                                      rel['out_coords'][:n_out],
                                      err_msg=f'layer {i} coords')
        ref = O.quantized_conv_features(
            in_feats, to_np(mod.weight), to_np(mod.scales),
            to_np(mod.biases), rel, in_channels=mod.in_channels,
            out_channels=mod.out_channels,
            storage_in_channels=to_np(mod.weight).shape[1] * 32 // mod.bits,
            group_size=mod.group_size, bits=mod.bits)[:n_out]
        ref = np.maximum(ref.astype(np.float32)
                         + to_np(mod.bias).astype(np.float32), 0.0)
        got = to_np(y.feats[:n_out].float())
        err = np.abs(got - ref)
        bad = err > ATOL_F16 + RTOL_F16 * np.abs(ref)
        assert not bad.any(), (
            f'layer {i} ({spec["kind"]} {mod.in_channels}->'
            f'{mod.out_channels}): {bad.sum()} of {bad.size} outside '
            f'tolerance, max err {err.max():.3e}')
        x = y
    return x


def test_config5_int8_encoder_small():
    out = _run_encoder(20000, 4)
    assert out.feats.shape[1] == 256


def test_config5_int8_encoder_full():
    """The BASELINE configuration: 4 batches of ~120k voxels."""
    out = _run_encoder(120000, 4)
    assert out.feats.shape[1] == 256
