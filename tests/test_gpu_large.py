"""A feature table past 2 GiB stays on the matrix cores.

8.6M rows x 128 fp16 channels is 2.2 GB of features.  The streamed
matrix-core conv addresses rows with unsigned 32-bit byte offsets, so any
table below 4 GiB takes it.  The cloud: 8.58M isolated voxels (spacing 3,
only their own centre edge), then a 20k-row sphere-shell cluster whose rows
sit past the 2 GiB mark of the table.  The conv is called through the C ABI
entry of the streamed route (which returns LATTICE_ERROR_UNSUPPORTED instead
of falling back), and checked against the fp64 sum (fp16 rtol 2e-2, atol
1e-2): the whole cluster against the oracle's relation of the cluster, and
sampled isolated rows against feats @ W[centre]."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = 'cuda'
LIB = (Path(__file__).resolve().parents[1] / 'mlx-lattice_amd' /
       'mlx_lattice_amd' / 'liblattice_hip.so')


def test_feature_table_over_2gib_takes_the_streamed_matrix_core_route():
    from mlx_lattice_amd._native import ext
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    n_total, c = 8_600_000, 128
    rng = np.random.default_rng(77)
    cluster = sphere_shell_cloud(20000, 128, rng=rng)
    n_iso = n_total - len(cluster)
    i = np.arange(n_iso, dtype=np.int64)
    iso = np.stack([np.zeros_like(i), 3 * (i % 1024), 3 * ((i // 1024) % 1024),
                    3 * (i // (1024 * 1024))], axis=1).astype(np.int32)
    shifted = cluster.copy()
    shifted[:, 3] += 40000                       # far from every isolated voxel
    coords = np.concatenate([iso, shifted])
    n = len(coords)
    assert (n + 1) * c * 2 > 2 ** 31 and (n + 1) * c * 2 <= 2 ** 32
    print(f'large table: {n} rows x {c} fp16 = {n * c * 2 / 2**30:.2f} GiB',
          flush=True)
    cd = torch.as_tensor(coords).to(DEV)
    active = torch.full((1,), n, dtype=torch.int32, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(78)
    feats = torch.randn((n, c), generator=gen, device=DEV).to(torch.float16)
    w = torch.as_tensor((rng.standard_normal((c, 3, 3, 3, c))
                         * np.sqrt(2.0 / (27 * c))).astype(np.float16)).to(DEV)
    rel = ext.build_submanifold_kernel_relation_with_view(cd, active, [3, 3, 3],
                                                          [1, 1, 1])
    reorder, _, kv, tiles = ext.build_sorted_implicit_gemm_view(rel[10], rel[11])
    frag = ext.conv_weight_fragments(w)
    assert frag.numel() > 0
    out = torch.empty((n, c), dtype=torch.float16, device=DEV)
    lib = ctypes.CDLL(str(LIB))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.lattice_hip_conv_workspace_bytes.restype = ctypes.c_size_t
    lib.lattice_hip_sparse_conv_features_sorted_fragments.argtypes = [
        I, P, I, I, P, I, I, P, P, P, I, P, P, I, P, ctypes.c_size_t, P]
    lib.lattice_hip_last_error.restype = ctypes.c_char_p
    wsb = lib.lattice_hip_conv_workspace_bytes(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    rc = lib.lattice_hip_sparse_conv_features_sorted_fragments(
        1, feats.data_ptr(), n, c, frag.data_ptr(), 27, c, kv.data_ptr(),
        tiles.data_ptr(), reorder.data_ptr(), n, out.data_ptr(), None, 0,
        ws.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.lattice_hip_last_error()
    torch.cuda.synchronize()

    def close(got, ref, what):
        err = np.abs(got - ref)
        bad = err > 1e-2 + 2e-2 * np.abs(ref)
        assert not bad.any(), f'{what}: {bad.sum()} outside, max {err.max():.3e}'

    w64 = O.mapped_weight(w.cpu().numpy().astype(np.float64))
    cf = feats[n_iso:].cpu().numpy()
    crel = O.kernel_relation(shifted, kernel_size=3)
    ref = O.conv_features_fp64(cf.astype(np.float64), w64, crel)
    close(out[n_iso:].float().cpu().numpy(), ref, 'cluster past 2 GiB')
    pick = np.concatenate([rng.integers(0, n_iso, 2000), np.arange(n_iso - 64, n_iso)])
    fi = feats[torch.as_tensor(pick).to(DEV)].cpu().numpy().astype(np.float64)
    close(out[torch.as_tensor(pick).to(DEV)].float().cpu().numpy(), fi @ w64[13],
          'isolated rows')
