"""The allocation-free matrix-core conv entry point
(lattice_hip_sparse_conv_features_sorted_implicit_gemm_noalloc), called
through the C ABI, against the entry point it mirrors
(lattice_hip_sparse_conv_features_sorted_implicit_gemm with a caller
workspace).  Both run the same kernels; only where the tile schedule lives
differs, so the outputs must agree bit for bit.  Two calls in a row, the
second on a smaller cloud (the scratch keeps the first call's schedule and
must not leak into the second).  Calls on two streams of one GPU share
the scratch and are put in submission order by the entry point."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = 'cuda'
ROOT_LIB = (Path(__file__).resolve().parents[1] / 'mlx-lattice_amd' /
            'mlx_lattice_amd' / 'liblattice_hip.so')
MAX_ROWS = 2097088   # LATTICE_NOALLOC_CONV_MAX_ROWS


def _lib():
    lib = ctypes.CDLL(str(ROOT_LIB))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.lattice_hip_conv_workspace_bytes.restype = ctypes.c_size_t
    lib.lattice_hip_sparse_conv_features_sorted_implicit_gemm.argtypes = [
        I, P, I, I, P, I, I, I, P, P, P, I, P, P, I, P, ctypes.c_size_t, P]
    lib.lattice_hip_sparse_conv_features_sorted_implicit_gemm_noalloc.argtypes = [
        I, P, I, I, P, I, I, I, P, P, P, I, P, P, I, P]
    lib.lattice_hip_last_error.restype = ctypes.c_char_p
    return lib


def _prepare(lib, n, grid, seed, c_in, c_out, epilogue=0):
    """A cloud, its sorted view and the workspace entry's output `ref`;
    returns (args, ref, got, bias, epilogue, keep) for the no-alloc call."""
    from mlx_lattice_amd._native import ext
    from mlx_lattice_amd.synthetic import sphere_shell_cloud

    rng = np.random.default_rng(seed)
    coords = sphere_shell_cloud(n, grid, rng=rng)
    n = len(coords)
    print(f'no-alloc conv case n={n} c_in={c_in} c_out={c_out} '
          f'epilogue={epilogue}', flush=True)
    c = torch.as_tensor(coords).to(DEV)
    active = torch.full((1,), n, dtype=torch.int32, device=DEV)
    rel = ext.build_submanifold_kernel_relation_with_view(c, active, [3, 3, 3],
                                                          [1, 1, 1])
    reorder, _, kv, tiles = ext.build_sorted_implicit_gemm_view(rel[10], rel[11])
    feats = torch.as_tensor(rng.standard_normal((n, c_in)).astype(np.float16)).to(DEV)
    w = torch.as_tensor((rng.standard_normal((c_out, 3, 3, 3, c_in)) * 0.05)
                        .astype(np.float16)).to(DEV)
    bias = torch.linspace(-1, 1, c_out, device=DEV, dtype=torch.float16)
    stream = torch.cuda.current_stream().cuda_stream
    wsb = lib.lattice_hip_conv_workspace_bytes(n)
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    ref = torch.full((n, c_out), float('nan'), dtype=torch.float16, device=DEV)
    got = torch.full((n, c_out), float('nan'), dtype=torch.float16, device=DEV)
    args = (1, feats.data_ptr(), n, c_in, w.data_ptr(), 1, 27, c_out,
            kv.data_ptr(), tiles.data_ptr(), reorder.data_ptr(), n)
    assert lib.lattice_hip_sparse_conv_features_sorted_implicit_gemm(
        *args, ref.data_ptr(), bias.data_ptr(), epilogue, ws.data_ptr(), wsb,
        stream) == 0
    torch.cuda.synchronize()
    return args, ref, got, bias, epilogue, (c, active, rel, kv, tiles, reorder, feats, w, ws)


def _noalloc(lib, prepared, stream):
    args, _, got, bias, epilogue, _ = prepared
    rc = lib.lattice_hip_sparse_conv_features_sorted_implicit_gemm_noalloc(
        *args, got.data_ptr(), bias.data_ptr(), epilogue, stream)
    assert rc == 0, lib.lattice_hip_last_error()


def _check(prepared):
    _, ref, got, _, _, _ = prepared
    assert not torch.isnan(got).any()
    assert torch.equal(got, ref)


def _case(lib, n, grid, seed, c_in, c_out, epilogue=0):
    prepared = _prepare(lib, n, grid, seed, c_in, c_out, epilogue)
    _noalloc(lib, prepared, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _check(prepared)


def test_noalloc_conv_matches_workspace_entry():
    lib = _lib()
    _case(lib, 60000, 160, 5, 64, 128)     # first call
    _case(lib, 9000, 96, 6, 32, 64)        # second call, smaller
    _case(lib, 20000, 128, 7, 64, 256)     # two launches share one schedule
    _case(lib, 12000, 128, 8, 64, 128, 1)  # with the fused ReLU


def test_noalloc_conv_orders_calls_on_two_streams():
    # A large call on one stream and, queued right behind it with no
    # synchronisation between the streams, a smaller one on another: the
    # second call's schedule would overwrite the first's in the shared
    # scratch while the first conv still reads it, unless the entry point
    # orders them.
    lib = _lib()
    big = _prepare(lib, 300000, 400, 9, 128, 128)
    small = _prepare(lib, 9000, 128, 10, 32, 64)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    print('no-alloc conv on two streams', flush=True)
    _noalloc(lib, big, s1.cuda_stream)
    _noalloc(lib, small, s2.cuda_stream)
    torch.cuda.synchronize()
    _check(big)
    _check(small)


def test_noalloc_conv_under_graph_capture():
    # The entry's launches recorded into a graph (no allocation, no event
    # while capturing), replayed three times with eager work and a
    # synchronisation between replays; every replay equals the workspace
    # entry's output.
    lib = _lib()
    prepared = _prepare(lib, 40000, 160, 12, 64, 128, 1)
    args, ref, got, bias, epilogue, _ = prepared
    print('no-alloc conv under graph capture', flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up on the capture stream
        _noalloc(lib, prepared, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.lattice_hip_sparse_conv_features_sorted_implicit_gemm_noalloc(
            *args, got.data_ptr(), bias.data_ptr(), epilogue,
            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.lattice_hip_last_error()
    for _ in range(3):
        got.fill_(float('nan'))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check(prepared)


def test_noalloc_conv_rejects_oversized_launches():
    lib = _lib()
    rc = lib.lattice_hip_sparse_conv_features_sorted_implicit_gemm_noalloc(
        1, None, 0, 64, None, 1, 27, 64, None, None, None, MAX_ROWS + 1,
        None, None, 0, None)
    assert rc != 0
    assert b'allocation-free' in lib.lattice_hip_last_error()
