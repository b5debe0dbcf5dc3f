"""Host-side checks that need no GPU: the C-ABI library loads and exports
every entry point declared in include/lattice_hip.h, the binding's host
logic (offsets, capacities, validation errors), and the Python operator
layer's pure-host parts (KernelSpec, relation containers, quantizer
layout)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / 'mlx-lattice_amd' / 'mlx_lattice_amd' / 'liblattice_hip.so'
HEADER = ROOT / 'include' / 'lattice_hip.h'


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r'\b(lattice_hip_\w+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    names = declared_symbols()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name


def test_c_abi_host_queries():
    lib = ctypes.CDLL(str(LIB))
    lib.lattice_hip_coord_hash_capacity.restype = ctypes.c_int
    assert lib.lattice_hip_coord_hash_capacity(400000) == 1 << 20
    assert lib.lattice_hip_coord_hash_capacity(0) == 1
    assert lib.lattice_hip_coord_hash_capacity(3) == 8
    size = (ctypes.c_int * 3)(3, 3, 3)
    dil = (ctypes.c_int * 3)(1, 1, 1)
    out = (ctypes.c_int32 * 81)()
    assert lib.lattice_hip_kernel_offsets(size, dil, out) == 27
    assert list(out)[39:42] == [0, 0, 0]
    bad = (ctypes.c_int * 3)(0, 3, 3)
    assert lib.lattice_hip_kernel_offsets(bad, dil, None) == -1
    lib.lattice_hip_kernel_relation_workspace_bytes.restype = ctypes.c_size_t
    assert lib.lattice_hip_kernel_relation_workspace_bytes(400000, 27) > 0
    lib.lattice_hip_block_table_bytes.restype = ctypes.c_size_t
    assert lib.lattice_hip_block_table_bytes(400000) == 64 << 20
    lib.lattice_hip_version.restype = ctypes.c_char_p
    assert b'gfx950' in lib.lattice_hip_version()


def test_c_abi_rejects_bad_arguments_without_touching_the_gpu():
    lib = ctypes.CDLL(str(LIB))
    lib.lattice_hip_last_error.restype = ctypes.c_char_p
    size = (ctypes.c_int * 3)(3, 3, 3)
    one = (ctypes.c_int * 3)(1, 1, 1)
    zero = (ctypes.c_int * 3)(0, 0, 0)
    neg = (ctypes.c_int * 3)(-1, 0, 0)
    rc = lib.lattice_hip_build_kernel_relation(
        None, 0, None, size, one, neg, one, None, None, ctypes.c_size_t(0),
        None)
    assert rc == 1 and b'padding' in lib.lattice_hip_last_error()
    rc = lib.lattice_hip_build_kernel_relation(
        None, 0, None, size, one, zero, one, None, None, ctypes.c_size_t(0),
        None)
    assert rc == 1 and b'outputs' in lib.lattice_hip_last_error()
    rc = lib.lattice_hip_sparse_quantized_conv_features(
        1, None, 0, 16, None, None, None, 27, 16, 16, 16, 4, None, None, None,
        0, None, None, None, None, 0, None, None, 0, None, ctypes.c_size_t(0),
        None)
    assert rc == 1 and b'group_size' in lib.lattice_hip_last_error()
    rc = lib.lattice_hip_sparse_conv_features(
        7, None, 0, 16, None, 0, 27, 16, None, None, None, 0, None, 0, None,
        None, 0, None)
    assert rc == 1 and b'float' in lib.lattice_hip_last_error()


def test_binding_host_logic():
    from mlx_lattice_amd._native import ext

    assert ext.coord_hash_capacity(5) == 16
    assert ext.kernel_offsets([3, 1, 1], [1, 1, 1]) == [[-1, 0, 0], [0, 0, 0],
                                                       [1, 0, 0]]
    assert ext.kernel_offsets([2, 2, 2], [2, 2, 2])[-1] == [2, 2, 2]
    coords = torch.zeros((3, 4), dtype=torch.int32)
    active = torch.tensor([3], dtype=torch.int32)
    with pytest.raises(ValueError, match='HIP device tensor'):
        ext.build_kernel_relation(coords, active, [3, 3, 3], [1, 1, 1],
                                  [0, 0, 0], [1, 1, 1])
    with pytest.raises(ValueError, match=r'shape \(N, 4\)'):
        ext.build_kernel_relation(torch.zeros((3, 3), dtype=torch.int32),
                                  active, [3, 3, 3], [1, 1, 1], [0, 0, 0],
                                  [1, 1, 1])
    with pytest.raises(ValueError, match='active_rows'):
        ext.build_kernel_relation(coords, torch.tensor([3]), [3, 3, 3],
                                  [1, 1, 1], [0, 0, 0], [1, 1, 1])
    with pytest.raises(ValueError, match='stride'):
        ext.build_kernel_relation(coords, active, [3, 3, 3], [0, 1, 1],
                                  [0, 0, 0], [1, 1, 1])
    feats = torch.zeros((3, 4), dtype=torch.float16)
    w = torch.zeros((8, 3, 3, 3, 4), dtype=torch.float32)
    e = torch.zeros(3 * 27, dtype=torch.int32)
    with pytest.raises(ValueError, match='match feats dtype'):
        ext.sparse_conv_features(feats, w, e, e, e,
                                 torch.zeros(2, dtype=torch.int32),
                                 torch.zeros(4, dtype=torch.int32),
                                 torch.zeros(4, dtype=torch.int32), e,
                                 torch.zeros(28, dtype=torch.int32), e, 3, 27)


def test_kernel_spec_and_offsets():
    from mlx_lattice_amd import KernelSpec
    from mlx_lattice_amd.core.coords.builders import kernel_offsets

    pointwise = KernelSpec(size=1)
    assert pointwise.size == (1, 1, 1) and pointwise.is_pointwise
    assert KernelSpec(size=(3, 3, 3)).volume == 27
    assert not KernelSpec(size=2).is_centered_submanifold
    for kwargs, match in ((dict(size=0), 'kernel_size'),
                          (dict(stride=0), 'stride'),
                          (dict(padding=-1), 'padding'),
                          (dict(dilation=0), 'dilation')):
        with pytest.raises(ValueError, match=match):
            KernelSpec(**kwargs)
    assert kernel_offsets((3, 1, 1)) == ((-1, 0, 0), (0, 0, 0), (1, 0, 0))


def test_relation_container_contract():
    from mlx_lattice_amd.core import KernelRelation, SparseRelationContract

    rows = torch.tensor([0, 1], dtype=torch.int32)
    out_coords = torch.tensor([[0, 0, 0, 0], [0, 1, 0, 0]], dtype=torch.int32)
    rel = KernelRelation(rows, rows, rows, kernel_offsets=((0, 0, 0),
                                                           (1, 0, 0)),
                         out_coords=out_coords, n_in_capacity=2)
    assert rel.edge_capacity == 2 and rel.n_out_capacity == 2
    assert rel.n_kernels == 2 and isinstance(rel.contract,
                                             SparseRelationContract)
    assert rel.out_view is rel.output_csr
    with pytest.raises(ValueError, match='same row count'):
        KernelRelation(rows, rows[:1], rows)
    with pytest.raises(ValueError, match='n_kernels'):
        KernelRelation(rows, rows, rows, kernel_offsets=((0, 0, 0),),
                       n_kernels=2)


@pytest.mark.parametrize('bits', [4, 8])
def test_quantizer_layout_and_round_trip(bits):
    from mlx_lattice_amd import dequantize_weight, quantize_weight

    rng = np.random.default_rng(bits)
    w = torch.as_tensor(rng.standard_normal((12, 3, 1, 1, 16)).astype(
        np.float32))
    q = quantize_weight(w, bits=bits)
    assert q.weight.dtype == torch.uint32
    assert q.in_channels == 16 and q.storage_in_channels == 32
    assert tuple(q.weight.shape) == (3, 32 * bits // 32, 12)
    assert tuple(q.scales.shape) == (3, 1, 12)
    deq = dequantize_weight(q)
    assert deq.shape == w.shape
    levels = 2 ** bits - 1
    span = (w.amax() - w.amin()).item()
    assert (deq - w).abs().max().item() <= span / levels
    memory = quantize_weight(torch.ones((64, 3, 3, 3, 64),
                                        dtype=torch.float16), bits=bits)
    assert memory.nbytes < 64 * 27 * 64 * 2


def test_quantized_words_follow_the_unpack_rule():
    from mlx_lattice_amd import quantize_weight
    from oracle import oracle as O

    rng = np.random.default_rng(2)
    w = torch.as_tensor(rng.standard_normal((8, 3, 3, 3, 64)).astype(
        np.float32))
    for bits in (4, 8):
        q = quantize_weight(w, group_size=32, bits=bits)
        deq_oracle = O.dequantize_mapped(
            q.weight.numpy(), q.scales.numpy(), q.biases.numpy(),
            in_channels=64, out_channels=8, storage_in_channels=64,
            group_size=32, bits=bits)
        from mlx_lattice_amd import dequantize_weight

        deq = dequantize_weight(q).numpy()
        mapped = deq.transpose(1, 2, 3, 4, 0).reshape(27, 64, 8)
        np.testing.assert_array_equal(mapped, deq_oracle)


def test_spec_literal_shell_subsample():
    """The literal config-3 cloud: distinct voxels, all on complete shells,
    drawn uniformly, so neighbours are sparse (about 2 active offsets per
    row at the full 400k / 200-sphere scale; checked here on 12 spheres)."""
    import numpy as np

    from mlx_lattice_amd.synthetic import (_shell_voxels,
                                           sphere_shell_subsample_cloud)

    rng = np.random.default_rng(5)
    cloud = sphere_shell_subsample_cloud(20000, 256, spheres=12, rng=rng)
    assert cloud.shape == (20000, 4) and cloud.dtype == np.int32
    assert len(np.unique(cloud, axis=0)) == 20000
    assert (cloud[:, 0] == 0).all()
    # every voxel lies on one of the 12 shells drawn by the same seed
    rng = np.random.default_rng(5)
    shells = set()
    for _ in range(12):
        r = rng.uniform(8.0, 60.0)
        margin = int(np.ceil(r)) + 1
        c = rng.uniform(margin, 256 - margin, size=3)
        shells.update(map(tuple, _shell_voxels(c, r).tolist()))
    assert all(tuple(v) in shells for v in cloud[:, 1:].tolist())
    assert len(shells) > 20000


@pytest.mark.parametrize('rows', [0, 1, 2, 3, 7, 8, 63, 64, 65, 1000, 65535,
                                  65536, 400000, 699050, 699051, 10 ** 7,
                                  (1 << 28) - 1])
def test_table_capacities_always_leave_empty_slots(rows):
    """Every probe loop of the coordinate tables stops at the first empty
    slot (or after `capacity` probes, flagging an overflow).  Both tables
    are sized so that empty slots always remain: the voxel table holds at
    most `rows` keys in at least 2 * rows slots, the 2x2x2 block table at
    most `rows` blocks in more than 1.5 * rows buckets."""
    lib = ctypes.CDLL(str(LIB))
    lib.lattice_hip_coord_hash_capacity.restype = ctypes.c_int
    lib.lattice_hip_block_table_capacity.restype = ctypes.c_int
    lib.lattice_hip_block_table_bytes.restype = ctypes.c_size_t
    cap = lib.lattice_hip_coord_hash_capacity(rows)
    assert cap >= max(2 * rows, 1) and cap & (cap - 1) == 0
    buckets = lib.lattice_hip_block_table_capacity(rows)
    assert buckets > rows + rows // 2 and buckets & (buckets - 1) == 0
    assert buckets < 2 * (rows + rows // 2 + 1)      # the next power of two
    assert lib.lattice_hip_block_table_bytes(rows) >= 64 * buckets


def test_header_declares_the_table_overflow_flag():
    """The overflow bit the bounded probe loops set is part of the ABI and
    is the bit the host-side status reader raises on."""
    text = HEADER.read_text()
    assert re.search(r'LATTICE_STATUS_TABLE_OVERFLOW\s*=\s*16', text)


def test_status_word_reader_raises_on_table_overflow():
    from mlx_lattice_amd.core.relations.views import _StatusWord

    assert _StatusWord(torch.tensor([8], dtype=torch.int32)).read() == 8
    with pytest.raises(RuntimeError, match='overflowed'):
        _StatusWord(torch.tensor([16 | 2], dtype=torch.int32)).read()
