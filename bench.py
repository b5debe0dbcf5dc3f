"""Benchmark of the sparse-convolution hot path on one MI355X.

Workload (the headline case): subm_conv3d k=3, fp16,
C_in = C_out = 128, batch 1, 400k voxels on sphere shells in a 512^3 grid,
Kaiming-normal weight, synthetic data (seeded).

One step = one pass of the hot path over the batch, inputs resident in HBM:
  1. kernel-map build: coordinate hash + submanifold relation (edges, CSR
     views, dense out_in_map / row masks) + mask-sorted implicit-GEMM view
     with its longest-first tile order (kept with the view, as the
     operator path keeps it);
  2. the implicit-GEMM convolution on the matrix cores.
Each phase is bracketed by HIP events on the stream the kernels run on.

``value`` = effective TFLOP/s of the convolution, F / t_conv with
F = 2 * E * C_in * C_out (E = active edges, useful MACs only).  The JSON line
also carries Mvoxels/s (N_out / t_conv), the kernel-map build time, the
roofline of the dominant kernel and the reference CPU route timed on the
host on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / 'mlx-lattice_amd'):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
# HBM bytes per conv_igemm launch on this workload, from rocprofv3 FETCH_SIZE
# and WRITE_SIZE passes scaled by a 1 GiB copy's counter readings
# (profiles/config3_kernel_traffic.md), valid for the kernel source whose
# SHA-256 prefix is given: when csrc/conv.hip changes, the bench reports
# traffic as null until the counters are measured again.
CONV_TRAFFIC = {'bytes': 1.1989e9, 'conv_hip_sha256': '94579b7b5780d8be'}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument('--gpus', type=int, default=1)
    p.add_argument('--steps', type=int, default=20)
    p.add_argument('--warmup', type=int, default=5)
    p.add_argument('--cpu-threads', type=int, default=16,
                   help='host threads for the CPU baseline (capped by the '
                        'machine)')
    p.add_argument('--cpu-sample-rows', type=int, default=131072,
                   help='output rows of the bounded CPU-baseline sample')
    p.add_argument('--no-cpu-baseline', action='store_true')
    p.add_argument('--no-secondary', action='store_true',
                   help='skip the timings of configs 2, 4 and 5')
    p.add_argument('--phase', choices=('all', 'config3', 'secondary',
                                       'backward', 'widened'),
                   default='all',
                   help='config3: only the headline step (for profiler '
                        'runs); secondary: only configs 2, 4 and 5 and '
                        'config 3 read literally; backward: only the config-3 '
                        'gradients; widened: only the gradient, pooling, '
                        'decoder and quantization lines')
    return p.parse_args()


def make_workload():
    import numpy as np

    from mlx_lattice_amd.synthetic import (
        config_rng,
        kaiming_weight,
        sphere_shell_cloud,
    )

    rng = config_rng(3)
    coords = sphere_shell_cloud(400000, 512, rng=rng)
    feats = rng.standard_normal((len(coords), 128)).astype(np.float16)
    weight = kaiming_weight((128, 3, 3, 3, 128), rng=rng).astype(np.float16)
    return coords, feats, weight


def host_cpu() -> dict:
    """The host's CPU model (lscpu's "Model name", read from
    /proc/cpuinfo), its hardware thread count and the threads this process
    may run on."""
    model = 'unknown'
    try:
        with open('/proc/cpuinfo') as fh:
            for line in fh:
                if line.lower().startswith('model name'):
                    model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {'model': model, 'hardware_threads': os.cpu_count() or 1,
            'usable_threads': usable}


def cpu_baseline(coords, feats, weight, threads: int, sample_rows: int,
                 repeats: int = 3):
    """Reference CPU route (oracle restatement, eval_typed with per-FMA fp16
    rounding for 128->128) on the first ``sample_rows`` output rows, plus the
    single-threaded relation build on the full cloud; each timed
    ``repeats`` times, the median reported (BASELINE.md's protocol)."""
    import statistics

    import numpy as np

    from oracle import oracle

    t_maps = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        rel = oracle.kernel_relation(coords, kernel_size=3)
        t_maps.append(time.perf_counter() - t0)
    t_map = statistics.median(t_maps)
    host = host_cpu()
    hw = oracle.hardware_concurrency()
    threads = max(1, min(threads, hw))
    n = min(sample_rows, len(coords))
    # parallel_for (cpu/algorithms.cpp:30-67) spawns ceil(n / 4096) workers
    # at most.
    workers = max(1, min(threads, (n + 4095) // 4096))
    sample = dict(rel)
    sample['counts'] = np.array([rel['counts'][0], n], np.int32)
    e_sample = int(rel['row_offsets'][n])
    t_convs = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        oracle.conv_features(feats, weight, sample, out_capacity=n,
                             threads=threads)
        t_convs.append(time.perf_counter() - t0)
    t_conv = statistics.median(t_convs)
    flops = 2.0 * e_sample * 128 * 128
    return {
        'value': round(flops / t_conv / 1e12, 6),
        'unit': 'TFLOP/s',
        'cores': workers,
        'kind': 'port',
        'workers': workers,
        'host_cpu': host['model'],
        'host_hardware_threads': host['hardware_threads'],
        'host_usable_threads': host['usable_threads'],
        'repeats': repeats,
        'sample': (f'reference CPU route restated (oracle/lattice_oracle.cpp)'
                   f' on {host["model"]} ({host["hardware_threads"]} hardware'
                   f' threads, {host["usable_threads"]} usable): relation '
                   f'build on all {len(coords)} rows, one thread (median of '
                   f'{repeats}: {t_map * 1e3:.1f} ms); conv on the first {n} '
                   f'output rows ({e_sample} edges) with {workers} worker '
                   f'threads (median of {repeats}: {t_conv:.2f} s, '
                   f'{n / t_conv / 1e6:.4f} Mvoxels/s)'),
        'map_build_ms': round(t_map * 1e3, 3),
        'mvoxels_per_s': round(n / t_conv / 1e6, 6),
    }


def _timed(fn, steps: int, warmup: int) -> float:
    """Mean milliseconds of ``fn`` over ``steps`` calls, HIP events on the
    current stream (the one the bindings launch on).  The warm-up repeats
    batches of ``warmup`` calls until 20 ms have passed: after the host
    work between two lines the GPU's clocks ramp up again over a few
    milliseconds of load, and the timed calls should see the clocks a busy
    GPU holds, as the headline's conv launches do."""
    import time

    import torch

    t0 = time.perf_counter()
    while True:
        for _ in range(max(warmup, 1)):
            fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= 0.02:
            break
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def secondary_workloads(steps: int = 10, warmup: int = 3) -> dict:
    """Configs 2, 4 and 5, and config 3 read literally (a uniform subsample
    of the complete shells), through the operator API.

    ``layer_ms`` builds a fresh coordinate manager every call, so it covers
    the kernel-map build, the sorted view, the conv and the bias;
    ``conv_ms`` reuses the cached relation and times the conv alone, which
    is what the effective TFLOP/s is computed from.
    """
    import numpy as np
    import torch

    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor, quantize_weight
    from mlx_lattice_amd.nn import Conv3d, SubmConv3d
    from mlx_lattice_amd.nn.quantized_conv import (QuantizedConv3d,
                                                   QuantizedSubmConv3d)
    from mlx_lattice_amd.synthetic import (config_rng, encoder_layers,
                                           kaiming_weight, lidar_cloud,
                                           sphere_shell_cloud,
                                           sphere_shell_subsample_cloud)

    dev = torch.device('cuda:0')
    out = {}

    def layer(coords, feats, run, c_in, c_out, k, workload, weight_bytes):
        x = SparseTensor(coords, feats)
        y = run(x)
        torch.cuda.synchronize()
        rel = x.coord_manager._kernel_relations
        relation = next(iter(rel.values()))
        edges = int(relation.counts[0].item())
        n_out = int(relation.counts[1].item())
        cap = int(y.feats.shape[0])
        layer_ms = _timed(lambda: run(SparseTensor(coords, feats)), steps,
                          warmup)
        conv_ms = _timed(lambda: run(x), steps, warmup)
        del y
        flops = 2.0 * edges * c_in * c_out
        # algorithmic bytes of the matrix-core conv: input rows once, every
        # capacity output row written once (fp16), the weight, and the
        # sorted view it reads (k-major map, reorder rows, tile masks)
        nbytes = (int(coords.shape[0]) * c_in * 2 + cap * c_out * 2
                  + weight_bytes + 4 * k * cap + 4 * cap + 16 * (cap // 64 + 1))
        tflops = flops / conv_ms / 1e9
        gbs = nbytes / conv_ms / 1e6
        hbm_bound = flops / nbytes < PEAK_FP16_TFLOPS / PEAK_HBM_GBS * 1e3
        return {
            'workload': workload,
            'voxels_in': int(coords.shape[0]), 'voxels_out': n_out,
            'edges': edges,
            'layer_ms': round(layer_ms, 4), 'conv_ms': round(conv_ms, 4),
            'tflops': round(tflops, 3),
            'mvoxels_per_s': round(n_out / conv_ms / 1e3, 3),
            'roofline': {
                'bound': 'hbm' if hbm_bound else 'mfma',
                'achieved': round(gbs if hbm_bound else tflops, 3),
                'peak': PEAK_HBM_GBS if hbm_bound else PEAK_FP16_TFLOPS,
                'unit': 'GB/s' if hbm_bound else 'TFLOP/s',
                'frac': round(gbs / PEAK_HBM_GBS if hbm_bound
                              else tflops / PEAK_FP16_TFLOPS, 4),
                'algorithmic_bytes': nbytes,
                'flops': flops,
                'interval': 'conv_ms (operator call on a cached relation)',
            },
        }

    rng = config_rng(2)
    c2 = torch.as_tensor(lidar_cloud(100000, 2, rng=rng)).to(dev)
    f2 = torch.as_tensor(rng.standard_normal((c2.shape[0], 64)).astype(
        np.float16)).to(dev)
    w2 = torch.as_tensor((rng.standard_normal((128, 2, 2, 2, 64))
                          * np.sqrt(2.0 / (8 * 64))).astype(np.float16)).to(dev)
    out['config2'] = layer(
        c2, f2, lambda x: ops.conv3d(x, w2, kernel_size=2, stride=2), 64, 128,
        8, 'conv3d k=2 s=2 fp16 64->128, 2 x ~100k LiDAR-like voxels',
        8 * 64 * 128 * 2)

    rng = config_rng(4)
    c4 = torch.as_tensor(sphere_shell_cloud(200000, 256, rng=rng)).to(dev)
    w4 = torch.as_tensor(kaiming_weight((64, 3, 3, 3, 64), rng=rng)).to(
        dev, torch.float16)
    f4 = torch.as_tensor(rng.standard_normal((c4.shape[0], 64)).astype(
        np.float16)).to(dev)
    q4 = quantize_weight(w4, group_size=32, bits=4)
    out['config4'] = layer(
        c4, f4, lambda x: ops.subm_conv3d(x, q4, kernel_size=3), 64, 64,
        27, 'QuantizedConv3d subm k=3 int4 g32 fp16 64->64, 200k sphere-shell '
        'voxels',
        # int4 codes + fp16 scales and biases per 32-channel group
        27 * 64 * 64 // 2 + 2 * 2 * 27 * (64 // 32) * 64)

    # Config 3 read literally: a uniform 400k subsample of the 200 complete
    # shells (about 2 active offsets per row, gather-bound).
    rng = config_rng(3)
    c3l = torch.as_tensor(sphere_shell_subsample_cloud(400000, 512,
                                                       rng=rng)).to(dev)
    f3l = torch.as_tensor(rng.standard_normal((c3l.shape[0], 128)).astype(
        np.float16)).to(dev)
    w3l = torch.as_tensor(kaiming_weight((128, 3, 3, 3, 128), rng=rng)).to(
        dev, torch.float16)
    out['config3_spec_literal'] = layer(
        c3l, f3l, lambda x: ops.subm_conv3d(x, w3l, kernel_size=3), 128, 128,
        27, 'subm_conv3d k=3 fp16 128->128, a uniform 400k subsample of the '
        'complete shells of 200 spheres in 512^3', 27 * 128 * 128 * 2)

    rng = config_rng(5)
    c5 = torch.as_tensor(lidar_cloud(120000, 4, rng=rng)).to(dev)
    f5 = torch.as_tensor(rng.random((c5.shape[0], 4)).astype(np.float16)).to(
        dev)
    mods = []
    for spec in encoder_layers(rng):
        c_out_l, *_, c_in_l = spec['weight'].shape
        if spec['kind'] == 'subm':
            dense = SubmConv3d(c_in_l, c_out_l, kernel_size=3, device=dev,
                               dtype=torch.float16)
            cls = QuantizedSubmConv3d
        else:
            dense = Conv3d(c_in_l, c_out_l, kernel_size=2, stride=2,
                           device=dev, dtype=torch.float16)
            cls = QuantizedConv3d
        dense.weight.data.copy_(torch.as_tensor(spec['weight']))
        dense.bias.data.copy_(torch.as_tensor(spec['bias']))
        mods.append(cls.from_conv(dense, group_size=32, bits=8))

    def encoder(x):
        # Each layer's bias and ReLU run in its conv kernel's store (the
        # result equals a separate bias add and maximum(feats, 0)).
        for mod in mods:
            x = mod(x, activation='relu')
        return x

    x5 = SparseTensor(c5, f5)
    encoder(x5)
    out['config5'] = {
        'workload': 'int8 g32 sparse encoder (stem subm 4->32, 3 x [k2s2 '
                    'down + 2 x subm], 32->64->128->256, bias + ReLU fused '
                    'into the conv store), '
                    f'4 x ~120k LiDAR-like voxels ({int(c5.shape[0])} rows)',
        'forward_ms': round(_timed(lambda: encoder(SparseTensor(c5, f5)),
                                   steps, warmup), 4),
        'forward_cached_maps_ms': round(_timed(lambda: encoder(x5), steps,
                                               warmup), 4),
    }
    return out


def backward_workload(feats, weight, coords, active, edges: int, steps: int,
                      warmup: int) -> dict:
    """Gradients of the config-3 conv (the reference primitive's vjp):
    the input gradient on the matrix cores over the forward's own sorted
    view with the mirrored transposed weight (a submanifold relation over
    distinct coordinates needs no transposed view), the weight gradient by
    the edge-balanced lock-step MFMA kernel."""
    import torch

    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd.ops._relation_exec import (
        sparse_conv_input_grad_from_relation,
        sparse_conv_weight_grad_from_relation,
    )

    x = SparseTensor(coords, feats)
    rel = x.coord_manager.submanifold_kernel_relation(x.coord_key,
                                                      kernel_size=3)
    n = int(coords.shape[0])
    gen = torch.Generator(device=feats.device).manual_seed(7)
    cot = torch.randn(feats.shape, generator=gen, device=feats.device,
                      dtype=torch.float32).to(feats.dtype)
    rel.kernel_csr  # grouped views, built once like the forward's views
    t_in = _timed(lambda: sparse_conv_input_grad_from_relation(
        cot, weight, rel, n), steps, warmup)
    t_w = _timed(lambda: sparse_conv_weight_grad_from_relation(
        feats, cot, weight, rel), steps, warmup)
    flops = 2.0 * edges * 128 * 128
    return {
        'workload': 'config3 gradients: input grad (matrix cores over the '
                    'forward sorted view, mirrored weight) and weight grad '
                    '(edge-balanced lock-step MFMA)',
        'input_grad_ms': round(t_in, 4),
        'input_grad_tflops': round(flops / t_in / 1e9, 2),
        'weight_grad_ms': round(t_w, 4),
        'weight_grad_tflops': round(flops / t_w / 1e9, 2),
    }


def pooling_workload(coords, steps: int, warmup: int) -> dict:
    """max_pool3d k=2 s=2 over the config-3 cloud with 64 fp32 channels
    (pooling is float32 only, as in the reference): the pooling kernel on a
    cached relation, against the HBM roofline of its algorithmic bytes
    (each input row read once, each output row written once, plus the CSR
    offsets and the edge rows)."""
    import torch

    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor

    n, c = int(coords.shape[0]), 64
    gen = torch.Generator(device=coords.device).manual_seed(11)
    feats = torch.randn((n, c), generator=gen, device=coords.device)
    x = SparseTensor(coords, feats)
    out = ops.max_pool3d(x, kernel_size=2, stride=2)
    torch.cuda.synchronize()
    rel = x.coord_manager.kernel_relation(x.coord_key, kernel_size=2,
                                          stride=2)
    n_out = int(rel.counts[1].item())
    e = int(rel.counts[0].item())
    t = _timed(lambda: ops.max_pool3d(x, kernel_size=2, stride=2), steps,
               warmup)
    bytes_ = n * c * 4 + out.feats.shape[0] * c * 4 + 4 * (n_out + 1) + 4 * e
    return {
        'workload': 'max_pool3d k=2 s=2, fp32 64 channels, config-3 cloud '
                    '(cached relation)',
        'rows_in': n, 'rows_out': n_out, 'ms': round(t, 4),
        'gbs': round(bytes_ / t / 1e6, 1),
        'hbm_frac': round(bytes_ / t / 1e6 / PEAK_HBM_GBS, 4),
    }


def decoder_workload(coords, steps: int, warmup: int) -> dict:
    """A decoder step on the config-3 cloud: the k=2 s=2 downsampled cloud
    (the encoder's next level) upsampled again by conv_transpose3d k=2 s=2,
    fp16 128 -> 128.  The transposed relation is direct (one output row per
    (row, offset)), so E = 8 * N_coarse and every output row has one edge.
    Reported: the relation build (HBM-bound: coords read, edges, offsets and
    output coordinates written); the conv on the dense expansion kernel,
    against the HBM roofline of its bytes (input rows read once, output
    written, weight); the generic matrix-core route over the same relation
    with its sorted view, for comparison; and the build of the
    deduplicating k=3 s=2 transposed relation."""
    import torch

    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd import SparseTensor
    from mlx_lattice_amd._native import ext
    from mlx_lattice_amd.ops._relation_exec import (
        sparse_conv_features_sorted_from_relation,
    )

    fine = SparseTensor(coords, torch.zeros((coords.shape[0], 1),
                                            device=coords.device))
    down = fine.coord_manager.kernel_relation(fine.coord_key, kernel_size=2,
                                              stride=2)
    n = int(down.counts[1].item())
    coarse = down.out_coords[:n].contiguous()
    active = torch.tensor([n], dtype=torch.int32, device=coords.device)
    c = 128
    gen = torch.Generator(device=coords.device).manual_seed(13)
    feats = torch.randn((n, c), generator=gen, device=coords.device
                        ).to(torch.float16)
    weight = (torch.randn((c, 2, 2, 2, c), generator=gen,
                          device=coords.device) * (2.0 / (8 * c)) ** 0.5
              ).to(torch.float16)
    x = SparseTensor(coarse, feats, stride=2)
    out = ops.conv_transpose3d(x, weight, kernel_size=2, stride=2)
    torch.cuda.synchronize()
    rel = x.coord_manager.transposed_kernel_relation(
        x.coord_key, kernel_size=2, stride=2)
    assert rel.direct_expansion and rel.sorted_implicit_gemm is None, \
        'the direct expansion route is expected'
    e = int(rel.counts[0].item())
    t_build = _timed(lambda: ext.build_transposed_kernel_relation_lazy(
        coarse, active, [2, 2, 2], [2, 2, 2], [0, 0, 0], [1, 1, 1]), steps, warmup)
    t_conv = _timed(lambda: ops.conv_transpose3d(x, weight, kernel_size=2,
                                                 stride=2), steps, warmup)
    # the generic matrix-core route over the same relation, for comparison
    t_view = _timed(lambda: (object.__setattr__(
        rel, 'sorted_implicit_gemm', None), object.__setattr__(
        rel, 'implicit_gemm', None), rel.require_sorted_implicit_gemm()),
        3, 1)
    t_generic = _timed(lambda: sparse_conv_features_sorted_from_relation(
        feats, weight, rel), steps, warmup)
    t_k3 = _timed(lambda: ext.build_transposed_kernel_relation_lazy(
        coarse, active, [3, 3, 3], [2, 2, 2], [0, 0, 0], [1, 1, 1]), steps, warmup)
    build_bytes = 16 * n + e * (12 + 4 + 16) + 4
    conv_bytes = n * c * 2 + e * c * 2 + 8 * c * c * 2
    flops = 2.0 * e * c * c
    del out
    return {
        'workload': 'config-3 decoder: conv_transpose3d k=2 s=2 fp16 '
                    '128->128 from the k2s2-downsampled cloud',
        'rows_in': n, 'rows_out': e,
        'relation_ms': round(t_build, 4),
        'relation_hbm_frac': round(build_bytes / t_build / 1e6 / PEAK_HBM_GBS,
                                   4),
        'conv_ms': round(t_conv, 4),
        'conv_tflops': round(flops / t_conv / 1e9, 2),
        'conv_hbm_frac': round(conv_bytes / t_conv / 1e6 / PEAK_HBM_GBS, 4),
        'generic_route_conv_ms': round(t_generic, 4),
        'generic_route_sorted_view_ms': round(t_view, 4),
        'k3s2_relation_ms': round(t_k3, 4),
    }


def quantization_workload(coords, steps: int, warmup: int) -> dict:
    """Point -> voxel quantization at the config-3 scale: 1M float32 points
    drawn inside the voxels of the config-3 cloud (2.5 points per voxel on
    average, unit voxels), then voxelize (mean, 64 fp32 channels) and
    devoxelize (trilinear map + interpolation, 64 channels).  All HBM-bound;
    each line reports its algorithmic bytes against 8 TB/s:
      quantize: points 12 B + batch 4 B read, keys 8 B written and read
        twice, inverse 4 B, counts 4 B per point; coords 16 B per voxel;
      voxelize: feats read, output written, the grouping read (4 B per
        point, 4 B per voxel);
      interpolate: 8 rows + 8 weights per point read, each distinct voxel
        row a corner names read once, output written (the minimum; the
        bytes of one read per (point, corner) are reported beside it as
        a diagnostic of the gather)."""
    import torch

    import mlx_lattice_amd.ops as ops
    from mlx_lattice_amd._native import ext

    dev = coords.device
    gen = torch.Generator(device=dev).manual_seed(17)
    n_vox = int(coords.shape[0])
    n = 1000000
    pick = torch.randint(0, n_vox, (n,), generator=gen, device=dev)
    base = coords[pick]
    pts = (base[:, 1:].float() + torch.rand((n, 3), generator=gen,
                                            device=dev)).contiguous()
    batches = base[:, 0].contiguous()
    active = torch.tensor([n], dtype=torch.int32, device=dev)
    q = ops.sparse_quantize(pts, 1.0, batch_indices=batches)
    v = int(q.active_rows.item())
    t_q = _timed(lambda: ext.sparse_quantize(pts, batches, active, [1.0],
                                             [0.0]),
                 steps, warmup)
    c = 64
    feats = torch.randn((n, c), generator=gen, device=dev)
    offsets, ids = q.voxel_groups(None)
    t_vox = _timed(lambda: ext.voxelize_features_grouped(
        feats, q.counts, offsets, ids, 'mean'), steps, warmup)
    t_group = _timed(lambda: ext.group_by_key(q.inverse_rows, None, n),
                     steps, warmup)
    vfeats = torch.randn((n, c), generator=gen, device=dev)
    pmap = ops.build_point_voxel_map(pts, q.coords, q.active_rows, 1.0,
                                     batch_indices=batches)
    t_map = _timed(lambda: ext.build_point_voxel_map(
        pts, batches, active, q.coords, q.active_rows, [1.0], [0.0],
        'linear'), steps, warmup)
    t_int = _timed(lambda: ext.interpolate_point_features(
        vfeats, pmap.rows, pmap.weights), steps, warmup)
    hbm = PEAK_HBM_GBS * 1e6
    b_q = n * (12 + 4 + 8 * 3 + 4 + 4) + v * 16
    b_vox = n * c * 4 + v * c * 4 + 4 * n + 4 * v
    found = pmap.rows[pmap.rows >= 0]
    corners = int(found.numel())
    distinct = int(torch.unique(found).numel())
    b_int = n * (32 + 32) + n * c * 4 + distinct * c * 4
    b_int_gather = n * (32 + 32) + n * c * 4 + corners * c * 4
    return {
        'workload': '1M points in the config-3 voxels (unit voxel): '
                    'sparse_quantize, voxelize mean 64 ch, trilinear '
                    'devoxelize 64 ch',
        'points': n, 'voxels': v,
        'quantize_ms': round(t_q, 4),
        'quantize_hbm_frac': round(b_q / t_q / hbm, 4),
        'group_ms': round(t_group, 4),
        'voxelize_ms': round(t_vox, 4),
        'voxelize_hbm_frac': round(b_vox / t_vox / hbm, 4),
        'corners_found': corners,
        'distinct_corner_rows': distinct,
        'point_map_ms': round(t_map, 4),
        'interpolate_ms': round(t_int, 4),
        'interpolate_hbm_frac': round(b_int / t_int / hbm, 4),
        'interpolate_per_corner_gbs': round(b_int_gather / t_int / 1e6, 1),
    }


def relation_bytes(n: int, edges: int) -> int:
    """Algorithmic HBM bytes of the submanifold relation (hash build + map:
    query, dense map, masks, edges, row offsets, counts), per unit:
      hash: 16 B coords read + 12 B per insert + 8 B per table slot cleared
        (capacity next_pow2(2N));
      map: 16 B coords + 12 B per probe (K per row) + 4 B per dense-map
        entry + 12 B per edge + 4 B per row offset + 8 B of counts."""
    cap = 1
    while cap < 2 * n:
        cap <<= 1
    k = 27
    b_hash = 16 * n + 12 * n + 8 * cap
    b_map = 16 * n + 12 * k * n + 4 * k * n + 12 * edges + 4 * (n + 1) + 8
    return b_hash + b_map


def sorted_view_bytes(n: int) -> int:
    """Algorithmic HBM bytes of the mask-sorted view: the stable sort of the
    row masks (a (key, index) pair, 8 B, read and written per row for each
    of its ceil(27 / 9) = 3 digit passes) and the gather (4 B order + 4 B
    mask + 4 K B map row read, 4 K B k-major map written per row, plus the
    tile quarter masks)."""
    k = 27
    return 3 * 16 * n + n * (8 + 8 * k) + 4 * ((n + 63) // 64) * 4


def hbm_roofline(nbytes: int, ms: float) -> dict:
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        'bytes': nbytes,
        'ms': round(ms, 4),
        'gbs': round(gbs, 1),
        'peak_gbs': PEAK_HBM_GBS,
        'frac': round(gbs / PEAK_HBM_GBS, 4),
    }


def conv_traffic():
    """CONV_TRAFFIC's bytes while csrc/conv.hip is the source they were
    measured on, else None."""
    import hashlib

    src = ROOT / 'mlx-lattice_amd' / 'csrc' / 'conv.hip'
    sha = hashlib.sha256(src.read_bytes()).hexdigest()[:16]
    if CONV_TRAFFIC['conv_hip_sha256'] != sha:
        return None, sha
    return CONV_TRAFFIC['bytes'], sha


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f'bench.py: --gpus {args.gpus} is not supported: this build '
              'measures one MI355X; the path shards by batch index with no '
              'exchange, so run one process per GPU.',
              file=sys.stderr)
        return 2
    import torch

    from mlx_lattice_amd._native import ext

    if args.phase == 'secondary':
        print(json.dumps({'secondary': secondary_workloads()}), flush=True)
        return 0
    coords_np, feats_np, weight_np = make_workload()
    dev = torch.device('cuda:0')
    coords = torch.as_tensor(coords_np).to(dev)
    feats = torch.as_tensor(feats_np).to(dev)
    weight = torch.as_tensor(weight_np).to(dev)
    active = torch.tensor([coords.shape[0]], dtype=torch.int32, device=dev)
    n_out = int(coords.shape[0])
    if args.phase == 'backward':
        native = ext.build_submanifold_kernel_relation_with_view(
            coords, active, [3, 3, 3], [1, 1, 1])
        edges = int(native[5][0].item())
        print(json.dumps({'backward': backward_workload(
            feats, weight, coords, active, edges, args.steps, args.warmup)}),
            flush=True)
        return 0
    if args.phase == 'widened':
        native = ext.build_submanifold_kernel_relation_with_view(
            coords, active, [3, 3, 3], [1, 1, 1])
        edges = int(native[5][0].item())
        print(json.dumps({
            'backward': backward_workload(feats, weight, coords, active,
                                          edges, args.steps, args.warmup),
            'pooling': pooling_workload(coords, args.steps, args.warmup),
            'decoder': decoder_workload(coords, args.steps, args.warmup),
            'quantization': quantization_workload(coords, args.steps,
                                                  args.warmup)}), flush=True)
        return 0

    def map_build():
        native = ext.build_submanifold_kernel_relation_with_view(
            coords, active, [3, 3, 3], [1, 1, 1])
        return native

    def sorted_view(native):
        # The sorted view with its tile order, as the operator path keeps
        # them (RelationSortedImplicitGemmView.tile_order): computed once per
        # view, reused by every conv over it.
        view = ext.build_sorted_implicit_gemm_view(native[10], native[11])
        return view + (ext.conv_tile_order(view[3], n_out),)

    # The weight in the streamed kernel's fragment order, made once per
    # weight as the operator path caches it (ops/_relation_exec.py
    # _weight_fragments), like the tile order per view.
    fragments = ext.conv_weight_fragments(weight)

    def conv(native, view):
        reorder, smap, kv, tiles, order = view
        return ext.sparse_conv_features_sorted_implicit_gemm(
            feats, weight, smap, kv, reorder, tiles, native[0], native[1],
            native[2], native[5], native[3], native[6], native[7], native[8],
            native[9], n_out, 27, tile_order=order,
            weight_fragments=fragments)

    for _ in range(args.warmup):
        native = map_build()
        view = sorted_view(native)
        out = conv(native, view)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)]
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record(stream)
        native = map_build()
        ev[i][1].record(stream)
        view = sorted_view(native)
        ev[i][2].record(stream)
        out = conv(native, view)
        ev[i][3].record(stream)
    torch.cuda.synchronize()
    t_wall = time.perf_counter() - t_wall

    rel_in_step_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps
    view_in_step_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / args.steps
    conv_in_step_ms = sum(e[2].elapsed_time(e[3]) for e in ev) / args.steps

    # The GEMM phase on its own: the same conv launched back to back over
    # the last step's resident map and view, so the interval holds the
    # kernels and not the host's launch gaps between the steps' phases.
    c0 = torch.cuda.Event(enable_timing=True)
    c1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    c0.record(stream)
    for _ in range(args.steps):
        out = conv(native, view)
    c1.record(stream)
    torch.cuda.synchronize()
    conv_ms = c0.elapsed_time(c1) / args.steps

    # The map-build phase on its own, like the GEMM phase above: the build
    # launched back to back, bracketed by one pair of events (each timing
    # event inside a step drains the queue before its timestamp, about
    # 5 us per event), then each of its two parts the same way.
    def back_to_back(fn):
        b0 = torch.cuda.Event(enable_timing=True)
        b1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        b0.record(stream)
        for _ in range(args.steps):
            fn()
        b1.record(stream)
        torch.cuda.synchronize()
        return b0.elapsed_time(b1) / args.steps

    map_ms = back_to_back(lambda: sorted_view(map_build()))
    rel_ms = back_to_back(map_build)
    view_ms = back_to_back(lambda: sorted_view(native))
    edges = int(native[5][0].item())
    flops = 2.0 * edges * 128 * 128
    conv_tflops = flops / (conv_ms * 1e-3) / 1e12
    traffic, conv_sha = conv_traffic()
    del out

    record = {
        'metric': 'subm_conv3d effective TFLOP/s + Mvoxels/s; kernel-map '
                  'build ms (1 MI355X)',
        'value': round(conv_tflops, 4),
        'unit': 'TFLOP/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(t_wall * 1e3 / args.steps, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f16',
        'data': 'synthetic',
        'config': {
            'workload': 'config3: subm_conv3d k=3 fp16 C_in=C_out=128, '
                        'batch 1, 400k voxels on 200 sphere shells in 512^3',
            'voxels': n_out,
            'edges': edges,
            'kernel_volume': 27,
            'c_in': 128,
            'c_out': 128,
        },
        'mvoxels_per_s': round(n_out / (conv_ms * 1e-3) / 1e6, 3),
        'kernel_map_build_ms': round(map_ms, 4),
        'kernel_map_build_in_step_ms': round(rel_in_step_ms + view_in_step_ms,
                                             4),
        # the whole map build (relation + sorted view), the interval of
        # kernel_map_build_ms, and its two parts
        'kernel_map_hbm': hbm_roofline(
            relation_bytes(n_out, edges) + sorted_view_bytes(n_out), map_ms),
        'relation_hbm': hbm_roofline(relation_bytes(n_out, edges), rel_ms),
        'sorted_view_hbm': hbm_roofline(sorted_view_bytes(n_out), view_ms),
        'relation_ms': round(rel_ms, 4),
        'sorted_view_ms': round(view_ms, 4),
        'conv_ms': round(conv_ms, 4),
        'conv_in_step_ms': round(conv_in_step_ms, 4),
        'roofline': {
            'bound': 'mfma',
            'achieved': round(conv_tflops, 4),
            'peak': PEAK_FP16_TFLOPS,
            'unit': 'TFLOP/s',
            'frac': round(conv_tflops / PEAK_FP16_TFLOPS, 5),
            'traffic': traffic,
            'traffic_source': ('rocprofv3 FETCH_SIZE + WRITE_SIZE, '
                               'profiles/config3_kernel_traffic.md'
                               if traffic is not None else
                               f'not measured for conv.hip {conv_sha}'),
            'kernel': 'conv_igemm_stream<f16, StreamShape<128, 1>, 2, 0>',
        },
    }
    if args.phase == 'config3':
        print(json.dumps(record), flush=True)
        return 0
    record['backward'] = backward_workload(feats, weight, coords, active,
                                           edges, args.steps, args.warmup)
    record['pooling'] = pooling_workload(coords, args.steps, args.warmup)
    record['decoder'] = decoder_workload(coords, args.steps, args.warmup)
    record['quantization'] = quantization_workload(coords, args.steps,
                                                   args.warmup)
    if not args.no_secondary:
        record['secondary'] = secondary_workloads()
    if not args.no_cpu_baseline:
        record['cpu_baseline'] = cpu_baseline(
            coords_np, feats_np, weight_np, args.cpu_threads,
            args.cpu_sample_rows)
    print(json.dumps(record), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
