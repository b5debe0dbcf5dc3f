"""Seeded synthetic voxel clouds for the five benchmark workloads.

Every generator returns ``(N, 4)`` int32 coordinates ``(batch, x, y, z)``,
deduplicated and then shuffled with the same seeded generator, because row
order matters for the first-seen semantics of the relation builders
(native/features/coordinates/cpu/quantization_detail.h:12-31 keeps the first
occurrence of each downsampled cell).

Seeds are ``0x1a771ce + config_index`` with ``numpy.random.Generator(PCG64)``.
Nothing here touches a GPU; the arrays are plain numpy.
"""

from __future__ import annotations

import numpy as np

SEED_BASE = 0x1A771CE

__all__ = [
    'SEED_BASE',
    'config_rng',
    'uniform_grid_cloud',
    'lidar_cloud',
    'sphere_shell_cloud',
    'sphere_shell_subsample_cloud',
    'kaiming_weight',
    'encoder_layers',
    'unique_rows_first_seen',
]


def config_rng(config_index: int) -> np.random.Generator:
    """Generator for BASELINE config ``config_index`` (1-based)."""
    return np.random.Generator(np.random.PCG64(SEED_BASE + config_index))


def unique_rows_first_seen(coords: np.ndarray) -> np.ndarray:
    """Drop duplicate rows, keeping each row's first occurrence in order."""
    if coords.shape[0] == 0:
        return coords
    _, first = np.unique(coords, axis=0, return_index=True)
    return coords[np.sort(first)]


def _finish(coords: np.ndarray, rng: np.random.Generator,
            shuffle: bool) -> np.ndarray:
    coords = unique_rows_first_seen(coords.astype(np.int32))
    if shuffle:
        coords = coords[rng.permutation(coords.shape[0])]
    return np.ascontiguousarray(coords, dtype=np.int32)


def uniform_grid_cloud(rows: int, grid: int, *, batch: int = 0,
                       rng: np.random.Generator,
                       shuffle: bool = True) -> np.ndarray:
    """``rows`` distinct voxels drawn without replacement from ``grid**3``."""
    flat = rng.choice(grid ** 3, size=rows, replace=False)
    x, rem = np.divmod(flat, grid * grid)
    y, z = np.divmod(rem, grid)
    coords = np.stack([np.full_like(x, batch), x, y, z], axis=1)
    return _finish(coords, rng, shuffle)


def _box_surface(rng: np.random.Generator, extent: tuple[int, int, int],
                 ) -> np.ndarray:
    sx, sy, sz = (int(v) for v in rng.integers(10, 81, size=3))
    sz = min(sz, extent[2])
    ox = int(rng.integers(0, extent[0] - sx))
    oy = int(rng.integers(0, extent[1] - sy))
    oz = int(rng.integers(0, max(extent[2] - sz, 0) + 1))
    gx, gy, gz = np.meshgrid(np.arange(sx), np.arange(sy), np.arange(sz),
                             indexing='ij')
    shell = ((gx == 0) | (gx == sx - 1) | (gy == 0) | (gy == sy - 1)
             | (gz == 0) | (gz == sz - 1))
    pts = np.stack([gx[shell] + ox, gy[shell] + oy, gz[shell] + oz], axis=1)
    return pts


def lidar_cloud(rows_per_batch: int, batches: int, *,
                rng: np.random.Generator,
                extent: tuple[int, int, int] = (1440, 1440, 40),
                shuffle: bool = True) -> np.ndarray:
    """LiDAR-like layout: 60% ground slab with density ~1/r, 40% box surfaces.

    The ground slab occupies ``z in [0, 3)``; ``r = R*u`` with ``u ~ U(0,1)``
    and a uniform angle gives an areal density proportional to ``1/r``.
    The remaining voxels lie on the surfaces of 30 axis-aligned boxes with
    sides drawn from ``U[10, 80]``.  Each batch is deduplicated on its own and
    the whole cloud is shuffled once.
    """
    out = []
    cx, cy = extent[0] / 2.0, extent[1] / 2.0
    radius = min(cx, cy) - 1.0
    for b in range(batches):
        ground_target = int(round(rows_per_batch * 0.6))
        box_target = rows_per_batch - ground_target
        boxes = np.concatenate([_box_surface(rng, extent) for _ in range(30)])
        boxes = unique_rows_first_seen(boxes)
        if boxes.shape[0] > box_target:
            boxes = boxes[rng.choice(boxes.shape[0], box_target,
                                     replace=False)]
        ground_parts = []
        have = 0
        while have < ground_target:
            draw = (ground_target - have) * 2 + 1024
            r = radius * rng.random(draw)
            theta = 2.0 * np.pi * rng.random(draw)
            x = np.floor(cx + r * np.cos(theta)).astype(np.int64)
            y = np.floor(cy + r * np.sin(theta)).astype(np.int64)
            z = rng.integers(0, 3, size=draw)
            pts = np.stack([x, y, z], axis=1)
            ground_parts.append(pts)
            merged = unique_rows_first_seen(np.concatenate(ground_parts))
            ground_parts = [merged]
            have = merged.shape[0]
        ground = ground_parts[0][:ground_target]
        pts = np.concatenate([ground, boxes])
        pts = unique_rows_first_seen(pts)
        out.append(np.concatenate(
            [np.full((pts.shape[0], 1), b, dtype=np.int64), pts], axis=1))
    return _finish(np.concatenate(out), rng, shuffle)


def sphere_shell_cloud(rows: int, grid: int, *, spheres: int = 200,
                       rng: np.random.Generator,
                       r_range: tuple[float, float] = (8.0, 60.0),
                       shuffle: bool = True) -> np.ndarray:
    """Voxels on 1-voxel-thick shells ``|‖p-c‖-r| < 0.5`` of random spheres.

    Complete spheres are taken in seeded order until ``rows`` distinct voxels
    are collected; the last sphere is truncated so ``N == rows`` exactly
    (shell density is preserved, so the average active-offset count per row
    stays that of a surface).
    """
    collected = np.zeros((0, 3), dtype=np.int64)
    seen: set[int] = set()
    parts = []
    total = 0
    for _ in range(spheres * 50):
        r = rng.uniform(*r_range)
        margin = int(np.ceil(r)) + 1
        c = rng.uniform(margin, grid - margin, size=3)
        lo = np.floor(c - r - 1).astype(np.int64)
        hi = np.ceil(c + r + 1).astype(np.int64)
        gx, gy, gz = np.meshgrid(np.arange(lo[0], hi[0] + 1),
                                 np.arange(lo[1], hi[1] + 1),
                                 np.arange(lo[2], hi[2] + 1), indexing='ij')
        d = np.sqrt((gx + 0.5 - c[0]) ** 2 + (gy + 0.5 - c[1]) ** 2
                    + (gz + 0.5 - c[2]) ** 2)
        shell = np.abs(d - r) < 0.5
        pts = np.stack([gx[shell], gy[shell], gz[shell]], axis=1)
        keys = (pts[:, 0] * grid + pts[:, 1]) * grid + pts[:, 2]
        fresh = np.array([k not in seen for k in keys.tolist()], dtype=bool)
        pts = pts[fresh]
        keys = keys[fresh]
        seen.update(keys.tolist())
        if total + pts.shape[0] >= rows:
            pts = pts[: rows - total]
            parts.append(pts)
            total += pts.shape[0]
            break
        parts.append(pts)
        total += pts.shape[0]
    collected = np.concatenate(parts) if parts else collected
    coords = np.concatenate(
        [np.zeros((collected.shape[0], 1), dtype=np.int64), collected], axis=1)
    return _finish(coords, rng, shuffle)


def _shell_voxels(c: np.ndarray, r: float) -> np.ndarray:
    """Voxels of the 1-voxel-thick shell ``|‖p + 0.5 - c‖ - r| < 0.5``."""
    lo = np.floor(c - r - 1).astype(np.int64)
    hi = np.ceil(c + r + 1).astype(np.int64)
    gx, gy, gz = np.meshgrid(np.arange(lo[0], hi[0] + 1),
                             np.arange(lo[1], hi[1] + 1),
                             np.arange(lo[2], hi[2] + 1), indexing='ij')
    d = np.sqrt((gx + 0.5 - c[0]) ** 2 + (gy + 0.5 - c[1]) ** 2
                + (gz + 0.5 - c[2]) ** 2)
    shell = np.abs(d - r) < 0.5
    return np.stack([gx[shell], gy[shell], gz[shell]], axis=1)


def sphere_shell_subsample_cloud(rows: int, grid: int, *, spheres: int = 200,
                                 rng: np.random.Generator,
                                 r_range: tuple[float, float] = (8.0, 60.0),
                                 ) -> np.ndarray:
    """The literal reading of the config-3 text: the complete shells of
    ``spheres`` random spheres (about 3.5M distinct voxels for 200 spheres
    of radius U[8, 60] in 512^3), then ``rows`` of them drawn uniformly
    without replacement and shuffled.  About 11% of each voxel's
    neighbours survive, so a row has about 2 active offsets and the conv is
    gather-bound (the truncated ``sphere_shell_cloud`` keeps whole spheres
    instead, about 10.6 offsets per row)."""
    parts = []
    for _ in range(spheres):
        r = rng.uniform(*r_range)
        margin = int(np.ceil(r)) + 1
        c = rng.uniform(margin, grid - margin, size=3)
        parts.append(_shell_voxels(c, r))
    pts = np.unique(np.concatenate(parts), axis=0)
    pick = rng.choice(pts.shape[0], size=min(rows, pts.shape[0]),
                      replace=False)
    pts = pts[np.sort(pick)]
    coords = np.concatenate(
        [np.zeros((pts.shape[0], 1), dtype=np.int64), pts], axis=1)
    return _finish(coords, rng, True)


def kaiming_weight(shape: tuple[int, ...], *, rng: np.random.Generator,
                   ) -> np.ndarray:
    """Kaiming-normal ``(C_out, Kx, Ky, Kz, C_in)`` weight, fan_in = K*C_in."""
    fan_in = int(np.prod(shape[1:]))
    return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(
        np.float32)


def encoder_layers(rng: np.random.Generator, *, in_channels: int = 4,
                   widths: tuple[int, ...] = (32, 64, 128, 256),
                   ) -> list[dict]:
    """Layer list of the config-5 int8 sparse encoder, as plain numpy.

    Stem: submanifold k=3, ``in_channels -> widths[0]``.  Each following
    stage: a k=2 stride-2 downsample to the next width, then two submanifold
    k=3 convs at that width.  Weights are Kaiming-normal float32 in the
    ``(C_out, Kx, Ky, Kz, C_in)`` layout; ``bias`` stands for a BatchNorm
    folded into the conv (shift ~ N(0, 0.1^2)), and every layer is followed
    by ReLU.  Quantization is left to the caller.
    """
    layers = []

    def add(kind: str, c_in: int, c_out: int) -> None:
        k = 3 if kind == 'subm' else 2
        layers.append(dict(
            kind=kind, kernel_size=k, stride=1 if kind == 'subm' else 2,
            weight=kaiming_weight((c_out, k, k, k, c_in), rng=rng),
            bias=(0.1 * rng.standard_normal(c_out)).astype(np.float32)))

    add('subm', in_channels, widths[0])
    for c_prev, c_next in zip(widths[:-1], widths[1:]):
        add('down', c_prev, c_next)
        add('subm', c_next, c_next)
        add('subm', c_next, c_next)
    return layers
