"""Packed affine INT4/INT8 weights (mlx_lattice/core/quantized.py:21-279).

Layout contract (kept identical to the reference):

* codes are packed LSB-first along C_in into ``uint32`` words:
  ``q(ci) = (word[ci * bits // 32] >> (ci * bits % 32)) & (2**bits - 1)``
  (native/features/convolution/cpu/quantized.cpp:54-62);
* spatial weights are stored ``weight (K, C_store * bits / 32, C_out)`` and
  ``scales / biases (K, C_store / group_size, C_out)`` in the weight dtype
  (quantized.py:164-177); pointwise weights keep ``(C_out, words)`` /
  ``(C_out, groups)`` per kernel row;
* the logical value is ``scale * q + bias`` and C_in is zero-padded in
  storage to a multiple of ``group_size``.

The quantiser itself is this build's own documented affine min/max rule
(the reference delegates it to ``mx.quantize`` of MLX, which is not available
here): per group, ``bias = min(w)``, ``scale = (max(w) - min(w)) /
(2**bits - 1)`` rounded to the weight dtype, ``q = clip(round((w - bias) /
scale), 0, 2**bits - 1)``.  Codes therefore differ from MLX's; the
convolution contract (packed conv == float conv of ``dequantize_weight``)
is what the kernels are held to.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import numpy as np
import torch

from mlx_lattice_amd.core.types import Triple

QuantizedWeightLayout = Literal['linear', 'kernel_major', 'dense_5d']

__all__ = [
    'QuantizedWeight',
    'QuantizedWeightLayout',
    'dequantize_weight',
    'quantize_weight',
]


@dataclass(frozen=True, slots=True)
class QuantizedWeight:
    """Packed affine INT4/INT8 inference weight (quantized.py:21-121)."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    group_size: int
    bits: int
    in_channels: int
    out_channels: int
    kernel_size: Triple
    layout: QuantizedWeightLayout

    def __post_init__(self) -> None:
        if self.bits not in (4, 8):
            raise ValueError('quantized weight bits must be 4 or 8.')
        if self.group_size not in (32, 64, 128):
            raise ValueError(
                'quantized weight group_size must be 32, 64, or 128.')
        if self.weight.dtype != torch.uint32 or self.weight.ndim != 3:
            raise ValueError(
                'packed weight must be a three-dimensional uint32 array.')
        if self.scales.dtype not in (torch.float16, torch.float32,
                                     torch.bfloat16):
            raise ValueError('quantized scales must be float16 or float32.')
        if self.biases.dtype != self.scales.dtype:
            raise ValueError('quantized biases must match scales dtype.')
        if self.scales.ndim != 3 or self.biases.shape != self.scales.shape:
            raise ValueError('scales and biases must have shape (K, C_out, G).')
        if self.in_channels <= 0 or self.out_channels <= 0:
            raise ValueError('quantized weight channels must be positive.')
        if any(size <= 0 for size in self.kernel_size):
            raise ValueError(
                'quantized weight kernel dimensions must be positive.')
        kernel_rows = _volume(self.kernel_size)
        if self.weight.shape[0] != kernel_rows:
            raise ValueError(
                'packed weight kernel rows do not match kernel_size.')
        if self.is_pointwise:
            if self.weight.shape[1] != self.out_channels:
                raise ValueError(
                    'pointwise packed weight output channels do not match.')
            if self.scales.shape[:2] != self.weight.shape[:2]:
                raise ValueError(
                    'pointwise weight and quantization rows must match.')
        else:
            if self.weight.shape[2] != self.out_channels:
                raise ValueError(
                    'spatial packed weight output channels do not match.')
            if (self.scales.shape[0] != self.weight.shape[0]
                    or self.scales.shape[2] != self.out_channels):
                raise ValueError(
                    'spatial weight and quantization rows must match.')
        if self.storage_in_channels % self.group_size != 0:
            raise ValueError(
                'packed storage channels must be divisible by group_size.')
        group_dim = 2 if self.is_pointwise else 1
        if (self.scales.shape[group_dim]
                != self.storage_in_channels // self.group_size):
            raise ValueError('quantization group count does not match storage.')
        if self.storage_in_channels < self.in_channels:
            raise ValueError('packed storage channels cannot be smaller than '
                             'logical channels.')

    @property
    def storage_in_channels(self) -> int:
        packed_dim = 2 if self.is_pointwise else 1
        return int(self.weight.shape[packed_dim]) * 32 // self.bits

    @property
    def is_pointwise(self) -> bool:
        return _volume(self.kernel_size) == 1

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size()
                   for t in (self.weight, self.scales, self.biases))

    def to(self, device: torch.device | str) -> QuantizedWeight:
        return QuantizedWeight(
            self.weight.to(device), self.scales.to(device),
            self.biases.to(device), self.group_size, self.bits,
            self.in_channels, self.out_channels, self.kernel_size, self.layout)


def quantize_weight(weight: torch.Tensor, *, group_size: int | None = None,
                    bits: int = 4) -> QuantizedWeight:
    """Pack a linear or sparse-convolution weight (quantized.py:125-188).

    Accepts ``(C_out, C_in)``, ``(K, C_in, C_out)`` or
    ``(C_out, Kx, Ky, Kz, C_in)`` float16/float32 weights.  ``group_size``
    ``None`` picks 64 for ``C_in >= 64`` else 32.
    """
    if weight.dtype not in (torch.float16, torch.float32, torch.bfloat16):
        raise ValueError('weight quantization supports float16 and float32.')
    if bits not in (4, 8):
        raise ValueError('weight quantization supports only 4 or 8 bits.')
    rows, layout, kernel_size, in_channels, out_channels = _weight_rows(weight)
    group_size = _resolve_group_size(in_channels, group_size)
    storage = _round_up(in_channels, group_size)
    dtype = weight.dtype
    device = weight.device
    values = rows.detach().to('cpu', torch.float32).numpy()
    if storage != in_channels:
        values = np.pad(values, [(0, 0), (0, storage - in_channels)])
    packed, scales, biases = _affine_quantize(values, group_size, bits, dtype)
    kernel_rows = _volume(kernel_size)
    packed = packed.reshape(kernel_rows, out_channels, -1)
    scales = scales.reshape(kernel_rows, out_channels, -1)
    biases = biases.reshape(kernel_rows, out_channels, -1)
    if kernel_rows > 1:
        packed = np.ascontiguousarray(packed.transpose(0, 2, 1))
        scales = np.ascontiguousarray(scales.transpose(0, 2, 1))
        biases = np.ascontiguousarray(biases.transpose(0, 2, 1))
    return QuantizedWeight(
        weight=torch.from_numpy(packed).to(device),
        scales=torch.from_numpy(scales).to(device=device, dtype=dtype),
        biases=torch.from_numpy(biases).to(device=device, dtype=dtype),
        group_size=group_size, bits=bits, in_channels=in_channels,
        out_channels=out_channels, kernel_size=kernel_size, layout=layout)


def dequantize_weight(weight: QuantizedWeight) -> torch.Tensor:
    """Logical float weight in the recorded layout (quantized.py:191-223)."""
    kernel_rows = _volume(weight.kernel_size)
    packed = weight.weight.cpu().numpy()
    scales = weight.scales.detach().to('cpu', torch.float32).numpy()
    biases = weight.biases.detach().to('cpu', torch.float32).numpy()
    if not weight.is_pointwise:
        packed = packed.transpose(0, 2, 1)
        scales = scales.transpose(0, 2, 1)
        biases = biases.transpose(0, 2, 1)
    n = kernel_rows * weight.out_channels
    codes = _unpack_codes(packed.reshape(n, -1), weight.bits)
    groups = np.arange(codes.shape[1]) // weight.group_size
    rows = (codes.astype(np.float32) * scales.reshape(n, -1)[:, groups]
            + biases.reshape(n, -1)[:, groups])[:, :weight.in_channels]
    out = torch.from_numpy(np.ascontiguousarray(rows)).to(
        device=weight.scales.device, dtype=weight.scales.dtype)
    if weight.layout == 'linear':
        return out.reshape(weight.out_channels, weight.in_channels)
    mapped = out.reshape(kernel_rows, weight.out_channels, weight.in_channels)
    if weight.layout == 'kernel_major':
        return mapped.permute(0, 2, 1).contiguous()
    return mapped.reshape(*weight.kernel_size, weight.out_channels,
                          weight.in_channels).permute(3, 0, 1, 2, 4).contiguous()


# ---------------------------------------------------------------- helpers --


def _affine_quantize(values: np.ndarray, group_size: int, bits: int,
                     dtype: torch.dtype):
    n, c = values.shape
    levels = (1 << bits) - 1
    grouped = values.reshape(n, c // group_size, group_size)
    w_min = grouped.min(axis=2)
    w_max = grouped.max(axis=2)
    scale = (w_max - w_min) / levels
    scale = np.where(scale > 0, scale, 1.0).astype(np.float32)
    # Round the affine parameters to the storage dtype first so the codes
    # are chosen against the values the kernels will actually use.
    scale_t = torch.from_numpy(scale).to(dtype).to(torch.float32).numpy()
    bias_t = torch.from_numpy(w_min.astype(np.float32)).to(dtype).to(
        torch.float32).numpy()
    scale_t = np.where(scale_t > 0, scale_t, 1.0).astype(np.float32)
    q = np.rint((grouped - bias_t[..., None]) / scale_t[..., None])
    q = np.clip(q, 0, levels).astype(np.uint32).reshape(n, c)
    per_word = 32 // bits
    q = q.reshape(n, c // per_word, per_word)
    shifts = (np.arange(per_word, dtype=np.uint32) * bits)[None, None, :]
    words = np.bitwise_or.reduce(q << shifts, axis=2).astype(np.uint32)
    return words, scale_t, bias_t


def _unpack_codes(words: np.ndarray, bits: int) -> np.ndarray:
    per_word = 32 // bits
    shifts = (np.arange(per_word, dtype=np.uint32) * bits)[None, None, :]
    codes = (words[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return codes.reshape(words.shape[0], -1)


def _weight_rows(weight: torch.Tensor):
    if weight.ndim == 2:
        out_channels, in_channels = map(int, weight.shape)
        return weight, 'linear', (1, 1, 1), in_channels, out_channels
    if weight.ndim == 3:
        kernel_rows, in_channels, out_channels = map(int, weight.shape)
        return (weight.permute(0, 2, 1).reshape(kernel_rows * out_channels,
                                                in_channels),
                'kernel_major', (kernel_rows, 1, 1), in_channels, out_channels)
    if weight.ndim == 5:
        out_channels, kx, ky, kz, in_channels = map(int, weight.shape)
        return (weight.permute(1, 2, 3, 0, 4).reshape(
            kx * ky * kz * out_channels, in_channels),
            'dense_5d', (kx, ky, kz), in_channels, out_channels)
    raise ValueError('weight must have shape (C_out, C_in), (K, C_in, C_out), '
                     'or (C_out, Kx, Ky, Kz, C_in).')


def _resolve_group_size(in_channels: int, group_size: int | None) -> int:
    if group_size is None:
        return 64 if in_channels >= 64 else 32
    if group_size not in (32, 64, 128):
        raise ValueError('group_size must be 32, 64, or 128.')
    return group_size


def _round_up(value: int, multiple: int) -> int:
    return ((value + multiple - 1) // multiple) * multiple


def _volume(size: Triple) -> int:
    return size[0] * size[1] * size[2]
