"""Parameter-owning sparse conv modules (mlx_lattice/nn/conv.py:49-323) as
``torch.nn.Module``s.  Weights use the reference layout
``(C_out, Kx, Ky, Kz, C_in)`` and the reference init
``U(-sqrt(1/(C_in*K)), +sqrt(1/(C_in*K)))`` with zero bias."""

from __future__ import annotations

import math
from collections.abc import Sequence

import torch
from torch import nn

from mlx_lattice_amd.core import CoordinateMapKey, KernelSpec, SparseTensor
from mlx_lattice_amd.ops import (
    conv3d,
    conv_transpose3d,
    generative_conv_transpose3d,
    subm_conv3d,
)

__all__ = ['Conv3d', 'ConvTranspose3d', 'GenerativeConvTranspose3d',
           'SubmConv3d']


class Conv3d(nn.Module):
    """Sparse 3D convolution delegating to :func:`conv3d`."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 3,
                 stride: int | Sequence[int] = 1,
                 padding: int | Sequence[int] = 0,
                 dilation: int | Sequence[int] = 1, bias: bool = True,
                 device=None, dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.spec = KernelSpec(size=kernel_size, stride=stride,
                               padding=padding, dilation=dilation)
        _init_kernel_params(self, in_channels, out_channels, self.spec, bias,
                            device, dtype)

    def forward(self, x: SparseTensor, *,
                coordinates: SparseTensor | CoordinateMapKey | torch.Tensor
                | None = None,
                activation: str | None = None) -> SparseTensor:
        return conv3d(x, self.weight, self.bias, kernel_size=self.spec.size,
                      stride=self.spec.stride, padding=self.spec.padding,
                      dilation=self.spec.dilation, coordinates=coordinates,
                      activation=activation)

    def to_quantized(self, group_size: int | None = None,
                     bits: int | None = None, *, mode: str = 'affine',
                     quantize_input: bool = False):
        from mlx_lattice_amd.nn.quantized_conv import QuantizedConv3d

        _validate_quantize_request(mode, quantize_input)
        return QuantizedConv3d.from_conv(self, group_size=group_size,
                                         bits=4 if bits is None else bits)


class SubmConv3d(nn.Module):
    """Submanifold sparse convolution delegating to :func:`subm_conv3d`."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 3,
                 dilation: int | Sequence[int] = 1, bias: bool = True,
                 device=None, dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.spec = KernelSpec(size=kernel_size, stride=1, padding=0,
                               dilation=dilation)
        _init_kernel_params(self, in_channels, out_channels, self.spec, bias,
                            device, dtype)

    def forward(self, x: SparseTensor, *,
                activation: str | None = None) -> SparseTensor:
        return subm_conv3d(x, self.weight, self.bias,
                           kernel_size=self.spec.size,
                           dilation=self.spec.dilation,
                           activation=activation)

    def to_quantized(self, group_size: int | None = None,
                     bits: int | None = None, *, mode: str = 'affine',
                     quantize_input: bool = False):
        from mlx_lattice_amd.nn.quantized_conv import QuantizedSubmConv3d

        _validate_quantize_request(mode, quantize_input)
        return QuantizedSubmConv3d.from_conv(self, group_size=group_size,
                                             bits=4 if bits is None else bits)


class ConvTranspose3d(nn.Module):
    """Sparse transposed convolution delegating to
    :func:`conv_transpose3d` (nn/conv.py:173-234)."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 2,
                 stride: int | Sequence[int] = 2,
                 padding: int | Sequence[int] = 0,
                 dilation: int | Sequence[int] = 1, bias: bool = True,
                 device=None, dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.spec = KernelSpec(size=kernel_size, stride=stride,
                               padding=padding, dilation=dilation)
        _init_kernel_params(self, in_channels, out_channels, self.spec, bias,
                            device, dtype)

    def forward(self, x: SparseTensor, *,
                activation: str | None = None) -> SparseTensor:
        return conv_transpose3d(x, self.weight, self.bias,
                                kernel_size=self.spec.size,
                                stride=self.spec.stride,
                                padding=self.spec.padding,
                                dilation=self.spec.dilation,
                                activation=activation)

    def to_quantized(self, group_size: int | None = None,
                     bits: int | None = None, *, mode: str = 'affine',
                     quantize_input: bool = False):
        from mlx_lattice_amd.nn.quantized_conv import QuantizedConvTranspose3d

        _validate_quantize_request(mode, quantize_input)
        return QuantizedConvTranspose3d.from_conv(
            self, group_size=group_size, bits=4 if bits is None else bits)


class GenerativeConvTranspose3d(nn.Module):
    """Generative transposed convolution delegating to
    :func:`generative_conv_transpose3d` (nn/conv.py:237-296)."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 2,
                 stride: int | Sequence[int] = 2, bias: bool = True,
                 device=None, dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self.spec = KernelSpec(size=kernel_size, stride=stride)
        _init_kernel_params(self, in_channels, out_channels, self.spec, bias,
                            device, dtype)

    def forward(self, x: SparseTensor, *,
                activation: str | None = None) -> SparseTensor:
        return generative_conv_transpose3d(x, self.weight, self.bias,
                                           kernel_size=self.spec.size,
                                           stride=self.spec.stride,
                                           activation=activation)

    def to_quantized(self, group_size: int | None = None,
                     bits: int | None = None, *, mode: str = 'affine',
                     quantize_input: bool = False):
        from mlx_lattice_amd.nn.quantized_conv import (
            QuantizedGenerativeConvTranspose3d,
        )

        _validate_quantize_request(mode, quantize_input)
        return QuantizedGenerativeConvTranspose3d.from_conv(
            self, group_size=group_size, bits=4 if bits is None else bits)


def _init_kernel_params(module: nn.Module, in_channels: int,
                        out_channels: int, spec: KernelSpec, bias: bool,
                        device, dtype: torch.dtype) -> None:
    scale = math.sqrt(1.0 / (in_channels * spec.volume))
    weight = torch.empty((out_channels, *spec.size, in_channels),
                         device=device, dtype=dtype).uniform_(-scale, scale)
    module.weight = nn.Parameter(weight, requires_grad=False)
    if bias:
        module.bias = nn.Parameter(
            torch.zeros(out_channels, device=device, dtype=dtype),
            requires_grad=False)
    else:
        module.bias = None


def _validate_quantize_request(mode: str, quantize_input: bool) -> None:
    if mode != 'affine':
        raise ValueError('quantized sparse convolution supports affine mode.')
    if quantize_input:
        raise ValueError(
            'quantized sparse convolution uses floating-point activations.')
