"""Affine weight-quantized sparse conv modules
(mlx_lattice/nn/quantized_conv.py:36-232)."""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import nn

from mlx_lattice_amd.core import (
    CoordinateMapKey,
    QuantizedWeight,
    SparseTensor,
    quantize_weight,
)
from mlx_lattice_amd.nn.conv import (
    Conv3d,
    ConvTranspose3d,
    GenerativeConvTranspose3d,
    SubmConv3d,
)
from mlx_lattice_amd.ops import (
    conv3d,
    conv_transpose3d,
    generative_conv_transpose3d,
    subm_conv3d,
)

__all__ = ['QuantizedConv3d', 'QuantizedConvTranspose3d',
           'QuantizedGenerativeConvTranspose3d', 'QuantizedSubmConv3d']


class _QuantizedConvBase(nn.Module):
    def _assign_quantized(self, weight: torch.Tensor, group_size: int | None,
                          bits: int) -> None:
        q = quantize_weight(weight, group_size=group_size, bits=bits)
        self.register_buffer('weight', q.weight, persistent=True)
        self.register_buffer('scales', q.scales, persistent=True)
        self.register_buffer('biases', q.biases, persistent=True)
        self.group_size = q.group_size
        self.bits = q.bits
        self.in_channels = q.in_channels
        self.out_channels = q.out_channels

    def _quantized_weight(self) -> QuantizedWeight:
        return QuantizedWeight(self.weight, self.scales, self.biases,
                               self.group_size, self.bits, self.in_channels,
                               self.out_channels, self.spec.size, 'dense_5d')

    def _copy_from(self, source: nn.Module, group_size: int | None,
                   bits: int) -> None:
        self.spec = source.spec
        self._assign_quantized(source.weight.detach(), group_size, bits)
        self.bias = (None if source.bias is None
                     else nn.Parameter(source.bias.detach().clone(),
                                       requires_grad=False))


class QuantizedConv3d(_QuantizedConvBase):
    """Packed int4/int8 ``Conv3d``; activations stay floating point."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 3,
                 stride: int | Sequence[int] = 1,
                 padding: int | Sequence[int] = 0,
                 dilation: int | Sequence[int] = 1, bias: bool = True,
                 group_size: int | None = None, bits: int = 4, device=None,
                 dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self._copy_from(Conv3d(in_channels, out_channels,
                               kernel_size=kernel_size, stride=stride,
                               padding=padding, dilation=dilation, bias=bias,
                               device=device, dtype=dtype), group_size, bits)

    def forward(self, x: SparseTensor, *,
                coordinates: SparseTensor | CoordinateMapKey | torch.Tensor
                | None = None,
                activation: str | None = None) -> SparseTensor:
        return conv3d(x, self._quantized_weight(), self.bias,
                      kernel_size=self.spec.size, stride=self.spec.stride,
                      padding=self.spec.padding, dilation=self.spec.dilation,
                      coordinates=coordinates, activation=activation)

    @classmethod
    def from_conv(cls, source: Conv3d, group_size: int | None = None,
                  bits: int = 4) -> QuantizedConv3d:
        out = cls.__new__(cls)
        _QuantizedConvBase.__init__(out)
        out._copy_from(source, group_size, bits)
        return out


class QuantizedSubmConv3d(_QuantizedConvBase):
    """Packed int4/int8 ``SubmConv3d``; coordinate identity preserved."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 3,
                 dilation: int | Sequence[int] = 1, bias: bool = True,
                 group_size: int | None = None, bits: int = 4, device=None,
                 dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self._copy_from(SubmConv3d(in_channels, out_channels,
                                   kernel_size=kernel_size, dilation=dilation,
                                   bias=bias, device=device, dtype=dtype),
                        group_size, bits)

    def forward(self, x: SparseTensor, *,
                activation: str | None = None) -> SparseTensor:
        return subm_conv3d(x, self._quantized_weight(), self.bias,
                           kernel_size=self.spec.size,
                           dilation=self.spec.dilation,
                           activation=activation)

    @classmethod
    def from_conv(cls, source: SubmConv3d, group_size: int | None = None,
                  bits: int = 4) -> QuantizedSubmConv3d:
        out = cls.__new__(cls)
        _QuantizedConvBase.__init__(out)
        out._copy_from(source, group_size, bits)
        return out


class QuantizedConvTranspose3d(_QuantizedConvBase):
    """Packed int4/int8 ``ConvTranspose3d`` (nn/quantized_conv.py:235-310)."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 2,
                 stride: int | Sequence[int] = 2,
                 padding: int | Sequence[int] = 0,
                 dilation: int | Sequence[int] = 1, bias: bool = True,
                 group_size: int | None = None, bits: int = 4, device=None,
                 dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self._copy_from(ConvTranspose3d(in_channels, out_channels,
                                        kernel_size=kernel_size,
                                        stride=stride, padding=padding,
                                        dilation=dilation, bias=bias,
                                        device=device, dtype=dtype),
                        group_size, bits)

    def forward(self, x: SparseTensor, *,
                activation: str | None = None) -> SparseTensor:
        return conv_transpose3d(x, self._quantized_weight(), self.bias,
                                kernel_size=self.spec.size,
                                stride=self.spec.stride,
                                padding=self.spec.padding,
                                dilation=self.spec.dilation,
                           activation=activation)

    @classmethod
    def from_conv(cls, source: ConvTranspose3d, group_size: int | None = None,
                  bits: int = 4) -> QuantizedConvTranspose3d:
        out = cls.__new__(cls)
        _QuantizedConvBase.__init__(out)
        out._copy_from(source, group_size, bits)
        return out


class QuantizedGenerativeConvTranspose3d(_QuantizedConvBase):
    """Packed int4/int8 ``GenerativeConvTranspose3d``
    (nn/quantized_conv.py:313-380)."""

    def __init__(self, in_channels: int, out_channels: int, *,
                 kernel_size: int | Sequence[int] = 2,
                 stride: int | Sequence[int] = 2, bias: bool = True,
                 group_size: int | None = None, bits: int = 4, device=None,
                 dtype: torch.dtype = torch.float32) -> None:
        super().__init__()
        self._copy_from(GenerativeConvTranspose3d(
            in_channels, out_channels, kernel_size=kernel_size,
            stride=stride, bias=bias, device=device, dtype=dtype),
            group_size, bits)

    def forward(self, x: SparseTensor, *,
                activation: str | None = None) -> SparseTensor:
        return generative_conv_transpose3d(x, self._quantized_weight(),
                                           self.bias,
                                           kernel_size=self.spec.size,
                                           stride=self.spec.stride,
                                           activation=activation)

    @classmethod
    def from_conv(cls, source: GenerativeConvTranspose3d,
                  group_size: int | None = None,
                  bits: int = 4) -> QuantizedGenerativeConvTranspose3d:
        out = cls.__new__(cls)
        _QuantizedConvBase.__init__(out)
        out._copy_from(source, group_size, bits)
        return out
