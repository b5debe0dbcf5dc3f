"""Sparse convolution operators (mlx_lattice/ops/conv.py:34-493).

``conv3d`` / ``subm_conv3d`` / ``conv_transpose3d`` /
``generative_conv_transpose3d`` keep the reference signatures, validation
messages and coordinate-identity rules.  Relations come from the coordinate
manager's cache and run on the gfx950 kernels.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from mlx_lattice_amd.core import (
    CoordinateMapKey,
    KernelSpec,
    QuantizedWeight,
    SparseTensor,
    dequantize_weight,
)
from mlx_lattice_amd.core.types import Triple
from mlx_lattice_amd.ops._relation_exec import (
    sparse_conv_features_from_relation,
    sparse_quantized_conv_features_from_relation,
)

__all__ = [
    'conv3d',
    'conv_transpose3d',
    'generative_conv_transpose3d',
    'subm_conv3d',
]

_FEATURE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def conv3d(x: SparseTensor, weight: torch.Tensor | QuantizedWeight,
           bias: torch.Tensor | None = None, *,
           kernel_size: int | Sequence[int] = 3,
           stride: int | Sequence[int] = 1,
           padding: int | Sequence[int] = 0,
           dilation: int | Sequence[int] = 1,
           coordinates: SparseTensor | CoordinateMapKey | torch.Tensor | None
           = None,
           activation: str | None = None) -> SparseTensor:
    """Sparse 3D convolution (ops/conv.py:34-109).

    The pointwise 1x1x1 case without ``coordinates`` is a feature matmul that
    keeps the input coordinates.  Otherwise a forward relation (or a target
    relation when ``coordinates`` is given) is built or reused and the
    features run through the native kernels.  Output stride is
    ``x.stride * stride``.

    ``activation='relu'`` (not in the reference signature) applies the
    reference's ``relu`` (``maximum(feats, 0)``, ops/feature.py:54-56) to the
    result, fused into the conv kernels' store when autograd does not need
    it; the result equals ``relu(conv3d(...))`` bit for bit.
    """
    spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                      dilation=dilation)
    output_stride = _mul_stride(x.stride, spec.stride)
    relu = _relu_requested(activation)
    if coordinates is None and spec.is_pointwise:
        return x.replace(feats=_activate(
            _with_bias(_pointwise_features(x, weight), bias), relu))
    if coordinates is not None:
        target_key = _target_key(x, coordinates, output_stride)
        reuse_input = target_key == x.coord_key
        return _relation_conv(
            x, _target_weight(weight, spec), bias, spec,
            map_kind='forward' if reuse_input else 'target',
            output_stride=target_key.stride, reuse_input_coords=reuse_input,
            target_key=target_key, relu=relu)
    return _relation_conv(x, weight, bias, spec, map_kind='forward',
                          output_stride=output_stride, relu=relu)


def subm_conv3d(x: SparseTensor, weight: torch.Tensor | QuantizedWeight,
                bias: torch.Tensor | None = None, *,
                kernel_size: int | Sequence[int] = 3,
                dilation: int | Sequence[int] = 1,
                activation: str | None = None) -> SparseTensor:
    """Submanifold sparse convolution: odd kernel, stride 1, output reuses
    the input coordinate identity (ops/conv.py:112-150).  ``activation`` as
    for ``conv3d``."""
    spec = KernelSpec(size=kernel_size, stride=1, padding=0,
                      dilation=dilation)
    _require_odd_kernel(spec.size, 'subm_conv3d')
    relu = _relu_requested(activation)
    if spec.size == (1, 1, 1) and spec.dilation == (1, 1, 1):
        return x.replace(feats=_activate(
            _with_bias(_pointwise_features(x, weight), bias), relu))
    return _relation_conv(x, weight, bias, spec, map_kind='submanifold',
                          output_stride=x.stride, reuse_input_coords=True,
                          relu=relu)


def conv_transpose3d(x: SparseTensor, weight, bias=None, *, kernel_size=2,
                     stride=2, padding=0, dilation=1,
                     activation: str | None = None) -> SparseTensor:
    """Sparse transposed convolution over the transposed relation
    (ops/conv.py:153-186).  The output stride is ``x.stride / stride``; each
    component of ``stride`` must divide the input stride.  ``activation``
    as for ``conv3d``."""
    spec = KernelSpec(size=kernel_size, stride=stride, padding=padding,
                      dilation=dilation)
    return _relation_conv(x, weight, bias, spec, map_kind='transposed',
                          output_stride=_div_stride(x.stride, spec.stride),
                          relu=_relu_requested(activation))


def generative_conv_transpose3d(x: SparseTensor, weight, bias=None, *,
                                kernel_size=2, stride=2,
                                activation: str | None = None) -> SparseTensor:
    """Transposed convolution whose output support is generated from every
    input row and offset (ops/conv.py:189-214): output row ``in * K + k``
    at ``coord * stride + offset[k]``.  ``activation`` as for ``conv3d``."""
    spec = KernelSpec(size=kernel_size, stride=stride)
    return _relation_conv(x, weight, bias, spec, map_kind='generative',
                          output_stride=_div_stride(x.stride, spec.stride),
                          relu=_relu_requested(activation))


# ------------------------------------------------------ execution policy --


def _relation_conv(x: SparseTensor, weight, bias, spec: KernelSpec, *,
                   map_kind: str, output_stride: Triple,
                   reuse_input_coords: bool = False,
                   target_key: CoordinateMapKey | None = None,
                   relu: bool = False) -> SparseTensor:
    _validate_feature_dtype(x.feats, weight)
    _validate_gpu_coord_dtype(x)
    _validate_weight_for_kernel(x, weight, spec.volume)
    relation = _kernel_relation(x, spec, map_kind, target_key=target_key)
    if relation.n_out_capacity is None or relation.n_kernels is None:
        raise ValueError('kernel relation is missing static shape metadata.')
    # The bias is added in the conv kernels' store (after rounding, as a
    # separate add would) unless autograd must see the add.
    fuse = bias is not None and not (
        torch.is_grad_enabled() and bias.requires_grad)
    fused = bias if fuse else None
    # The ReLU joins the store when nothing needs its gradient and the bias
    # (which comes first) is fused or absent.
    needs_grad = torch.is_grad_enabled() and (
        x.feats.requires_grad
        or (isinstance(weight, torch.Tensor) and weight.requires_grad)
        or (bias is not None and bias.requires_grad))
    fuse_relu = relu and not needs_grad and (bias is None or fuse)
    feats = (sparse_quantized_conv_features_from_relation(
                 x.feats, weight, relation, fused, relu=fuse_relu)
             if isinstance(weight, QuantizedWeight)
             else sparse_conv_features_from_relation(
                 x.feats, weight, relation, fused, relu=fuse_relu))
    if not fuse:
        feats = _with_bias(feats, bias)
    if relu and not fuse_relu:
        feats = _activate(feats, True)
    if reuse_input_coords:
        return x.replace(feats=feats)
    if relation.out_coords is None:
        raise ValueError('kernel relation is missing output coordinates.')
    if target_key is not None and map_kind == 'target':
        return SparseTensor(
            x.coord_manager.coords(target_key), feats,
            stride=output_stride, coord_key=target_key,
            coord_manager=x.coord_manager,
            active_rows=x.coord_manager.active_rows(target_key))
    return SparseTensor(relation.out_coords, feats,
                        stride=output_stride, coord_manager=x.coord_manager,
                        active_rows=relation.out_count)


def _kernel_relation(x: SparseTensor, spec: KernelSpec, map_kind: str, *,
                     target_key: CoordinateMapKey | None = None):
    manager = x.coord_manager
    if map_kind == 'forward':
        return manager.kernel_relation(
            x.coord_key, kernel_size=spec.size, stride=spec.stride,
            padding=spec.padding, dilation=spec.dilation)
    if map_kind == 'submanifold':
        return manager.submanifold_kernel_relation(
            x.coord_key, kernel_size=spec.size, dilation=spec.dilation)
    if map_kind == 'transposed':
        return manager.transposed_kernel_relation(
            x.coord_key, kernel_size=spec.size, stride=spec.stride,
            padding=spec.padding, dilation=spec.dilation)
    if map_kind == 'generative':
        return manager.generative_relation(
            x.coord_key, kernel_size=spec.size, stride=spec.stride)
    if map_kind == 'target':
        if target_key is None:
            raise ValueError('target_key is required for target relations.')
        return manager.target_kernel_relation(
            x.coord_key, target_key, kernel_size=spec.size,
            stride=spec.stride, padding=spec.padding, dilation=spec.dilation)
    raise ValueError(
        "map_kind must be 'forward', 'submanifold', 'transposed', "
        "'generative', or 'target'.")


def _target_key(x: SparseTensor, coordinates, output_stride: Triple,
                ) -> CoordinateMapKey:
    if isinstance(coordinates, SparseTensor):
        if coordinates.stride != output_stride:
            raise ValueError(
                'target coordinates must use the convolution output stride.')
        if coordinates.coord_manager is x.coord_manager:
            return coordinates.coord_key
        return x.coord_manager.insert_coords(
            coordinates.coords, coordinates.stride, coordinates.active_rows)
    if isinstance(coordinates, CoordinateMapKey):
        if not x.coord_manager.owns(coordinates):
            raise ValueError(
                'target coordinate key must belong to x.coord_manager.')
        if coordinates.stride != output_stride:
            raise ValueError('target coordinate key must use the convolution '
                             'output stride.')
        return coordinates
    return x.coord_manager.insert_coords(coordinates, output_stride)


def _pointwise_features(x: SparseTensor, weight) -> torch.Tensor:
    _validate_feature_dtype(x.feats, weight)
    if isinstance(weight, QuantizedWeight):
        matrix = dequantize_weight(weight).to(x.feats.device)
        if matrix.ndim == 5:
            matrix = matrix[:, 0, 0, 0, :]
        elif matrix.ndim == 3:
            matrix = matrix[0].T
        return x.feats @ matrix.T
    return x.feats @ _pointwise_weight_matrix(x, weight).T


def _target_weight(weight, spec: KernelSpec):
    if isinstance(weight, QuantizedWeight):
        return weight
    if not spec.is_pointwise or weight.ndim != 2:
        return weight
    return weight.T.unsqueeze(0)


# -------------------------------------------------------------- validation --


def _validate_feature_dtype(feats: torch.Tensor, weight) -> None:
    if feats.dtype not in _FEATURE_DTYPES:
        raise ValueError('convolution supports float32 and float16 tensors.')
    weight_dtype = (weight.scales.dtype if isinstance(weight, QuantizedWeight)
                    else weight.dtype)
    if weight_dtype != feats.dtype:
        raise ValueError('convolution weights must match feature dtype.')


def _validate_gpu_coord_dtype(x: SparseTensor) -> None:
    if x.coords.dtype != torch.int32:
        raise ValueError('GPU sparse convolution requires int32 coordinates.')


def _pointwise_weight_matrix(x: SparseTensor, weight: torch.Tensor):
    if weight.ndim == 2:
        if weight.shape[1] != x.channels:
            raise ValueError('weight input channels must match x.channels.')
        return weight
    if (weight.ndim == 5 and weight.shape[1] == 1 and weight.shape[2] == 1
            and weight.shape[3] == 1):
        if weight.shape[4] != x.channels:
            raise ValueError('weight input channels must match x.channels.')
        return weight[:, 0, 0, 0, :]
    if weight.ndim == 3 and weight.shape[0] == 1:
        if weight.shape[1] != x.channels:
            raise ValueError('weight input channels must match x.channels.')
        return weight[0].T
    raise ValueError('pointwise weight must have shape (C_out, C_in), '
                     '(C_out, 1, 1, 1, C_in), or (1, C_in, C_out).')


def _validate_weight_for_kernel(x: SparseTensor, weight,
                                kernel_rows: int) -> None:
    if isinstance(weight, QuantizedWeight):
        if weight.in_channels != x.channels:
            raise ValueError(
                'quantized weight input channels must match x.channels.')
        if _volume(weight.kernel_size) != kernel_rows:
            raise ValueError('quantized weight kernel rows must match the '
                             'convolution kernel.')
        return
    if weight.ndim == 3:
        if weight.shape[1] != x.channels:
            raise ValueError('weight input channels must match x.channels.')
        if weight.shape[0] != kernel_rows:
            raise ValueError(
                'weight kernel rows must match the convolution kernel.')
        return
    if weight.ndim != 5:
        raise ValueError('mapped convolution weight must have shape '
                         '(K, C_in, C_out) or (C_out, Kx, Ky, Kz, C_in).')
    if weight.shape[4] != x.channels:
        raise ValueError('weight input channels must match x.channels.')
    if int(weight.shape[1] * weight.shape[2] * weight.shape[3]) != kernel_rows:
        raise ValueError(
            'weight kernel rows must match the convolution kernel.')


def _relu_requested(activation: str | None) -> bool:
    if activation is None:
        return False
    if activation != 'relu':
        raise ValueError("activation must be None or 'relu'.")
    return True


def _activate(feats: torch.Tensor, relu: bool) -> torch.Tensor:
    """The reference's ``relu`` (``maximum(feats, 0)``, ops/feature.py:54-56):
    v where v > 0 or v is NaN, +0 otherwise (the fused store's rule)."""
    if not relu:
        return feats
    keep = (feats > 0) | torch.isnan(feats)
    return torch.where(keep, feats, torch.zeros((), dtype=feats.dtype,
                                                device=feats.device))


def _with_bias(feats: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    if bias is None:
        return feats
    if bias.ndim != 1:
        raise ValueError('bias must have shape (C_out,).')
    if bias.shape[0] != feats.shape[1]:
        raise ValueError('bias channels must match output channels.')
    if bias.dtype != feats.dtype:
        raise ValueError('bias dtype must match output features.')
    return feats + bias


def _require_odd_kernel(values: Triple, op_name: str) -> None:
    if any(value % 2 == 0 for value in values):
        raise ValueError(f'{op_name} requires odd kernel_size values.')


def _mul_stride(lhs: Triple, rhs: Triple) -> Triple:
    return (lhs[0] * rhs[0], lhs[1] * rhs[1], lhs[2] * rhs[2])


def _div_stride(lhs: Triple, rhs: Triple) -> Triple:
    out = []
    for left, right in zip(lhs, rhs, strict=True):
        if left % right != 0:
            raise ValueError(
                'transpose stride must divide the input tensor stride.')
        out.append(left // right)
    return (out[0], out[1], out[2])


def _volume(size: Triple) -> int:
    return size[0] * size[1] * size[2]
