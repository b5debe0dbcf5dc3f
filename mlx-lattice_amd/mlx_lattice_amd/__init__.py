"""MI355X-native sparse convolution hot path of mlx-lattice.

The operator API of the reference (``conv3d`` / ``subm_conv3d`` with an
optional ``coordinates`` target, ``QuantizedConv3d`` with packed affine
int4/int8 weights) over torch tensors, computed by gfx950 HIP kernels behind
the C ABI in ``include/lattice_hip.h``.
"""

from mlx_lattice_amd.core import (
    CoordinateManager,
    CoordinateMapKey,
    KernelRelation,
    KernelSpec,
    QuantizedWeight,
    SparseTensor,
    dequantize_weight,
    quantize_weight,
)

__version__ = '0.1.0'

__all__ = [
    'CoordinateManager',
    'CoordinateMapKey',
    'KernelRelation',
    'KernelSpec',
    'QuantizedWeight',
    'SparseTensor',
    'dequantize_weight',
    'quantize_weight',
]
