from mlx_lattice_amd.nn.conv import (
    Conv3d,
    ConvTranspose3d,
    GenerativeConvTranspose3d,
    SubmConv3d,
)
from mlx_lattice_amd.nn.quantized_conv import (
    QuantizedConv3d,
    QuantizedConvTranspose3d,
    QuantizedGenerativeConvTranspose3d,
    QuantizedSubmConv3d,
)

__all__ = [
    'Conv3d',
    'ConvTranspose3d',
    'GenerativeConvTranspose3d',
    'QuantizedConv3d',
    'QuantizedConvTranspose3d',
    'QuantizedGenerativeConvTranspose3d',
    'QuantizedSubmConv3d',
    'SubmConv3d',
]
