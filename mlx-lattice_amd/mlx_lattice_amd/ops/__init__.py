from mlx_lattice_amd.core.coords.builders import (
    build_kernel_relation,
    build_relation_implicit_gemm_view,
    build_submanifold_kernel_relation,
    build_target_kernel_relation,
    kernel_offsets,
)
from mlx_lattice_amd.ops.conv import (
    conv3d,
    conv_transpose3d,
    generative_conv_transpose3d,
    subm_conv3d,
)

__all__ = [
    'build_kernel_relation',
    'build_relation_implicit_gemm_view',
    'build_submanifold_kernel_relation',
    'build_target_kernel_relation',
    'conv3d',
    'conv_transpose3d',
    'generative_conv_transpose3d',
    'kernel_offsets',
    'subm_conv3d',
]
