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
from mlx_lattice_amd.ops.pool import (
    avg_pool3d,
    global_avg_pool,
    global_max_pool,
    global_sum_pool,
    max_pool3d,
    pool3d,
    sum_pool3d,
)
from mlx_lattice_amd.ops.tensor import sparse_collate

__all__ = [
    'avg_pool3d',
    'build_kernel_relation',
    'build_relation_implicit_gemm_view',
    'build_submanifold_kernel_relation',
    'build_target_kernel_relation',
    'conv3d',
    'conv_transpose3d',
    'generative_conv_transpose3d',
    'global_avg_pool',
    'global_max_pool',
    'global_sum_pool',
    'kernel_offsets',
    'max_pool3d',
    'pool3d',
    'sparse_collate',
    'subm_conv3d',
    'sum_pool3d',
]
