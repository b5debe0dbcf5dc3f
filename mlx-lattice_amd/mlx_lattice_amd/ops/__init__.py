from mlx_lattice_amd.core.coords.builders import (
    build_relation_implicit_gemm_view,
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
from mlx_lattice_amd.ops.quantization import (
    build_point_voxel_map,
    devoxelize,
    interpolate_point_features,
    sparse_quantize,
    voxelize,
    voxelize_with_quantization,
)
from mlx_lattice_amd.ops.relations import (
    build_generative_relation,
    build_kernel_relation,
    build_submanifold_kernel_relation,
    build_target_kernel_relation,
    build_transposed_kernel_relation,
    generative_kernel_relation,
    kernel_offsets,
    kernel_relation,
    submanifold_kernel_relation,
    target_kernel_relation,
    transposed_kernel_relation,
)
from mlx_lattice_amd.ops.tensor import sparse_collate

__all__ = [
    'avg_pool3d',
    'build_generative_relation',
    'build_point_voxel_map',
    'build_kernel_relation',
    'build_relation_implicit_gemm_view',
    'build_submanifold_kernel_relation',
    'build_target_kernel_relation',
    'build_transposed_kernel_relation',
    'conv3d',
    'conv_transpose3d',
    'devoxelize',
    'generative_conv_transpose3d',
    'generative_kernel_relation',
    'global_avg_pool',
    'global_max_pool',
    'global_sum_pool',
    'interpolate_point_features',
    'kernel_offsets',
    'kernel_relation',
    'max_pool3d',
    'pool3d',
    'sparse_collate',
    'sparse_quantize',
    'subm_conv3d',
    'submanifold_kernel_relation',
    'sum_pool3d',
    'target_kernel_relation',
    'transposed_kernel_relation',
    'voxelize',
    'voxelize_with_quantization',
]
