from mlx_lattice_amd.core.coords import CoordinateManager, CoordinateMapKey
from mlx_lattice_amd.core.coords.quantization import (
    PointVoxelMap,
    SparseQuantization,
)
from mlx_lattice_amd.core.quantized import (
    QuantizedWeight,
    dequantize_weight,
    quantize_weight,
)
from mlx_lattice_amd.core.relations import (
    KernelRelation,
    KernelSpec,
    RelationCSRView,
    RelationEdges,
    RelationImplicitGemmView,
    RelationSortedImplicitGemmView,
    SparseRelationContract,
)
from mlx_lattice_amd.core.tensor import SparseTensor

__all__ = [
    'CoordinateManager',
    'CoordinateMapKey',
    'KernelRelation',
    'KernelSpec',
    'PointVoxelMap',
    'QuantizedWeight',
    'RelationCSRView',
    'RelationEdges',
    'RelationImplicitGemmView',
    'RelationSortedImplicitGemmView',
    'SparseQuantization',
    'SparseRelationContract',
    'SparseTensor',
    'dequantize_weight',
    'quantize_weight',
]
