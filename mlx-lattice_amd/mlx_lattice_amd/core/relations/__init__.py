from mlx_lattice_amd.core.relations.specs import KernelSpec
from mlx_lattice_amd.core.relations.views import (
    KernelRelation,
    RelationCSRView,
    RelationEdges,
    RelationImplicitGemmView,
    RelationSortedImplicitGemmView,
    RelationView,
    SparseRelationContract,
)

__all__ = [
    'KernelRelation',
    'KernelSpec',
    'RelationCSRView',
    'RelationEdges',
    'RelationImplicitGemmView',
    'RelationSortedImplicitGemmView',
    'RelationView',
    'SparseRelationContract',
]
