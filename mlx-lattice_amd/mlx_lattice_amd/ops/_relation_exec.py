"""Dispatch of a prebuilt relation to the native conv kernels
(mlx_lattice/ops/_relation_exec.py:19-250).

Route policy (this build's, the reference routes by Metal capability):
fp16/bf16 features with ``C_in % 32 == 0``, ``C_out`` in {16, 32, 64, 128,
256} and at most 32 kernel offsets run the matrix-core implicit GEMM over the
mask-sorted view, for every relation kind whose edges fit the dense
(out_row, offset) map; everything else (fp32, small or odd channel counts)
runs the CSR bandwidth kernel.  Both routes compute the same sum with an fp32
accumulator.
"""

from __future__ import annotations

import weakref

import torch

from mlx_lattice_amd._native import ext
from mlx_lattice_amd.core.quantized import QuantizedWeight
from mlx_lattice_amd.core.relations import KernelRelation

_MATRIX_CORE_C_OUT = (16, 32, 64, 128, 256)
# (id(weight), kind) -> (weak reference, shape, dtype, version, value)
_WEIGHT_CACHE: dict[tuple[int, str], tuple[weakref.ReferenceType, tuple,
                                           torch.dtype, int, torch.Tensor]] = {}


def _empty_i32(device) -> torch.Tensor:
    return torch.empty(0, dtype=torch.int32, device=device)


def _require_static(relation: KernelRelation) -> None:
    if relation.n_out_capacity is None or relation.n_kernels is None:
        raise ValueError('kernel relation is missing static shape metadata.')


def _matrix_core_eligible(dtype: torch.dtype, c_in: int, c_out: int,
                          relation: KernelRelation, n_in: int = 0) -> bool:
    """Shapes the matrix-core kernel takes; its 32-bit gather offsets need
    the feature table under 2 GiB.  The relation must fit the dense
    (out_row, offset) map: a transposed relation with a repeated input
    coordinate runs the CSR route."""
    return (relation.dense_map_exact
            and dtype in (torch.float16, torch.bfloat16)
            and c_in % 32 == 0 and c_in <= 512
            and c_out in _MATRIX_CORE_C_OUT
            and relation.n_kernels is not None and relation.n_kernels <= 32
            and n_in * c_in * 2 < 2 ** 31)


def _small_dense_map(dtype: torch.dtype, c_in: int, c_out: int,
                     relation: KernelRelation) -> torch.Tensor | None:
    """The relation's dense map for the dense-map conv of few input
    channels (C_in 4 or 8, C_out 16 or 32, fp16/bf16), when the relation
    already holds it: the native CSR entry then contracts a row's whole
    neighbourhood on the matrix cores instead of walking its edges."""
    view = relation.implicit_gemm
    if (view is None or dtype not in (torch.float16, torch.bfloat16)
            or c_in not in (4, 8) or c_out not in (16, 32)
            or relation.n_kernels is None or relation.n_kernels * c_in > 256
            or view.out_in_map.dtype != torch.int32
            or tuple(view.out_in_map.shape) != (relation.n_out_capacity,
                                                relation.n_kernels)
            or not relation.dense_map_exact):
        return None
    return view.out_in_map


_EXPAND_CHANNELS = (32, 64, 128, 256)


def _expand_eligible(feats: torch.Tensor, c_out: int,
                     relation: KernelRelation) -> bool:
    """A direct expanded relation (output row in * K + k = the single edge
    (in, k)) runs as a dense matrix-core GEMM without gathers."""
    return (relation.direct_expansion
            and relation.contract.source_active_rows is not None
            and feats.dtype in (torch.float16, torch.bfloat16)
            and int(feats.shape[1]) in _EXPAND_CHANNELS
            and c_out in _EXPAND_CHANNELS
            and int(feats.shape[1]) * c_out <= 16384
            and relation.n_in_capacity == int(feats.shape[0])
            and relation.n_out_capacity
            == int(feats.shape[0]) * int(relation.n_kernels))


def sparse_conv_features_from_relation(feats: torch.Tensor,
                                       weight: torch.Tensor,
                                       relation: KernelRelation,
                                       bias: torch.Tensor | None = None,
                                       relu: bool = False,
                                       ) -> torch.Tensor:
    """Execute sparse convolution over a prebuilt relation
    (_relation_exec.py:84-116).  Differentiable in ``feats`` and ``weight``:
    the backward pass is the reference primitive's vjp
    (native/features/convolution/primitive.cpp:137-176).  ``relu`` fuses a
    ReLU after the bias into the store (the operators pass it only when
    autograd does not need the activation)."""
    _require_static(relation)
    if torch.is_grad_enabled() and (feats.requires_grad
                                    or weight.requires_grad
                                    or (bias is not None
                                        and bias.requires_grad)):
        if relu:
            raise ValueError('a fused ReLU is not differentiable; apply it '
                             'separately when gradients are needed.')
        out = _SparseConvFeatures.apply(feats, weight, relation)
        return out if bias is None else _add_bias(out, bias)
    return _conv_features(feats, weight, relation, bias, relu)


def _add_bias(feats: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    if bias.ndim != 1:
        raise ValueError('bias must have shape (C_out,).')
    if bias.shape[0] != feats.shape[1]:
        raise ValueError('bias channels must match output channels.')
    if bias.dtype != feats.dtype:
        raise ValueError('bias dtype must match output features.')
    return feats + bias


class _SparseConvFeatures(torch.autograd.Function):
    """Sparse conv features with the reference's gradients: the input
    gradient over the input-grouped CSR and the weight gradient over the
    kernel-grouped CSR (cpu/algorithms.cpp:355-481)."""

    @staticmethod
    def forward(ctx, feats, weight, relation):
        ctx.relation = relation
        ctx.save_for_backward(feats, weight)
        return _conv_features(feats, weight, relation)

    @staticmethod
    def backward(ctx, grad_out):
        feats, weight = ctx.saved_tensors
        relation = ctx.relation
        grad_out = grad_out.contiguous()
        grad_feats = grad_weight = None
        if ctx.needs_input_grad[0]:
            grad_feats = sparse_conv_input_grad_from_relation(
                grad_out, weight, relation, int(feats.shape[0]))
        if ctx.needs_input_grad[1]:
            grad_weight = sparse_conv_weight_grad_from_relation(
                feats, grad_out, weight, relation)
        return grad_feats, grad_weight, None


def _input_grad_matrix_core_eligible(cot: torch.Tensor, weight: torch.Tensor,
                                     relation: KernelRelation) -> bool:
    """The input gradient is the forward's implicit GEMM over the
    transposed relation: its contraction runs over C_out and it writes C_in
    columns."""
    c_in = int(weight.shape[1] if weight.ndim == 3 else weight.shape[4])
    c_out = int(cot.shape[1])
    return (relation.contract.kind != 'target'
            and cot.dtype in (torch.float16, torch.bfloat16)
            and c_out % 32 == 0 and c_out <= 512
            and c_in in _MATRIX_CORE_C_OUT
            and relation.n_kernels is not None and relation.n_kernels <= 32
            and int(cot.shape[0]) * c_out * 2 < 2 ** 31
            # a repeated coordinate gives an input row several output rows
            # at one offset, which the dense transposed map cannot hold
            and relation.transposed_map_exact)


def _transposed_weight(weight: torch.Tensor) -> torch.Tensor:
    """(C_out, Kx, Ky, Kz, C_in) or (K, C_in, C_out) -> the 5D weight of the
    transposed conv, (C_in, Kx, Ky, Kz, C_out) (cached)."""
    def make(w):
        if w.ndim == 5:
            return w.permute(4, 1, 2, 3, 0).contiguous()
        k, c_in, c_out = w.shape
        return w.permute(1, 0, 2).contiguous().reshape(c_in, k, 1, 1, c_out)

    return _cached_weight(weight, 'transposed', make)


def _mirrored_weight(weight: torch.Tensor) -> torch.Tensor:
    """The transposed weight with its offsets reversed, W'[j] = W[K-1-j]^T,
    as a 5D (C_in, Kx, Ky, Kz, C_out) weight (cached)."""
    def make(w):
        if w.ndim == 5:
            return w.flip(1, 2, 3).permute(4, 1, 2, 3, 0).contiguous()
        k, c_in, c_out = w.shape
        return w.flip(0).permute(1, 0, 2).contiguous().reshape(
            c_in, k, 1, 1, c_out)

    return _cached_weight(weight, 'mirrored', make)


def _mirror_symmetric(relation: KernelRelation) -> bool:
    """A submanifold relation whose offsets come in opposite pairs,
    offset[K-1-k] = -offset[k] (odd kernels), and whose coordinates do not
    repeat: input row i then meets output row o at offset k exactly when
    o = out_in_map[i][K-1-k], so the transposed map is the forward map with
    its offsets reversed."""
    if relation.contract.kind != 'submanifold':
        return False
    offs = relation.contract.kernel_offsets
    k = len(offs)
    return k > 0 and all(
        tuple(-v for v in offs[k - 1 - j]) == tuple(offs[j]) for j in range(k))


def sparse_conv_input_grad_from_relation(cot: torch.Tensor,
                                         weight: torch.Tensor,
                                         relation: KernelRelation,
                                         in_capacity: int) -> torch.Tensor:
    """Input gradient ``(in_capacity, C_in)`` (make_sparse_conv_features_
    input_grad, primitive.cpp:597-639): on the matrix cores when the shapes
    allow, otherwise over the input-grouped CSR.  A submanifold relation
    over distinct coordinates runs the forward's own sorted view with the
    mirrored transposed weight (grad[i] = sum_j cot[out_in_map[i][j]] @
    W[K-1-j]^T); other relations run their transposed sorted view."""
    _require_static(relation)
    if _input_grad_matrix_core_eligible(cot, weight, relation):
        if _mirror_symmetric(relation):
            view = relation.require_sorted_implicit_gemm()
            mirrored = _mirrored_weight(weight)
            return ext.sparse_conv_features_sorted_implicit_gemm(
                cot, mirrored, view.sorted_out_in_map,
                view.sorted_kv_out_in_map, view.reorder_rows, view.tile_masks,
                None, None, None, None, None, None, None, None, None,
                in_capacity, relation.n_kernels, tile_order=view.tile_order(),
                weight_fragments=_weight_fragments(mirrored))
        view = relation.require_transposed_sorted_implicit_gemm()
        transposed = _transposed_weight(weight)
        return ext.sparse_conv_features_sorted_implicit_gemm(
            cot, transposed, view.sorted_out_in_map,
            view.sorted_kv_out_in_map, view.reorder_rows, view.tile_masks,
            None, None, None, None, None, None, None, None, None,
            in_capacity, relation.n_kernels, tile_order=view.tile_order(),
            weight_fragments=_weight_fragments(transposed))
    input_csr = relation.input_csr
    return ext.sparse_conv_input_grad(
        cot, weight, relation.edges.out_rows, relation.edges.kernel_ids,
        relation.counts, input_csr.row_offsets, input_csr.edge_ids,
        in_capacity, relation.n_kernels)


def sparse_conv_weight_grad_from_relation(feats: torch.Tensor,
                                          cot: torch.Tensor,
                                          weight: torch.Tensor,
                                          relation: KernelRelation,
                                          ) -> torch.Tensor:
    """Weight gradient in ``weight``'s shape (make_sparse_conv_features_
    weight_grad, primitive.cpp:641-680) over the kernel-grouped CSR."""
    _require_static(relation)
    kernel_csr = relation.kernel_csr
    return ext.sparse_conv_weight_grad(
        feats, cot, weight, relation.edges.in_rows, relation.edges.out_rows,
        relation.counts, kernel_csr.row_offsets, kernel_csr.edge_ids,
        relation.n_kernels)


def _conv_features(feats: torch.Tensor, weight: torch.Tensor,
                   relation: KernelRelation,
                   bias: torch.Tensor | None = None,
                   relu: bool = False) -> torch.Tensor:
    """Forward features on the matrix-core or the CSR route; ``bias``
    (optional) is added in the kernels' store, after the conv result is
    rounded, exactly as a separate ``feats + bias``; ``relu`` then applies
    ``maximum(v, 0)`` in the same store."""
    c_out = int(weight.shape[2] if weight.ndim == 3 else weight.shape[0])
    if feats.ndim == 2 and _expand_eligible(feats, c_out, relation):
        return ext.sparse_conv_features_expand(
            feats, weight, relation.contract.source_active_rows,
            relation.n_kernels, bias=bias, relu=relu)
    if feats.ndim == 2 and _matrix_core_eligible(
            feats.dtype, int(feats.shape[1]), c_out, relation,
            int(feats.shape[0])):
        return sparse_conv_features_sorted_from_relation(feats, weight,
                                                         relation, bias=bias,
                                                         relu=relu)
    dense = (_small_dense_map(feats.dtype, int(feats.shape[1]), c_out,
                              relation) if feats.ndim == 2 else None)
    return ext.sparse_conv_features_csr(
        feats, weight, relation.edges.in_rows, relation.edges.kernel_ids,
        relation.counts, relation.output_csr.row_offsets,
        relation.n_out_capacity, relation.n_kernels, bias=bias, relu=relu,
        out_in_map=dense)


def sparse_conv_features_sorted_from_relation(feats: torch.Tensor,
                                              weight: torch.Tensor,
                                              relation: KernelRelation, *,
                                              store_sorted: bool = False,
                                              bias: torch.Tensor | None = None,
                                              relu: bool = False,
                                              ) -> torch.Tensor:
    """Matrix-core implicit GEMM over the sorted view
    (_relation_exec.py:119-156)."""
    _require_static(relation)
    c_out = int(weight.shape[2] if weight.ndim == 3 else weight.shape[0])
    if not _matrix_core_eligible(feats.dtype, int(feats.shape[1]), c_out,
                                 relation, int(feats.shape[0])):
        raise ValueError(
            'sorted implicit GEMM is not supported for this relation, '
            'feature tensor, or weight tensor.')
    view = relation.require_sorted_implicit_gemm()
    w5 = _matrix_core_weight(weight)
    return ext.sparse_conv_features_sorted_implicit_gemm(
        feats, w5, view.sorted_out_in_map,
        view.sorted_kv_out_in_map, view.reorder_rows, view.tile_masks,
        relation.edges.in_rows, relation.edges.out_rows,
        relation.edges.kernel_ids, relation.counts,
        relation.output_csr.row_offsets, None, None, None, None,
        relation.n_out_capacity, relation.n_kernels,
        store_sorted=store_sorted, bias=bias, tile_order=view.tile_order(),
        relu=relu, weight_fragments=_weight_fragments(w5))


def sparse_quantized_conv_features_from_relation(
        feats: torch.Tensor, weight: QuantizedWeight,
        relation: KernelRelation,
        bias: torch.Tensor | None = None,
        relu: bool = False) -> torch.Tensor:
    """Quantized sparse convolution over a prebuilt relation
    (_relation_exec.py:19-61); the sorted plan is passed when the matrix-core
    route applies.  ``bias`` and ``relu`` are fused into the store."""
    _require_static(relation)
    if relation.n_kernels != weight.weight.shape[0]:
        raise ValueError('quantized weight kernel rows must match the relation.')
    device = feats.device
    kv = reorder = tiles = _empty_i32(device)
    order = None
    dense = None
    if _matrix_core_eligible(feats.dtype, weight.in_channels,
                             weight.out_channels, relation,
                             int(feats.shape[0])):
        view = relation.require_sorted_implicit_gemm()
        kv = view.sorted_kv_out_in_map
        reorder = view.reorder_rows
        tiles = view.tile_masks
        order = view.tile_order()
    else:
        dense = _small_dense_map(feats.dtype, weight.in_channels,
                                 weight.out_channels, relation)
    return ext.sparse_quantized_conv_features(
        feats, weight.weight, weight.scales, weight.biases,
        relation.edges.in_rows, relation.edges.out_rows,
        relation.edges.kernel_ids, relation.counts,
        relation.output_csr.row_offsets, kv, reorder, tiles,
        relation.n_out_capacity, relation.n_kernels, weight.in_channels,
        weight.out_channels, weight.storage_in_channels, weight.group_size,
        weight.bits, bias=bias, tile_order=order, relu=relu,
        weight_fragments=(_quantized_fragments(weight)
                          if order is not None else None),
        out_in_map=dense)


def sparse_pool_features_from_relation(feats: torch.Tensor,
                                       relation: KernelRelation, *,
                                       input_exclusive: bool,
                                       mode: str) -> torch.Tensor:
    """Sparse pooling over a prebuilt kernel relation
    (_relation_exec.py:253-276), differentiable in ``feats``."""
    _require_static(relation)
    if torch.is_grad_enabled() and feats.requires_grad:
        return _SparsePoolFeatures.apply(feats, relation, input_exclusive,
                                         mode)
    return _pool_features(feats, relation, input_exclusive, mode)


def _pool_features(feats, relation, input_exclusive, mode):
    return ext.sparse_pool_features(
        feats, relation.edges.in_rows, relation.edges.out_rows,
        relation.edges.kernel_ids, relation.output_csr.row_offsets,
        relation.counts, input_exclusive, mode, relation.n_out_capacity,
        relation.n_kernels)


class _SparsePoolFeatures(torch.autograd.Function):
    """Pooling with the reference's vjp (pooling/primitive.cpp:109-160):
    the gradient walks the input-grouped CSR; max routes the cotangent to
    the inputs equal to the pooled value, split over ties."""

    @staticmethod
    def forward(ctx, feats, relation, input_exclusive, mode):
        pooled = _pool_features(feats, relation, input_exclusive, mode)
        ctx.relation = relation
        ctx.mode = mode
        ctx.save_for_backward(feats, pooled)
        return pooled

    @staticmethod
    def backward(ctx, grad_out):
        feats, pooled = ctx.saved_tensors
        relation = ctx.relation
        input_csr = relation.input_csr
        grad = ext.sparse_pool_features_grad(
            grad_out.contiguous(), feats, pooled, relation.edges.in_rows,
            relation.edges.out_rows, relation.output_csr.row_offsets,
            relation.counts, input_csr.row_offsets, input_csr.edge_ids,
            ctx.mode)
        return grad, None, None, None


def _cached_weight(weight: torch.Tensor, kind: str, make) -> torch.Tensor:
    """``make(weight)``, cached by the weight's identity, shape, dtype and
    version counter (so an in-place update, as an optimizer step makes,
    rebuilds it), like the reference's ``_mapped_weight``
    (_relation_exec.py:217-250)."""
    key = (id(weight), kind)
    shape = tuple(weight.shape)
    cached = _WEIGHT_CACHE.get(key)
    if cached is not None:
        ref, cached_shape, cached_dtype, version, value = cached
        if (ref() is weight and cached_shape == shape
                and cached_dtype == weight.dtype
                and version == weight._version):
            return value
    value = make(weight)

    def _drop(ref, key=key):
        entry = _WEIGHT_CACHE.get(key)
        if entry is not None and entry[0] is ref:
            _WEIGHT_CACHE.pop(key, None)

    _WEIGHT_CACHE[key] = (weakref.ref(weight, _drop), shape, weight.dtype,
                          weight._version, value)
    return value


def _weight_fragments(weight5d: torch.Tensor) -> torch.Tensor:
    """The streamed matrix-core conv's fragment-ordered copy of a 5D
    fp16/bf16 weight (``ext.conv_weight_fragments``; empty when the shape
    takes the other matrix-core kernel), cached with the weight."""
    return _cached_weight(weight5d, 'fragments', ext.conv_weight_fragments)


def _quantized_fragments(weight: QuantizedWeight) -> torch.Tensor:
    """The streamed matrix-core conv's fragment-ordered packed copy of a
    quantized weight (``ext.quantized_weight_fragments``: codes, scale and
    bias per 16-byte piece, dequantised in the kernel; empty when the shape
    takes the other matrix-core kernel), cached with the packed words and
    rebuilt when they, the scales or the biases change."""
    kind = ('quantized fragments', id(weight.scales), weight.scales._version,
            id(weight.biases), weight.biases._version)

    def make(words):
        return ext.quantized_weight_fragments(
            words, weight.scales, weight.biases, weight.in_channels,
            weight.out_channels, weight.storage_in_channels,
            weight.group_size, weight.bits)

    return _cached_weight(weight.weight, kind, make)


def _matrix_core_weight(weight: torch.Tensor) -> torch.Tensor:
    """5D weights go to the kernels as they are (C_in contiguous per
    (C_out, k)); a mapped ``(K, C_in, C_out)`` weight is transposed once to
    ``(C_out, K, 1, 1, C_in)`` and cached."""
    if weight.ndim == 5:
        return weight

    def make(w):
        k, c_in, c_out = w.shape
        return w.permute(2, 0, 1).contiguous().reshape(c_out, k, 1, 1, c_in)

    return _cached_weight(weight, 'mapped', make)
