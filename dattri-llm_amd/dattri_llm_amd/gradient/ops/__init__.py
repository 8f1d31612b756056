"""Layer-type-aware gradient operations on the MI355X kernels.

Same public names and signatures as ``dattri_llm.gradient.ops`` for the
scoring path (``dattri_llm/gradient/ops/__init__.py:123``): ``_factors``
functions take raw batch-first ``(activation, pre_activation_grad)``
tensors, the unsuffixed ones take :class:`Factorized` (or dense tensors).
"""

from dattri_llm_amd.gradient.ops import cost, dtypes, kronecker, moe
from dattri_llm_amd.gradient.ops.cost import CostModel, calibrate, get_routing_policy, set_routing_policy
from dattri_llm_amd.gradient.ops.dot import (
    block_grad_norm_sq,
    cross_dot,
    cross_dot_factors,
    cross_dot_per_token,
    cross_gram,
    cross_gram_per_token,
    cross_gram_per_token_dense,
    dot,
    dot_factors,
    effective_dims,
    grad_norm_sq,
    grad_norm_sq_factors,
    layerwise_cross_dot,
    layerwise_cross_dot_per_token,
    maybe_use_materialized_gram,
    maybe_use_materialized_norm,
    pairwise_dot,
    pairwise_dot_factors,
    route_flops,
)
from dattri_llm_amd.gradient.ops.dtypes import as_float, compute_dtype, get_compute_dtype, set_compute_dtype
from dattri_llm_amd.gradient.ops.kronecker import (
    FisherAccumulator,
    KroneckerAccumulator,
    LayerFisherAccumulator,
    LayerKroneckerAccumulator,
    dense_inverse,
    ekfac_materialize,
    ekfac_materialize_factors,
    ekfac_precondition,
    fim,
    fim_factors,
    kfac,
    kfac_cross,
    kfac_cross_factors,
    kfac_eigh,
    kfac_factors,
    kfac_precondition,
    kfac_precondition_materialized,
    sym_inverse,
)
from dattri_llm_amd.gradient.ops.materialize import (
    materialize,
    materialize_blocked,
    materialize_factors,
    materialize_group,
)
from dattri_llm_amd.gradient.ops.preprocess import (
    extract_module_kwargs,
    preprocess_factorized,
    preprocess_factors,
    to_3d,
)
from dattri_llm_amd.gradient.ops.projection import (
    CAPTURE_STYLES,
    MASK_KEYS,
    PROJECTION_STYLES,
    DattriProjector,
    ProjectionMatrix,
    apply_projection,
    capture_projected,
    gaussian_projector,
    mask_coordinates,
    mask_factorized,
    mask_factors,
    mask_materialized,
    maybe_materialize_projected,
    project_activation,
    project_factorized,
    project_factors,
    project_gradient,
    project_layer,
    project_materialized,
    project_materialized_factors,
    project_outer_factors,
    should_materialize,
)
from dattri_llm_amd.gradient.ops.types import (
    ALL_LAYER_TYPES,
    CONV_TRANSPOSE_TYPES,
    CONV_TYPES,
    EMBEDDING_TYPES,
    LINEAR_TYPES,
    NORM_TYPES,
    PARAM_GRAD_TYPES,
    canonical_class_name,
    is_conv,
    is_conv_transpose,
    is_embedding,
    is_kfac_eligible,
    is_linear,
    is_norm,
)

from dattri_llm_amd.gradient.ops.optimizer import (  # noqa: E402  (names only: outside the scoring path)
    OPTIMIZER_STATE_KEYS,
    adam_preconditioner,
    adamw_influence_coupling,
    adamw_influence_push,
    adamw_influence_transition,
    precondition,
)

__all__ = [
    "OPTIMIZER_STATE_KEYS", "adam_preconditioner", "adamw_influence_coupling", "adamw_influence_push",
    "adamw_influence_transition", "precondition",
    "FisherAccumulator", "KroneckerAccumulator", "LayerFisherAccumulator", "LayerKroneckerAccumulator",
    "dense_inverse", "ekfac_materialize", "ekfac_materialize_factors", "ekfac_precondition", "fim",
    "fim_factors", "kfac", "kfac_cross", "kfac_cross_factors", "kfac_eigh", "kfac_factors",
    "kfac_precondition", "kfac_precondition_materialized", "kronecker", "sym_inverse",
    "ALL_LAYER_TYPES", "CAPTURE_STYLES", "CONV_TRANSPOSE_TYPES", "CONV_TYPES", "EMBEDDING_TYPES",
    "LINEAR_TYPES", "MASK_KEYS", "NORM_TYPES", "PARAM_GRAD_TYPES", "PROJECTION_STYLES", "CostModel",
    "DattriProjector", "ProjectionMatrix", "apply_projection", "as_float", "block_grad_norm_sq", "calibrate",
    "canonical_class_name", "capture_projected", "compute_dtype", "cost", "cross_dot",
    "cross_dot_factors", "cross_dot_per_token", "cross_gram", "cross_gram_per_token",
    "cross_gram_per_token_dense", "dot", "dot_factors", "dtypes", "effective_dims",
    "extract_module_kwargs", "gaussian_projector", "get_compute_dtype", "get_routing_policy",
    "grad_norm_sq", "grad_norm_sq_factors", "is_conv", "is_conv_transpose", "is_embedding",
    "is_kfac_eligible", "is_linear", "is_norm", "layerwise_cross_dot", "layerwise_cross_dot_per_token",
    "mask_coordinates", "mask_factorized", "mask_factors", "mask_materialized",
    "materialize", "materialize_blocked", "materialize_factors", "materialize_group", "maybe_materialize_projected", "maybe_use_materialized_gram",
    "maybe_use_materialized_norm", "moe", "pairwise_dot", "pairwise_dot_factors", "preprocess_factorized",
    "preprocess_factors", "project_activation", "project_factorized", "project_factors",
    "project_gradient", "project_layer", "project_materialized", "project_materialized_factors",
    "project_outer_factors", "route_flops", "set_compute_dtype",
    "set_routing_policy", "should_materialize", "to_3d",
]
