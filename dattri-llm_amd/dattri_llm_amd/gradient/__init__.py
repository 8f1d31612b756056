"""Gradient data model and ops (the reference's ``dattri_llm.gradient`` surface on this path).

Besides the data model, the names the reference's package re-exports from its
ops (``dot``, ``materialize``, the K-FAC accumulators, ...) resolve to this
package's kernels-backed versions.  Hook managers, callbacks and the storage
manager belong to the capture's control plane and are not part of this package.
"""

from dattri_llm_amd.gradient import ops
from dattri_llm_amd.gradient.capture import FusedCapture
from dattri_llm_amd.gradient.gradient import Factorized, Gradient, GradientRecord
from dattri_llm_amd.gradient.ops import (
    FisherAccumulator,
    KroneckerAccumulator,
    LayerFisherAccumulator,
    LayerKroneckerAccumulator,
    canonical_class_name,
    dot,
    fim,
    grad_norm_sq,
    kfac,
    materialize,
    pairwise_dot,
)
from dattri_llm_amd.gradient.routing import RowLayout, locate_rows
from dattri_llm_amd.gradient.store import AsyncGradientWriter, GradientStore

__all__ = [
    "AsyncGradientWriter",
    "Factorized",
    "FisherAccumulator",
    "FusedCapture",
    "Gradient",
    "GradientRecord",
    "GradientStore",
    "KroneckerAccumulator",
    "LayerFisherAccumulator",
    "LayerKroneckerAccumulator",
    "RowLayout",
    "canonical_class_name",
    "dot",
    "fim",
    "grad_norm_sq",
    "kfac",
    "locate_rows",
    "materialize",
    "ops",
    "pairwise_dot",
]
