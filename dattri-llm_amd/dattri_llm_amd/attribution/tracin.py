"""TracIn / GradCos on the MI355X scoring path.

Follows the scoring half of ``dattri_llm/attribution/algorithm/tracin.py`` and
``attribution/base.py``: the score of a train block against a query block is
the layerwise cross-gram (base.py:657-698, tracin.py:92-126); GradCos divides
it by both sides' whole-model gradient norms (tracin.py:125-148); the query
block is routed once before scoring (``route_test_rep``, the contract of
base.py:586-655, planned in :mod:`dattri_llm_amd.attribution.routing`).

GradCos norms: a train block's are computed once per block (reusing the dense
copies the score already made), a query block's once per routed block -- not
once per train block -- and each costs one launch per representation (all
dense layers in one row-dot launch; factorized linears on the ghost kernel's
diagonal pairs).
"""

from __future__ import annotations

import weakref
from typing import ClassVar

import torch

from dattri_llm_amd.attribution.base import InnerProductAttributor
from dattri_llm_amd.attribution.score import AttributionScore
from dattri_llm_amd.gradient import ops
from dattri_llm_amd.gradient.gradient import Gradient

_EPS = 1e-8  # added to the product of the norms (tracin.py:108)


class TracInAttributor(InnerProductAttributor):
    """Gradient-dot (TracIn) or cosine (GradCos) attribution over gradient sources.

    Args:
        train_batch_size: train samples per scoring block (the reference's
            ``per_device_train_batch_size``), used by the query routing rule.
        device: where scoring runs.
        cache_budget: budget factory ``device -> CacheBudget`` for the dense query cache.
    """

    algorithm: ClassVar[str] = "TracIn"

    def __init__(self, train_batch_size: int = 1, device="cuda", *, cache_budget=None) -> None:
        super().__init__(train_batch_size, device, cache_budget=cache_budget)
        self._metric = "dot"
        # query block -> {shared layers: (B,) whole-model norms}; entries die with the block
        self._query_norms: weakref.WeakKeyDictionary = weakref.WeakKeyDictionary()

    def _set_metric(self, normalized_grad: bool) -> None:
        self._metric = "cosine" if normalized_grad else "dot"
        self.algorithm = "GradCos" if normalized_grad else "TracIn"

    # -- scores -------------------------------------------------------------

    def _norms(self, rep: Gradient, layers: list[str], dense_cache=None) -> torch.Tensor:
        return ops.block_grad_norm_sq(rep, layers, dense_cache).clamp_min(0).sqrt()

    def _query_norms_of(self, test_rep: Gradient, layers: list[str]) -> torch.Tensor:
        per_block = self._query_norms.setdefault(test_rep, {})
        key = tuple(layers)
        if key not in per_block:
            per_block[key] = self._norms(test_rep, layers)
        return per_block[key]

    def _cosine(self, dot: torch.Tensor, train_rep: Gradient, test_rep: Gradient, layers: list[str],
                dense_cache=None) -> torch.Tensor:
        """``dot`` (train axis first, query axis last) over the product of the
        two sides' whole-model gradient norms, plus 1e-8."""
        n_tr = self._norms(train_rep, layers, dense_cache)
        n_te = self._query_norms_of(test_rep, layers)
        shape = (n_tr.shape[0],) + (1,) * (dot.dim() - 1)
        return dot / (n_tr.view(shape) * n_te + _EPS)

    def inner_product(self, train_rep: Gradient, test_rep: Gradient, *, dense_cache=None) -> torch.Tensor:
        """``(B_train, B_test)`` scores of one train block against one query block."""
        layers = self._shared(train_rep, test_rep)
        if not layers:
            return torch.zeros(train_rep.batch_size, test_rep.batch_size, device=self.device)
        dot = ops.layerwise_cross_dot(train_rep, test_rep, dense_cache=dense_cache)
        return dot if self._metric == "dot" else self._cosine(dot, train_rep, test_rep, layers, dense_cache)

    def inner_product_per_token(self, train_rep: Gradient, test_rep: Gradient) -> torch.Tensor:
        """(B_train, T_train, B_test) decomposition of :meth:`inner_product` over the
        train side's token positions (tracin.py:110-126, base.py:677-698); for
        GradCos each position's share of the cosine (the per-token dots over the
        two whole-sample norms)."""
        layers = self._shared(train_rep, test_rep)
        if not layers:
            return self._zeros_per_token(train_rep, test_rep)
        dot = ops.layerwise_cross_dot_per_token(train_rep, test_rep)
        return dot if self._metric == "dot" else self._cosine(dot, train_rep, test_rep, layers)

    def attribute_from_cache(self, train_source, test_source, *, selected_training_steps=None, layer_name=None,
                             verbose: bool = False, loop_over_test: bool = False, algorithm_meta: dict | None = None,
                             attribution_granularity: str = "instance", normalized_grad: bool = False,
                             train_blocks_per_pass: int = 1) -> AttributionScore:
        """Score stored gradients (tracin.py:186-215); ``normalized_grad``
        selects GradCos and is recorded in the metadata.  The other arguments
        are :meth:`InnerProductAttributor.attribute_from_cache`'s."""
        self._set_metric(normalized_grad)
        return super().attribute_from_cache(
            train_source, test_source, selected_training_steps=selected_training_steps, layer_name=layer_name,
            verbose=verbose, loop_over_test=loop_over_test, algorithm_meta=algorithm_meta,
            attribution_granularity=attribution_granularity, train_blocks_per_pass=train_blocks_per_pass,
            normalized_grad=normalized_grad)

    def attribute_sources(self, train_source, test_source, *, normalized_grad: bool = False,
                          batch_size: int | None = None, loop_over_test: bool = False,
                          attribution_granularity: str = "instance",
                          train_blocks_per_pass: int = 1) -> AttributionScore:
        """Score two ``(step, Gradient, hashes)`` sources (base.py:704-770);
        ``loop_over_test`` re-streams a reusable test source per train block
        instead of caching it; ``attribution_granularity="token"`` gives one row
        per training token position (:meth:`inner_product_per_token`);
        ``train_blocks_per_pass`` > 1 reads a dense query block once per that
        many train blocks, with the same scores."""
        self._set_metric(normalized_grad)
        return self._score(train_source, test_source, batch_size=batch_size, loop_over_test=loop_over_test,
                           attribution_granularity=attribution_granularity,
                           algorithm_meta={"normalized_grad": normalized_grad},
                           train_blocks_per_pass=train_blocks_per_pass)
