"""Which query layers are scored dense: the routing plan of a query block.

The contract is dattri-llm's ``_route_test_rep`` (``attribution/base.py:586-655``),
run once per query block before the scoring loop:

* a factorized linear layer goes dense when the cost rule
  (``ops.maybe_use_materialized_gram`` with the train batch, the query batch
  and the query length) prefers it; a layer without an outer-product form
  (norms, embeddings) always asks to go dense; dense layers stay as they are;
* the dense copies live through the whole loop, so they are admitted against
  a byte budget one layer at a time, largest flop saving first (ties by
  layer name, larger first); what is charged is the growth over the
  factorized payload the dense copy replaces, and a layer that does not fit
  stays factorized;
* whatever stays factorized is preprocessed once (``finalize_factors``).

Here the decision is a :class:`QueryPlan` -- one :class:`LayerRoute` per
candidate layer -- computed from shapes alone, then applied: admitted linear
layers are materialized in the k-blocked layout the score kernel streams.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from dattri_llm_amd.attribution.utils import finalize_factors
from dattri_llm_amd.gradient import ops
from dattri_llm_amd.gradient.gradient import Factorized, Gradient
from dattri_llm_amd.gradient.ops.materialize import materialize_blocked
from dattri_llm_amd.utils.cache import CacheBudget


@dataclass(frozen=True)
class LayerRoute:
    """A query layer that asks to be scored dense."""

    name: str
    saving: float  # flops one train block saves by scoring it dense (inf: no factorized route)
    growth: int  # bytes its dense copy adds over the factors it replaces
    admitted: bool = False


@dataclass
class QueryPlan:
    """The routing decision for one query block."""

    routes: list[LayerRoute] = field(default_factory=list)
    held: int = 0  # bytes the admitted dense copies add

    @property
    def dense(self) -> list[str]:
        return [r.name for r in self.routes if r.admitted]


def _has_outer_product_form(layer_type: str) -> bool:
    return ops.is_linear(layer_type) or ops.is_conv(layer_type) or ops.is_conv_transpose(layer_type)


def plan_query(test_rep: Gradient, train_batch: int, budget: CacheBudget) -> QueryPlan:
    """The layers of ``test_rep`` that go dense, in admission order."""
    asks = []
    for name in test_rep.layer_names:
        value = test_rep.data[name]
        if not isinstance(value, Factorized):
            continue
        layer_type = test_rep.layer_types[name]
        if not _has_outer_product_form(layer_type):
            saving = float("inf")
        else:
            b_test, s, k, d = ops.effective_dims(value, layer_type)
            if not ops.maybe_use_materialized_gram(train_batch, b_test, s, k, d):
                continue
            cost_f, cost_m = ops.route_flops(train_batch, b_test, s, k, d)
            saving = cost_f - cost_m
        layer = test_rep.select_layers([name])
        asks.append(LayerRoute(name, saving, max(layer.materialized_nbytes - layer.nbytes, 0)))
    plan = QueryPlan()
    for ask in sorted(asks, key=lambda r: (r.saving, r.name), reverse=True):
        admitted = budget.fits(ask.growth, plan.held)
        plan.routes.append(LayerRoute(ask.name, ask.saving, ask.growth, admitted))
        if admitted:
            plan.held += ask.growth
    return plan


def apply_plan(test_rep: Gradient, plan: QueryPlan, budget: CacheBudget) -> Gradient:
    """``test_rep`` with the admitted layers dense (k-blocked where the layout
    allows) and the rest finalized, releasing each factorized payload as its
    replacement is built."""
    if plan.dense:
        test_rep = test_rep.map_layers(lambda _n, v, lt: materialize_blocked(v, lt), layers=plan.dense, consume=True)
    return finalize_factors(test_rep, budget=budget, held=plan.held)
