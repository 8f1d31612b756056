"""K-FAC and EK-FAC influence attribution on the MI355X scoring path.

Follows the in-memory workflow of ``dattri_llm/attribution/algorithm/kronecker.py``:

* :meth:`KroneckerAttributor.fit_raw` (kronecker.py:290-348) sweeps a
  re-iterable train source into the damping-free fit.  That fit holds the
  per-layer Kronecker factors of the linear and convolution layers stored
  factorized.  It also holds a dense empirical Fisher for the layers stored
  materialized, and for the norm layers under ``non_kfac_strategy="direct"``
  (kronecker.py:638-734).
* :meth:`KroneckerAttributor.damp_fit` (kronecker.py:361-403) folds the damping in.
* :meth:`KroneckerAttributor.transform_test_rep` (kronecker.py:599-636)
  preconditions each query block once, and the block is then scored against
  raw train blocks by the plain layerwise cross-gram.

K-FAC (kronecker.py:1360-1442) keeps a factorized query layer factorized:
``(a A^-1, g G^-1)`` are final factors that the cross-gram cost rule still
routes.  EK-FAC (kronecker.py:1445-1601) rotates into the Kronecker
eigenbasis, corrects the spectrum with a second train sweep, and returns a
dense query layer.  The covariances come from ``da_row_gram``.  The
rotations, inverses and scores run on the kernels behind
:mod:`dattri_llm_amd.gradient.ops`.

The reference's persisted fits (``fisher_dir``), off-device factor caches,
capture-time covariances and preconditioned-test stores are storage around
this workflow and are not built.  A fit is reused in memory instead: pass
the result of :meth:`fit` to ``attribute_sources(raw_fit=...)``.
"""

from __future__ import annotations

import warnings
from typing import ClassVar

import torch

from dattri_llm_amd.attribution.base import InnerProductAttributor
from dattri_llm_amd.attribution.score import AttributionScore
from dattri_llm_amd.gradient import ops
from dattri_llm_amd.gradient.gradient import Factorized, Gradient

NON_KFAC_STRATEGIES = ("ignore", "direct")


def _mean_eigenvalue(matrix: torch.Tensor) -> torch.Tensor:
    """The trace over the size of a square matrix, or of a stack of them (kronecker.py:136-140)."""
    return matrix.diagonal(dim1=-2, dim2=-1).float().mean()


class KroneckerAttributor(InnerProductAttributor):
    """Shared workflow of the K-FAC family (kronecker.py:158-227).

    A subclass supplies :meth:`fit_factors` (damping-free per-layer factors),
    :meth:`damp` (fold a damping in, data-free) and
    :meth:`precondition_test_layer` (one query layer times its damped inverse).
    """

    algorithm: ClassVar[str] = "Kronecker"

    def __init__(self, train_batch_size: int = 1, device="cuda", *, cache_budget=None) -> None:
        super().__init__(train_batch_size, device, cache_budget=cache_budget)
        self._damping = 1e-3
        self._non_kfac_strategy = "ignore"
        self._direct_fim_max_params = 4096
        self._relative_damping = False
        self._raw_fit: tuple[dict, dict] | None = None
        self._preconditioner: tuple[dict, dict] | None = None
        self._skipped_materialized: set[str] = set()
        self._fisher_saw_embedding: set[str] = set()
        self._direct_norm_layers = False

    # -- subclass hooks ---------------------------------------------------------

    def fit_factors(self, train_source, fisher_acc: ops.FisherAccumulator) -> dict:
        """The damping-free ``{layer: factors}``; feeds every block of its first
        sweep to :meth:`accumulate_fisher` (kronecker.py:230-249)."""
        raise NotImplementedError

    def damp(self, raw_factors: dict, damping: float) -> dict:
        """``raw_factors`` with *damping* folded in (kronecker.py:251-258)."""
        raise NotImplementedError

    def precondition_test_layer(self, value, layer_type: str, factors):
        """One query layer times its layer's damped inverse Fisher (kronecker.py:260-277)."""
        raise NotImplementedError

    # -- options ----------------------------------------------------------------

    def set_options(self, damping: float = 1e-3, non_kfac_strategy: str = "ignore",
                    direct_fim_max_params: int = 4096, relative_damping: bool = False) -> None:
        """Validate and store the per-call options; forget the previous fit (kronecker.py:555-597)."""
        if damping < 0:
            raise ValueError(f"damping must be non-negative, got {damping}.")
        if non_kfac_strategy not in NON_KFAC_STRATEGIES:
            raise ValueError(f"non_kfac_strategy must be 'ignore' or 'direct', got {non_kfac_strategy!r}.")
        if direct_fim_max_params <= 0:
            raise ValueError(f"direct_fim_max_params must be positive, got {direct_fim_max_params}.")
        self._damping = damping
        self._non_kfac_strategy = non_kfac_strategy
        self._direct_fim_max_params = direct_fim_max_params
        self._relative_damping = relative_damping
        self._raw_fit = None
        self._preconditioner = None

    def _damping_for(self, damping: float, spectrum_mean) -> float:
        """``damping``, or ``damping`` times the spectrum's mean eigenvalue under
        ``relative_damping`` (kronecker.py:350-359)."""
        return damping * float(spectrum_mean) if self._relative_damping else damping

    # -- layer selection ----------------------------------------------------------

    def kfac_layers(self, grad: Gradient) -> list[str]:
        """Linear and convolution layers stored factorized; a layer of those types
        stored materialized is recorded for the direct Fisher (kronecker.py:638-659)."""
        names = []
        for name, value in grad.data.items():
            if not ops.is_kfac_eligible(grad.layer_types[name]):
                continue
            if isinstance(value, Factorized):
                names.append(name)
            else:
                self._skipped_materialized.add(name)
        return names

    def fisher_layers(self, grad: Gradient) -> list[str]:
        """Layers entering the dense empirical Fisher: every per-sample layer
        stored materialized, and the norm layers under the direct strategy
        (kronecker.py:661-681)."""
        names = []
        for name, value in grad.data.items():
            layer_type = grad.layer_types[name]
            if layer_type == ops.PARAM_GRAD_TYPES:
                continue
            if isinstance(value, torch.Tensor) or (self._direct_norm_layers and ops.is_norm(layer_type)):
                names.append(name)
        return names

    def accumulate_fisher(self, fisher_acc: ops.FisherAccumulator, grad: Gradient) -> None:
        """Fold one train block into the direct Fisher; note factorized embeddings,
        which no preconditioner covers (kronecker.py:683-701)."""
        fisher_acc.update(grad, self.fisher_layers(grad))
        if self._direct_norm_layers:
            self._fisher_saw_embedding.update(
                name for name, value in grad.data.items()
                if ops.is_embedding(grad.layer_types[name]) and isinstance(value, Factorized))

    # -- the fit --------------------------------------------------------------------

    def _blocks(self, source):
        for _step, block, _hashes in source:
            yield block.to(self.device)

    def fit_raw(self, train_source) -> tuple[dict, dict]:
        """The damping-free ``(factors, fisher)`` from one (EK-FAC: two) sweeps
        over a re-iterable train source (kronecker.py:290-348)."""
        if not getattr(train_source, "reusable", False):
            raise ValueError(
                f"{type(self).__name__} needs a re-iterable train source (reusable=True): the Fisher "
                "pre-pass re-reads the train gradients before scoring.")
        self._skipped_materialized = set()
        self._fisher_saw_embedding = set()
        self._direct_norm_layers = self._non_kfac_strategy == "direct"
        max_params = self._direct_fim_max_params
        fisher_acc = ops.FisherAccumulator(max_params)
        raw_factors = self.fit_factors(train_source, fisher_acc)
        if self._skipped_materialized:
            n_skipped = len(self._skipped_materialized)
            warnings.warn(
                f"{n_skipped} of the {n_skipped + len(raw_factors)} K-FAC-eligible layers are not "
                f"preconditioned by {self.algorithm}" + (" (none is)" if not raw_factors else "")
                + ".  Layers stored materialized have no (a, g) factors to build the Kronecker "
                f"covariances from; they take the direct dense empirical Fisher instead, bounded by "
                f"direct_fim_max_params={max_params}: {sorted(self._skipped_materialized)}.",
                stacklevel=2)
        if fisher_acc.skipped:
            warnings.warn(
                "The direct dense-Fisher fallback skipped layers whose parameter count exceeds "
                f"direct_fim_max_params={max_params}: {dict(sorted(fisher_acc.skipped.items()))}.",
                stacklevel=2)
        if self._fisher_saw_embedding:
            warnings.warn(
                "non_kfac_strategy='direct' does not cover embedding layers; leaving ignored: "
                f"{sorted(self._fisher_saw_embedding)}.", stacklevel=2)
        raw_fisher = fisher_acc.result()
        if not raw_factors and not raw_fisher:
            raise ValueError(
                "No eligible layers found in the training gradients: no K-FAC-eligible (linear/conv) layer"
                + (f" and no direct-Fisher (norm) layer within direct_fim_max_params={max_params}"
                   if self._non_kfac_strategy == "direct"
                   else " (pass non_kfac_strategy='direct' to include norm layers)") + ".")
        return raw_factors, raw_fisher

    def fit(self, train_source, *, non_kfac_strategy: str = "ignore",
            direct_fim_max_params: int = 4096) -> tuple[dict, dict]:
        """The damping-free fit of *train_source*, to reuse across
        ``attribute_sources(raw_fit=...)`` calls with different dampings
        (the in-memory form of kronecker.py:911-1000)."""
        self.set_options(non_kfac_strategy=non_kfac_strategy, direct_fim_max_params=direct_fim_max_params)
        return self.fit_raw(train_source)

    def damp_fit(self, raw_fit: tuple[dict, dict], damping: float) -> tuple[dict, dict]:
        """``(damped factors, {layer: F^-1})`` of a raw fit (kronecker.py:361-403);
        the dense Fishers are inverted through Cholesky."""
        raw_factors, raw_fisher = raw_fit
        factors = self.damp({name: tuple(t.to(self.device) for t in raw) for name, raw in raw_factors.items()},
                            damping)
        fisher_inverse = {}
        for name, fisher in raw_fisher.items():
            fisher = fisher.to(self.device)
            fisher_inverse[name] = ops.dense_inverse(fisher, self._damping_for(damping, _mean_eigenvalue(fisher)))
        return factors, fisher_inverse

    def prepare_scoring(self, train_source, test_source) -> None:  # noqa: ARG002 - the fit reads the train side
        """Fit unless a fit was handed in, then damp (kronecker.py:517-553)."""
        if self._preconditioner is not None:
            return
        if self._raw_fit is None:
            self._raw_fit = self.fit_raw(train_source)
        self._preconditioner = self.damp_fit(self._raw_fit, self._damping)

    # -- the query side -----------------------------------------------------------------

    def transform_test_rep(self, test_rep: Gradient) -> Gradient:
        """The whole preconditioner applied to one query block: K-FAC layers by
        :meth:`precondition_test_layer`, direct-Fisher layers as ``dense F^-1``,
        every other layer dropped (kronecker.py:599-636)."""
        if self._preconditioner is None:
            raise RuntimeError("prepare_scoring() must run before transform_test_rep().")
        factors, fisher_inverse = self._preconditioner

        def precondition(name, value, layer_type):
            if name in factors:
                return self.precondition_test_layer(value, layer_type, factors[name])
            if name in fisher_inverse:
                dense = value if isinstance(value, torch.Tensor) else ops.materialize(value, layer_type)
                return dense.reshape(dense.shape[0], -1).float() @ fisher_inverse[name]
            return None

        return test_rep.map_layers(precondition)

    # -- the scoring pass ---------------------------------------------------------------

    def _meta(self) -> dict:
        meta = {"damping": self._damping, "relative_damping": self._relative_damping,
                "non_kfac_strategy": self._non_kfac_strategy,
                "direct_fim_max_params": self._direct_fim_max_params}
        mode = getattr(self, "mode", None)
        if mode is not None:
            meta["mode"] = mode
        return meta

    def attribute_sources(self, train_source, test_source, *, damping: float = 1e-3,
                          non_kfac_strategy: str = "ignore", direct_fim_max_params: int = 4096,
                          relative_damping: bool = False, raw_fit: tuple[dict, dict] | None = None,
                          batch_size: int | None = None, loop_over_test: bool = False,
                          attribution_granularity: str = "instance",
                          algorithm_meta: dict | None = None) -> AttributionScore:
        """Influence scores of two ``(step, Gradient, hashes)`` sources: the fit
        (or *raw_fit*), the damping, each query block preconditioned once, then
        the scoring loop (kronecker.py:1102-1270)."""
        self.set_options(damping, non_kfac_strategy, direct_fim_max_params, relative_damping)
        self._raw_fit = raw_fit
        meta = {**self._meta(), "attribution_granularity": attribution_granularity, **(algorithm_meta or {})}
        result = self._score(train_source, test_source, batch_size=batch_size, loop_over_test=loop_over_test,
                             attribution_granularity=attribution_granularity, algorithm_meta=meta)
        result.algorithm_meta["direct_fim_layers"] = sorted(self._preconditioner[1])
        return result


class KFACAttributor(KroneckerAttributor):
    """K-FAC: ``F^-1 ~ (A + lambda)^-1 (x) (G + lambda)^-1`` per linear or
    convolution layer (kronecker.py:1360-1442)."""

    algorithm: ClassVar[str] = "KFAC"

    def fit_factors(self, train_source, fisher_acc: ops.FisherAccumulator) -> dict:
        """One sweep: the raw ``{layer: (A, G)}`` covariances (kronecker.py:1375-1403)."""
        kron = ops.KroneckerAccumulator()
        for train_g in self._blocks(train_source):
            kron.update(train_g, self.kfac_layers(train_g))
            self.accumulate_fisher(fisher_acc, train_g)
        return kron.result(consume=True)

    def damp(self, raw_factors: dict, damping: float) -> dict:
        """``{layer: (A^-1, G^-1)}``, each factor damped on its own (kronecker.py:1405-1419)."""
        return {
            name: (ops.sym_inverse(A, self._damping_for(damping, _mean_eigenvalue(A))),  # noqa: N806
                   ops.sym_inverse(G, self._damping_for(damping, _mean_eigenvalue(G))))  # noqa: N806
            for name, (A, G) in raw_factors.items()  # noqa: N806
        }

    def precondition_test_layer(self, value, layer_type: str, factors):
        """``G^-1 dW A^-1`` per query sample: a factorized layer becomes the final
        factors ``(a A^-1, g G^-1)``; a dense one takes the two-sided product
        (kronecker.py:1421-1442)."""
        a_inv, g_inv = factors
        if isinstance(value, torch.Tensor):
            return ops.kfac_precondition_materialized(value, a_inv, g_inv)
        a, g = ops.kfac_precondition(value, layer_type, a_inv, g_inv)
        return Factorized(a, g, module_kwargs=None, batch_first=True)


class EKFACAttributor(KroneckerAttributor):
    """EK-FAC: the Kronecker eigenbasis with the spectrum replaced by the
    empirical second moments of the rotated train gradients
    (kronecker.py:1445-1601).  ``mode`` ``"exact"`` and ``"approx"`` name two
    projection conventions that give the same scores; it is recorded in the
    score's metadata."""

    algorithm: ClassVar[str] = "EKFAC"
    EKFAC_MODES = ("exact", "approx")

    def __init__(self, train_batch_size: int = 1, device="cuda", *, cache_budget=None,
                 mode: str = "exact") -> None:
        if mode not in self.EKFAC_MODES:
            raise ValueError(f"mode must be one of {self.EKFAC_MODES}, got {mode!r}.")
        super().__init__(train_batch_size, device, cache_budget=cache_budget)
        self.mode = mode

    def fit_factors(self, train_source, fisher_acc: ops.FisherAccumulator) -> dict:
        """Two sweeps: the eigenbases of the covariances, then the undamped
        spectrum ``mean_i (U_G^T dW_i U_A)^2`` in that basis (kronecker.py:1486-1575)."""
        kron = ops.KroneckerAccumulator()
        for train_g in self._blocks(train_source):
            kron.update(train_g, self.kfac_layers(train_g))
            self.accumulate_fisher(fisher_acc, train_g)
        covariances = kron.result(consume=True)
        del kron
        eig = {}
        for name in list(covariances):
            A, G = covariances.pop(name)  # noqa: N806
            _, u_a, _, u_g = ops.kfac_eigh(A, G)
            eig[name] = (u_a, u_g)
        lam_sum: dict[str, torch.Tensor] = {}
        counts: dict[str, int] = {}
        for train_g in (self._blocks(train_source) if eig else ()):
            for name, (u_a, u_g) in eig.items():
                if name not in train_g.data:
                    continue
                rotated = ops.ekfac_materialize(train_g.data[name], train_g.layer_types[name], u_a, u_g)
                square_sum = (rotated * rotated).sum(0)
                lam_sum[name] = lam_sum[name] + square_sum if name in lam_sum else square_sum
                counts[name] = counts.get(name, 0) + rotated.shape[0]
        return {name: (u_a, u_g, lam_sum[name] / counts[name]) for name, (u_a, u_g) in eig.items()}

    def damp(self, raw_factors: dict, damping: float) -> dict:
        """``{layer: (U_A, U_G, lambda + damping)}``, a spectrum shift (kronecker.py:1577-1587)."""
        return {name: (u_a, u_g, lam + self._damping_for(damping, lam.mean()))
                for name, (u_a, u_g, lam) in raw_factors.items()}

    def precondition_test_layer(self, value, layer_type: str, factors) -> torch.Tensor:
        """``U_G ((U_G^T dW U_A) / lambda) U_A^T`` per query sample, dense (kronecker.py:1589-1601)."""
        u_a, u_g, lam = factors
        rotated = ops.ekfac_materialize(value, layer_type, u_a, u_g)
        return ops.ekfac_precondition(rotated, u_a, u_g, lam, layer_type)
