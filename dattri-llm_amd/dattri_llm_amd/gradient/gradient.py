"""Gradient data model: ``Factorized`` factor pairs and ``Gradient`` blocks.

The containers of ``dattri_llm/gradient/gradient.py`` kept as they are
(:20-116, :183-1191): a block maps layer names to a :class:`Factorized`
``(activation, pre_activation_grad)`` capture or a dense ``(B, d)`` tensor,
with per-layer representation, layer type and indexing, so blocks built by
the reference's capture side score here unchanged.  The arithmetic methods
(:meth:`Gradient.materialize`, :meth:`Gradient.project`,
:meth:`Gradient.similarity`) run on the MI355X ops.
"""

from __future__ import annotations

from dataclasses import InitVar, dataclass, field
from typing import TYPE_CHECKING, Literal

import torch

from dattri_llm_amd.gradient import ops

if TYPE_CHECKING:
    from collections.abc import Callable, Iterable

GradientRepresentation = Literal["materialized", "factorized"]
Indexing = Literal["batch", "batch_token"]


@dataclass(frozen=True, eq=False)
class Factorized:
    """A per-layer factorized ("ghost") gradient (gradient.py:20-116)."""

    activation: torch.Tensor
    pre_activation_grad: torch.Tensor
    module_kwargs: dict | None = field(default=None, compare=False, repr=False, hash=False)
    batch_first: bool = field(default=True, compare=False)

    def to(self, device=None, dtype=None, non_blocking: bool = False) -> Factorized:
        return Factorized(
            self.activation.to(device=device, dtype=dtype, non_blocking=non_blocking),
            self.pre_activation_grad.to(device=device, dtype=dtype, non_blocking=non_blocking),
            module_kwargs=self.module_kwargs,
            batch_first=self.batch_first,
        )

    def pin_memory(self) -> Factorized:
        def pin(t):
            return t if t.device.type != "cpu" or t.is_pinned() else t.pin_memory()

        return Factorized(pin(self.activation), pin(self.pre_activation_grad),
                          module_kwargs=self.module_kwargs, batch_first=self.batch_first)

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.activation, self.pre_activation_grad))

    def as_batch_first(self) -> Factorized:
        if self.batch_first:
            return self
        return Factorized(self.activation.transpose(0, 1), self.pre_activation_grad.transpose(0, 1),
                          module_kwargs=self.module_kwargs, batch_first=True)


GradientData = torch.Tensor | Factorized


@dataclass(frozen=True, eq=False)
class Gradient:
    """A per-step, multi-layer container of per-sample gradients (gradient.py:183-1191)."""

    representation: dict[str, GradientRepresentation]
    data: dict[str, GradientData]
    layer_types: dict[str, str]
    indexing: dict[str, Indexing] = field(default_factory=dict)
    validate_on_init: InitVar[bool] = True

    def __post_init__(self, validate_on_init: bool) -> None:
        object.__setattr__(self, "indexing", {n: self.indexing.get(n, "batch") for n in self.data})
        if validate_on_init:
            self.validate()

    # -- properties ----------------------------------------------------------
    @property
    def layer_names(self) -> set[str]:
        return set(self.data.keys())

    @property
    def batch_size(self) -> int:
        """Largest per-layer sample count, ignoring batch-level layers (gradient.py:208-237)."""
        best = 0
        for name, x in self.data.items():
            if self.layer_types.get(name) == ops.PARAM_GRAD_TYPES:
                continue
            if isinstance(x, Factorized):
                best = max(best, x.activation.shape[0 if x.batch_first else 1])
            else:
                best = max(best, x.shape[0])
        if best:
            return best
        raise ValueError(
            "batch_size is undefined for a gradient holding only batch-level "
            "param_grad layers (their tensors have no per-sample axis)."
        )

    @property
    def token_dim(self) -> dict[str, int | None]:
        out: dict[str, int | None] = {}
        for name, value in self.data.items():
            if self.indexing[name] == "batch_token":
                if isinstance(value, Factorized):
                    out[name] = value.activation.shape[1 if value.batch_first else 0]
                else:
                    out[name] = value.shape[1]
            else:
                out[name] = None
        return out

    @property
    def device(self) -> torch.device:
        x = next(iter(self.data.values()))
        return x.activation.device if isinstance(x, Factorized) else x.device

    @property
    def dtype(self) -> torch.dtype:
        x = next(iter(self.data.values()))
        return x.activation.dtype if isinstance(x, Factorized) else x.dtype

    @property
    def nbytes(self) -> int:
        return sum(v.nbytes if isinstance(v, Factorized) else v.numel() * v.element_size()
                   for v in self.data.values())

    @property
    def materialized_nbytes(self) -> int:
        """Bytes :meth:`materialize` would produce, from shapes only (gradient.py:279-307)."""
        total = 0
        for name, val in self.data.items():
            if not isinstance(val, Factorized):
                total += val.numel() * val.element_size()
                continue
            bf = val.as_batch_first()
            a, g = bf.activation, bf.pre_activation_grad
            b, itemsize = a.shape[0], g.element_size()
            layer_type = self.layer_types.get(name, "nn.Linear")
            if ops.is_norm(layer_type):
                total += b * a.shape[-1] * itemsize
            elif ops.is_embedding(layer_type):
                mk = bf.module_kwargs or {}
                vocab = mk.get("num_embeddings") or int(a.max().item()) + 1
                total += b * vocab * g.shape[-1] * itemsize
            else:
                total += b * a.shape[-1] * g.shape[-1] * itemsize
        return total

    # -- structure ------------------------------------------------------------
    def validate(self) -> None:
        """Internal consistency checks (gradient.py:361-465)."""
        if not self.data:
            raise ValueError("data cannot be empty")
        missing = set(self.data) - set(self.representation)
        if missing:
            raise ValueError(f"Missing representation for layers: {sorted(missing)}")
        batch_size = None
        batch_layer = None
        for name, value in self.data.items():
            layer_repr = self.representation[name]
            layer_type = self.layer_types[name]
            if layer_repr == "factorized":
                if not isinstance(value, Factorized):
                    raise TypeError(f"{name} must be Factorized")
                shape = tuple(value.activation.shape)
                bf = value.as_batch_first()
                act, gout = bf.activation, bf.pre_activation_grad
                if layer_type == "nn.EmbeddingBag":
                    if act.ndim != 2 or gout.ndim != 2:
                        raise ValueError(f"{name} has invalid embedding-bag factor dimensions")
                    if act.shape[0] != gout.shape[0]:
                        raise ValueError(f"{name} embedding-bag batch dimension mismatch")
                elif ops.is_embedding(layer_type):
                    if act.ndim != 2 or gout.ndim != 3:
                        raise ValueError(f"{name} has invalid embedding factor dimensions")
                    if act.shape != gout.shape[:2]:
                        raise ValueError(f"{name} embedding batch/token dimensions mismatch")
                elif ops.is_conv(layer_type) or ops.is_conv_transpose(layer_type):
                    if act.shape[0] != gout.shape[0]:
                        raise ValueError(f"{name} conv factor batch size mismatch: {act.shape[0]} != {gout.shape[0]}")
                elif act.shape[:-1] != gout.shape[:-1]:
                    raise ValueError(f"{name} factor batch/token dimensions mismatch")
                cur = act.shape[0]
            else:
                if not isinstance(value, torch.Tensor):
                    raise TypeError(f"{name} must be Tensor")
                if value.ndim < 1:
                    raise ValueError(f"{name} must be at least 1D")
                if (layer_type != ops.PARAM_GRAD_TYPES and self.indexing[name] == "batch_token"
                        and value.ndim != 3):
                    raise ValueError(f"{name} declared as batch_token but tensor is {value.ndim}D, expected 3D")
                cur = value.shape[0]
                shape = tuple(value.shape)
            if layer_type != ops.PARAM_GRAD_TYPES and cur != 1:
                if batch_size is None:
                    batch_size, batch_layer = cur, (name, shape)
                elif batch_size != cur:
                    first_name, first_shape = batch_layer
                    raise ValueError(
                        "All layers must have the same batch size: "
                        f"{first_name} has {batch_size} samples (captured shape {first_shape}) but "
                        f"{name} has {cur} (captured shape {shape}). The sample axis is read from dim 0 "
                        "of every per-sample layer; a layer whose input is sequence-first (T, B, ...) "
                        "must be declared in HookManager(non_batch_first_layers=...), and a layer fed "
                        "flattened or routed token rows (an MoE router or expert) in "
                        "HookManager(moe_routed_layers=...)."
                    )

    def map_layers(self, fn: Callable, *, layers: Iterable[str] | None = None, consume: bool = False) -> Gradient:
        """Apply ``fn(name, value, layer_type)`` per selected layer (gradient.py:309-359)."""
        selected = set(self.data) if layers is None else set(layers)
        new_data, new_repr, new_index = {}, {}, {}
        for name in list(self.data):
            release = consume and name in selected
            old = self.data.pop(name) if release else self.data[name]
            value = fn(name, old, self.layer_types[name]) if name in selected else old
            del old
            if value is None:
                continue
            new_data[name] = value
            if isinstance(value, Factorized):
                new_repr[name], new_index[name] = "factorized", self.indexing[name]
            else:
                new_repr[name] = "materialized"
                new_index[name] = "batch" if name in selected else self.indexing[name]
        return Gradient(new_repr, new_data, {k: v for k, v in self.layer_types.items() if k in new_data},
                        new_index, validate_on_init=False)

    def select_layers(self, names: Iterable[str]) -> Gradient:
        keep = [n for n in names if n in self.data]
        return Gradient({n: self.representation[n] for n in keep}, {n: self.data[n] for n in keep},
                        {n: self.layer_types[n] for n in keep}, {n: self.indexing[n] for n in keep},
                        validate_on_init=False)

    def clone(self) -> Gradient:
        data = {}
        for name, v in self.data.items():
            data[name] = (Factorized(v.activation.clone(), v.pre_activation_grad.clone(),
                                     module_kwargs=v.module_kwargs, batch_first=v.batch_first)
                          if isinstance(v, Factorized) else v.clone())
        return Gradient(dict(self.representation), data, dict(self.layer_types), dict(self.indexing))

    def to(self, device=None, dtype=None, non_blocking: bool = False) -> Gradient:
        data = {n: v.to(device=device, dtype=dtype, non_blocking=non_blocking) for n, v in self.data.items()}
        return Gradient(dict(self.representation), data, self.layer_types, dict(self.indexing))

    # -- arithmetic -------------------------------------------------------------
    def materialize(self) -> Gradient:
        """Every factorized layer as its dense per-sample gradient (gradient.py:539-567)."""
        if all(r == "materialized" for r in self.representation.values()):
            return self
        data, rep, index = {}, {}, dict(self.indexing)
        for name, value in self.data.items():
            if self.representation[name] == "factorized" and isinstance(value, Factorized):
                data[name] = ops.materialize(value, self.layer_types[name])
                rep[name] = "materialized"
                index[name] = "batch"
            else:
                data[name], rep[name] = value, self.representation[name]
        return Gradient(rep, data, self.layer_types, index)

    def project(self, projector, projection: dict, *, capture_style: str = "factorized") -> Gradient:
        """LoGRA-project every configured layer (the ``"logra"`` part of gradient.py:569-662).

        ``projection`` maps layer names (or ``"__default__"``) to
        ``{"style": "logra", "proj_dim": k, "proj_seed": s, ...}``."""
        proj = ops.DattriProjector.coerce(projector)
        data, rep, index = {}, {}, {}
        for name, value in self.data.items():
            kw = projection.get(name, projection.get("__default__"))
            lt = self.layer_types[name]
            if kw is None or not ops.is_linear(lt) or not isinstance(value, Factorized):
                data[name], rep[name], index[name] = value, self.representation[name], self.indexing[name]
                continue
            kw = dict(kw)
            style = kw.pop("style", "logra")
            payload, is_fact = ops.project_layer(value, lt, proj, style=style, capture_style=capture_style, **kw)
            if is_fact:
                data[name] = Factorized(*payload, module_kwargs=None)
                rep[name], index[name] = "factorized", self.indexing[name]
            else:
                data[name], rep[name], index[name] = payload, "materialized", "batch"
        return Gradient(rep, data, dict(self.layer_types), index)

    def _layer_norm_sq(self, name: str, mode: str) -> torch.Tensor:
        return ops.grad_norm_sq(self.data[name], self.layer_types[name], mode=mode)

    def similarity(self, other: Gradient, metric: str = "dot", reduce: str = "none", mode: str = "auto",
                   eps: float = 1e-8):
        """Per-sample gradient similarity (gradient.py:963-1070)."""
        if metric not in {"dot", "cosine"}:
            raise ValueError("metric must be 'dot' or 'cosine'")
        if reduce not in {"none", "all"}:
            raise ValueError("reduce must be 'none' or 'all'")
        if mode not in {"factorized", "materialized", "auto"}:
            raise ValueError("mode must be 'factorized', 'materialized', or 'auto'")
        per_layer = ops.layerwise_cross_dot(self, other, mode=mode, reduce="none")
        if reduce == "none":
            if metric == "cosine":
                for name in per_layer:
                    n_s = self._layer_norm_sq(name, mode).clamp_min(0).sqrt()
                    n_o = other._layer_norm_sq(name, mode).clamp_min(0).sqrt()
                    per_layer[name] = per_layer[name] / (n_s[:, None] * n_o[None, :] + eps)
            return per_layer
        if not per_layer:
            raise ValueError("No shared layers to compute an overall similarity")
        total = ops.layerwise_cross_dot(self, other, layers=list(per_layer), mode=mode, reduce="sum")
        if metric == "cosine":
            b_s, b_o = self.batch_size, other.batch_size

            def expand(v, b):
                return v.expand(b) if v.shape[0] == 1 else v

            ns = torch.stack([expand(self._layer_norm_sq(n, mode), b_s) for n in per_layer]).sum(0).clamp_min(0)
            no = torch.stack([expand(other._layer_norm_sq(n, mode), b_o) for n in per_layer]).sum(0).clamp_min(0)
            total = total / (ns.sqrt()[:, None] * no.sqrt()[None, :] + eps)
        return total

    def __repr__(self) -> str:
        return f"Gradient(layers={sorted(self.data)}, batch={self.batch_size})"


@dataclass
class GradientRecord:
    """A gradient snapshot with its identity (gradient.py:1198-1237)."""

    step: int
    input_hash: str | list[str]
    gradient: Gradient
    sample_id_key: str | int | None = None
