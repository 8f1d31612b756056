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


def base_layer_name(name: str) -> str:
    """The module path of a layer name: a module invoked several times in one
    step is recorded as ``"name"``, ``"name@2"``, ... and module paths hold
    no ``@`` (gradient.py:122-131)."""
    return name.split("@", 1)[0]


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

    def select_layers(self, names: Iterable[str], include_derived: bool = False) -> Gradient:
        """A copy holding only *names* (gradient.py:664-698); with
        ``include_derived`` a name also selects its invocation layers
        (``"lin"`` pulls in ``"lin@2"``, ...).  Raises ``KeyError`` for an
        unknown name."""
        wanted = set(names)
        if include_derived:
            wanted |= {n for n in self.data if base_layer_name(n) in wanted}
        missing = wanted - set(self.data)
        if missing:
            raise KeyError(f"Unknown layers: {sorted(missing)}")
        keep = [n for n in self.data if n in wanted]
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

    def pin_memory(self) -> Gradient:
        """Every host payload in page-locked memory (gradient.py:516-537): what
        asynchronous host-to-device copies of whole blocks need.  Idempotent;
        device payloads pass through."""

        def pin(v):
            if isinstance(v, Factorized):
                return v.pin_memory()
            return v if v.device.type != "cpu" or v.is_pinned() else v.pin_memory()

        return Gradient(dict(self.representation), {n: pin(v) for n, v in self.data.items()}, self.layer_types,
                        dict(self.indexing))

    # -- batch / token reshaping (gradient.py:698-961) ---------------------------
    def _sample_axis(self, value: GradientData, dim: str) -> int:
        """Axis of ``dim`` ("batch" or "token") in a layer's payload."""
        batch_first = value.batch_first if isinstance(value, Factorized) else True
        return (0 if batch_first else 1) if dim == "batch" else (1 if batch_first else 0)

    @staticmethod
    def _rows(value: GradientData) -> int:
        if isinstance(value, Factorized):
            return value.activation.shape[0 if value.batch_first else 1]
        return value.shape[0]

    def _check_compatible(self, other: Gradient, require_same_batch: bool) -> None:
        """The two blocks describe the same layers the same way (gradient.py:1150-1191)."""
        if self.layer_names != other.layer_names:
            raise ValueError("Layer sets differ")
        for what, mine, theirs in (("representations", self.representation, other.representation),
                                   ("indexing", self.indexing, other.indexing)):
            bad = sorted(n for n in self.layer_names if mine.get(n) != theirs.get(n))
            if bad:
                raise ValueError(f"Layers have differing {what}: {bad}")
        if self.layer_types != other.layer_types:
            raise ValueError(f"Layer types differ: {self.layer_types} vs {other.layer_types}")
        if require_same_batch:
            if self.batch_size != other.batch_size:
                raise ValueError("Batch sizes differ")
            mine, theirs = self.token_dim, other.token_dim
            bad = sorted(n for n in self.layer_names if mine[n] != theirs[n])
            if bad:
                raise ValueError(f"Token dimensions differ for layers: {bad}")

    def _require_token_axis(self, what: str) -> None:
        bad = sorted(n for n in self.layer_names if self.indexing[n] != "batch_token")
        if bad:
            raise ValueError(f"Token {what} requires all layers to have indexing='batch_token'. "
                             f"Non-conforming: {bad}")

    def concatenate(self, other: Gradient, dim: Literal["batch", "token"] = "batch") -> Gradient:
        """Join two blocks along the batch or token axis (gradient.py:698-836).

        * Batch joins accept different token counts on ``"batch_token"``
          layers: the shorter side gets extra positions with an exactly-zero
          output gradient (integer activations, i.e. token ids, take the
          layer's ``padding_idx`` or 0), which contribute nothing downstream.
        * A layer broadcast on both sides (one shared row while the block holds
          several samples) becomes one shared row, the two rows averaged with
          the blocks' sample counts as weights: on the output-gradient factor
          when the two activations are identical, else on the materialized
          gradients (the layer then turns ``"materialized"``).
        """
        if dim not in ("batch", "token"):
            raise ValueError("dim must be 'batch' or 'token'")
        self._check_compatible(other, require_same_batch=False)
        if dim == "token":
            self._require_token_axis("concatenation")
            if self.batch_size != other.batch_size:
                raise ValueError("Token concatenation requires the same batch size")
        n_self, n_other = self.batch_size, other.batch_size
        data, rep, index = {}, dict(self.representation), dict(self.indexing)
        for name in self.layer_names:
            mine, theirs = self.data[name], other.data[name]
            if type(mine) is not type(theirs):
                raise TypeError(f"{name} has mismatched data types")
            shared = (self._rows(mine) == 1 < n_self, self._rows(theirs) == 1 < n_other)
            if dim == "batch" and any(shared):
                if not all(shared):
                    raise ValueError(f"{name} is a broadcast (batch-collapsed) gradient on one side but "
                                     "per-sample on the other; the two cannot be concatenated along the "
                                     "batch axis.")
                data[name], merged_dense = _merge_shared_rows(mine, theirs, n_self, n_other,
                                                              self.layer_types[name])
                if merged_dense:
                    rep[name], index[name] = "materialized", "batch"
                continue
            if isinstance(mine, Factorized):
                if mine.batch_first != theirs.batch_first:
                    raise ValueError(f"{name} has mismatched batch_first layout between gradients")
                if dim == "batch" and self.indexing[name] == "batch_token":
                    mine, theirs = _pad_factor_tokens(mine, theirs)
                ax = self._sample_axis(mine, dim)
                data[name] = Factorized(torch.cat([mine.activation, theirs.activation], dim=ax),
                                        torch.cat([mine.pre_activation_grad, theirs.pre_activation_grad], dim=ax),
                                        module_kwargs=mine.module_kwargs, batch_first=mine.batch_first)
            else:
                if dim == "batch" and self.indexing[name] == "batch_token":
                    t = max(mine.shape[1], theirs.shape[1])
                    mine, theirs = _pad_axis(mine, t, 1), _pad_axis(theirs, t, 1)
                data[name] = torch.cat([mine, theirs], dim=self._sample_axis(mine, dim))
        return Gradient(rep, data, self.layer_types, index)

    def aggregate(self, dim: Literal["token"] = "token") -> Gradient:
        """Sum the token axis out of every ``"batch_token"`` layer
        (gradient.py:838-886); ``"batch"`` layers pass through.  A sum, not a
        mean: dL/dW = sum_t g_t a_t^T for any loss, so the per-token
        gradients already carry the loss's own normalization."""
        if dim != "token":
            raise NotImplementedError("Only token aggregation is supported")
        data, rep = {}, {}
        for name, value in self.data.items():
            if self.indexing[name] != "batch_token":
                data[name], rep[name] = value, self.representation[name]
            elif isinstance(value, Factorized):
                data[name], rep[name] = ops.materialize(value, self.layer_types[name]), "materialized"
            else:
                data[name], rep[name] = value.sum(dim=1), self.representation[name]
        return Gradient(rep, data, self.layer_types, {})

    def slice(self, dim: Literal["batch", "token"], index) -> Gradient:
        """Select samples or token positions of every layer (gradient.py:888-961).

        An int index keeps the axis (length 1).  A layer broadcast along the
        batch (one shared row for several samples) serves every requested
        sample with that row; batch-level parameter gradients pass through."""
        if dim not in ("batch", "token"):
            raise ValueError("dim must be 'batch' or 'token'")
        if dim == "token":
            self._require_token_axis("slicing")

        def take(x: torch.Tensor, ax: int) -> torch.Tensor:
            sel = index
            if isinstance(sel, slice):  # explicit positions along this axis (a broadcast row spans the batch)
                sel = torch.arange(self.batch_size if dim == "batch" and x.shape[ax] == 1 else x.shape[ax])[sel]
            if dim == "batch" and x.shape[ax] == 1:
                count = 1 if isinstance(sel, int) else (sel.numel() if torch.is_tensor(sel) else len(sel))
                sel = 0 if isinstance(sel, int) else torch.zeros(count, dtype=torch.long, device=x.device)
            if isinstance(sel, int):
                return x.narrow(ax, sel, 1)
            if not torch.is_tensor(sel):
                sel = torch.as_tensor(list(sel), dtype=torch.long)
            return x.index_select(ax, sel.to(device=x.device, dtype=torch.long))

        data = {}
        for name, value in self.data.items():
            if self.layer_types[name] == ops.PARAM_GRAD_TYPES:
                data[name] = value
            elif isinstance(value, Factorized):
                ax = self._sample_axis(value, dim)
                data[name] = Factorized(take(value.activation, ax), take(value.pre_activation_grad, ax),
                                        module_kwargs=value.module_kwargs, batch_first=value.batch_first)
            else:
                data[name] = take(value, self._sample_axis(value, dim))
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

    def similarity_per_token(self, other: Gradient, reduce: Literal["none", "all"] = "all"):
        """Each token position's share of the per-sample similarity
        (gradient.py:1072-1133): ``K[i, t, j]`` over this block's factorized
        ``"batch_token"`` layers (the only ones that still carry a token axis),
        so summing over ``t`` gives :meth:`similarity`'s ``(B_self, B_other)``.
        ``other``'s layer may be factorized or dense.  ``reduce="none"`` gives
        ``{layer: (B_self, T_self, B_other)}``, ``"all"`` their sum."""
        if reduce not in {"none", "all"}:
            raise ValueError("reduce must be 'none' or 'all'")
        per_layer = {}
        for name in sorted(self.layer_names & other.layer_names):
            mine = self.data[name]
            if isinstance(mine, Factorized) and self.indexing[name] == "batch_token":
                per_layer[name] = ops.cross_dot_per_token(mine, other.data[name], self.layer_types[name])
        if reduce == "none":
            return per_layer
        if not per_layer:
            raise ValueError("No shared factorized batch_token layers for per-token similarity")
        total = None
        for k in per_layer.values():
            total = k.clone() if total is None else total.add_(k)
        return total

    def __repr__(self) -> str:
        return f"Gradient(layers={sorted(self.data)}, batch={self.batch_size})"


def _pad_axis(t: torch.Tensor, length: int, axis: int, value=0) -> torch.Tensor:
    """``t`` extended to ``length`` along ``axis`` with ``value``."""
    extra = length - t.shape[axis]
    if extra <= 0:
        return t
    shape = list(t.shape)
    shape[axis] = extra
    return torch.cat([t, t.new_full(shape, value)], dim=axis)


def _pad_factor_tokens(x: Factorized, y: Factorized) -> tuple[Factorized, Factorized]:
    """Both factor pairs at the longer token count: extra positions carry an
    exactly-zero output gradient; an integer activation (token ids) is filled
    with the layer's ``padding_idx`` when it has one, else 0 (the zero gradient
    row keeps either inert)."""
    axis = 1 if x.batch_first else 0
    length = max(x.activation.shape[axis], y.activation.shape[axis])

    def extend(f: Factorized) -> Factorized:
        if f.activation.shape[axis] == length:
            return f
        fill = 0
        if not f.activation.is_floating_point():
            pad_idx = (f.module_kwargs or {}).get("padding_idx")
            fill = 0 if pad_idx is None else pad_idx
        return Factorized(_pad_axis(f.activation, length, axis, fill), _pad_axis(f.pre_activation_grad, length, axis),
                          module_kwargs=f.module_kwargs, batch_first=f.batch_first)

    return extend(x), extend(y)


def _merge_shared_rows(x: GradientData, y: GradientData, n_x: int, n_y: int, layer_type: str):
    """One shared row from two broadcast rows, weighted by the blocks' sample
    counts; returns (row, became_dense).  Identical activations let the
    factorized form average the output-gradient factor alone (the gradient is
    linear in it); otherwise the rows are averaged as materialized gradients."""
    wx, wy = float(n_x), float(n_y)
    if isinstance(x, Factorized):
        xb, yb = x.as_batch_first(), y.as_batch_first()
        if xb.activation.shape == yb.activation.shape and torch.equal(xb.activation, yb.activation):
            g = (wx * xb.pre_activation_grad + wy * yb.pre_activation_grad) / (wx + wy)
            return Factorized(xb.activation, g, module_kwargs=xb.module_kwargs, batch_first=True), False
        mx, my = ops.materialize(x, layer_type), ops.materialize(y, layer_type)
        return (wx * mx + wy * my) / (wx + wy), True
    return (wx * x + wy * y) / (wx + wy), False


@dataclass
class GradientRecord:
    """A gradient snapshot with its identity (gradient.py:1198-1237)."""

    step: int
    input_hash: str | list[str]
    gradient: Gradient
    sample_id_key: str | int | None = None
