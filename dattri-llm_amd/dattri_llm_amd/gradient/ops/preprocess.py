"""Preprocessing of raw hook captures into the (a, g) form the kernels contract.

Mirrors ``dattri_llm/gradient/ops/preprocess.py`` for the layer families of the
scoring path: linear layers (bias folded as a ones column, :436-437) and token
norms (RMSNorm / LayerNorm x_hat, :366-384, computed by the ``da_norm_xhat``
kernel, with the bias augmentation of ``norm.py:95-110``) and embeddings
(``nn.Embedding`` padding positions, ``nn.EmbeddingBag`` bags spread over their
tokens, :403-416 and :126-169), convolutions (the unfolding of
``conv.py``) and channel norms (GroupNorm / InstanceNorm x_hat laid out
(B, S, C), :386-401, by the ``da_channel_norm_xhat`` kernel).

The public ``preprocess_factors`` returns exactly the reference's tensors.  The
scoring kernels never need them: :func:`final_linear` and :func:`norm_spec`
describe the same preprocessing so a kernel applies it on the fly (the bias is
an implicit ones column, x_hat is recomputed in registers).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from dattri_llm_amd import kernels
from dattri_llm_amd.gradient.ops import conv, dtypes
from dattri_llm_amd.gradient.ops.types import (
    CONV_TRANSPOSE_TYPES,
    CONV_TYPES,
    TOKEN_NORM_TYPES,
    is_linear,
    is_norm,
)

NORM_KIND = {"nn.RMSNorm": 0, "nn.LayerNorm": 1}


def to_3d(x: torch.Tensor) -> torch.Tensor:
    """(B, D) -> (B, 1, D); (B, T, D) unchanged (preprocess.py:447-455)."""
    return x.unsqueeze(1) if x.ndim == 2 else x


def extract_module_kwargs(module, layer_type: str) -> dict:
    """Minimal serialisable hyperparameters of a hooked module
    (preprocess.py:231-298)."""
    kwargs: dict = {"has_bias": getattr(module, "bias", None) is not None}
    if layer_type in ("nn.Embedding", "nn.EmbeddingBag") and getattr(module, "scale_grad_by_freq", False):
        raise NotImplementedError(
            f"{layer_type} with scale_grad_by_freq=True is not supported: the inverse-frequency "
            "gradient scaling is a whole-batch statistic that the factorized capture does not model."
        )
    if layer_type == "nn.Embedding":
        kwargs["num_embeddings"] = module.num_embeddings
        kwargs["padding_idx"] = module.padding_idx
    elif layer_type in CONV_TYPES or layer_type in CONV_TRANSPOSE_TYPES:
        for key in ("kernel_size", "stride", "padding", "dilation", "groups"):
            kwargs[key] = getattr(module, key)
    elif layer_type in ("nn.LayerNorm", "nn.RMSNorm"):
        kwargs["normalized_shape"] = tuple(module.normalized_shape)
        kwargs["eps"] = module.eps
    elif layer_type == "nn.GroupNorm":
        kwargs.update(num_groups=module.num_groups, num_channels=module.num_channels, eps=module.eps)
    elif layer_type in ("nn.InstanceNorm1d", "nn.InstanceNorm2d", "nn.InstanceNorm3d"):
        kwargs.update(num_features=module.num_features, eps=module.eps)
    elif layer_type == "nn.EmbeddingBag":
        kwargs.update(num_embeddings=module.num_embeddings, mode=module.mode, padding_idx=module.padding_idx)
    return kwargs


@dataclass(frozen=True)
class NormSpec:
    """How to normalise a token norm's raw activation inside a kernel."""

    kind: int  # 0 RMSNorm, 1 LayerNorm
    eps: float
    has_bias: bool
    width: int


def norm_spec(a: torch.Tensor, layer_type: str, module_kwargs: dict, include_bias: bool) -> NormSpec:
    """The reference's eps rule: ``eps=None`` is the raw activation dtype's
    machine epsilon (norm.py:38-39, applied before any dtype alignment)."""
    shape = tuple(module_kwargs.get("normalized_shape", (a.shape[-1],)))
    if len(shape) != 1:
        raise NotImplementedError(
            f"{layer_type} over {len(shape)} trailing axes: the norm kernels normalise the last axis only"
        )
    eps = module_kwargs["eps"]
    if eps is None:
        eps = torch.finfo(a.dtype).eps
    return NormSpec(NORM_KIND[layer_type], float(eps), bool(module_kwargs["has_bias"] and include_bias), shape[0])


def fold_norm_rows(x: torch.Tensor, width: int) -> torch.Tensor:
    """Every axis between batch and the normalised one becomes a position
    axis (norm.py:65-87): (B, ..., d) -> (B, P, d); 2-D (B, d) -> (B, 1, d)."""
    if x.ndim == 2:
        return x.unsqueeze(1)
    if x.ndim == 3:
        return x
    return x.reshape(x.shape[0], -1, width)


def channel_norm_spec(layer_type: str, module_kwargs: dict) -> tuple[int, float]:
    """(groups, eps) of a GroupNorm / InstanceNorm (preprocess.py:386-401):
    InstanceNorm normalises each channel alone."""
    if layer_type == "nn.GroupNorm":
        return int(module_kwargs["num_groups"]), float(module_kwargs["eps"])
    return int(module_kwargs["num_features"]), float(module_kwargs["eps"])


def channel_norm_factors(a, g, layer_type: str, module_kwargs: dict, include_bias: bool = True):
    """A channel norm's preprocessed factors (norm.py:120-141): x_hat and g as
    (B, S, C), with a bias ``[x_hat, 1]`` and ``[g, g]``.  x_hat comes from
    ``da_channel_norm_xhat`` in a's dtype; the rest is layout."""
    groups, eps = channel_norm_spec(layer_type, module_kwargs)
    x_hat = kernels.channel_norm_xhat(a, groups=groups, eps=eps, out_dtype=a.dtype)
    n, c = a.shape[:2]
    x_sc = x_hat.reshape(n, c, -1).transpose(1, 2).contiguous()
    g_sc = g.reshape(n, c, -1).transpose(1, 2).contiguous()
    if module_kwargs["has_bias"] and include_bias:
        return torch.cat([x_sc, torch.ones_like(x_sc)], dim=-1), torch.cat([g_sc, g_sc], dim=-1)
    return x_sc, g_sc


def final_linear(a, g, layer_type: str, module_kwargs: dict | None, include_bias: bool):
    """A linear layer's final factors without forming the ones column:
    ``(a, g, bias)`` where ``bias`` says an implicit ones column follows ``a``."""
    if module_kwargs is None:
        return a, g, False
    return a, g, bool(module_kwargs["has_bias"] and include_bias)


def preprocess_factors(
    a: torch.Tensor,
    g: torch.Tensor,
    layer_type: str,
    module_kwargs: dict | None = None,
    include_bias: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Transform raw captures into the reference's ``(a, g)`` form
    (preprocess.py:301-439)."""
    if module_kwargs is None:
        return a, g
    has_bias = module_kwargs["has_bias"] and include_bias
    if layer_type in TOKEN_NORM_TYPES:
        spec = norm_spec(a, layer_type, module_kwargs, include_bias)
        x_hat = kernels.norm_xhat(a, kind=spec.kind, eps=spec.eps, out_dtype=a.dtype)
        if x_hat.ndim > 3:
            x_hat = x_hat.reshape(x_hat.shape[0], -1, spec.width)
            g = g.reshape(g.shape[0], -1, spec.width)
        if has_bias:
            return torch.cat([x_hat, torch.ones_like(x_hat)], dim=-1), torch.cat([g, g], dim=-1)
        return x_hat, g
    if layer_type == "nn.Embedding":
        pad = module_kwargs.get("padding_idx")
        if pad is not None:
            g = g.masked_fill((a == pad).unsqueeze(-1), 0)
        return a, g
    if layer_type == "nn.EmbeddingBag":
        ids, rows = _bag_rows(a, g, module_kwargs["mode"], module_kwargs.get("padding_idx"))
        if module_kwargs.get("padding_idx") is not None:
            rows = rows.masked_fill((a == module_kwargs["padding_idx"]).unsqueeze(-1), 0)
        return a, rows.contiguous()
    if is_norm(layer_type):  # GroupNorm / InstanceNorm (preprocess.py:386-401)
        return channel_norm_factors(a, g, layer_type, module_kwargs, include_bias)
    if layer_type in CONV_TYPES or layer_type in CONV_TRANSPOSE_TYPES:
        return conv.preprocess(a, g, layer_type, module_kwargs, include_bias)
    if is_norm(layer_type) or not is_linear(layer_type):
        raise NotImplementedError(
            f"preprocess_factors: {layer_type!r} is outside the MI355X scoring path "
            "(linear, convolution, embedding and RMSNorm/LayerNorm layers)."
        )
    if has_bias:
        return torch.cat([a, torch.ones_like(a[..., :1])], dim=-1), g
    return a, g


def _bag_rows(a: torch.Tensor, g: torch.Tensor, mode: str, padding_idx):
    """An EmbeddingBag's per-bag gradient ``g (N, E)`` spread over its ``T``
    tokens (preprocess.py:126-169): the returned rows are a stride-0 ``(N, T, E)``
    view of ``g`` scaled by ``1/T`` for ``mode='mean'`` (``1/(non-pad count)``,
    at least 1, with a ``padding_idx``), and the ids have padding positions set
    to -1 (they then add nothing).  The scaling is the reference's division in
    g's dtype, done once per bag instead of once per token."""
    if mode == "max":
        raise NotImplementedError("EmbeddingBag mode='max' is not supported for factorized gradients.")
    if a.ndim != 2 or g.ndim != 2:
        raise NotImplementedError("EmbeddingBag factorization supports only 2-D inputs (N, T) without offsets.")
    t = a.shape[1]
    ids = a
    if padding_idx is not None:
        pad = a == padding_idx
        ids = a.masked_fill(pad, -1)
        if mode == "mean":
            g = g / (~pad).sum(dim=1).clamp_min(1).view(-1, 1).to(g.dtype)
    elif mode == "mean":
        g = g / t
    return ids, g.unsqueeze(1).expand(-1, t, -1)


def final_embedding(a, g, layer_type: str, module_kwargs: dict | None):
    """An embedding layer's kernel operands ``(ids, g)``: ``g`` the per-token
    gradient rows (an EmbeddingBag's per-bag rows spread as a stride-0 view),
    ``ids`` int64 with padding positions set to -1.  A negative id matches and
    scatters nothing, which is what the reference's zeroed gradient at those
    positions contributes (preprocess.py:403-408)."""
    if module_kwargs is None:
        return a, g
    if layer_type == "nn.EmbeddingBag":
        return _bag_rows(a, g, module_kwargs["mode"], module_kwargs.get("padding_idx"))
    pad = module_kwargs.get("padding_idx")
    return (a if pad is None else a.masked_fill(a == pad, -1)), g


def preprocess_factorized(f, layer_type: str, include_bias: bool = True):
    """:func:`preprocess_factors` on a ``Factorized`` (batch-first-safe)."""
    bf = f.as_batch_first()
    return preprocess_factors(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs, include_bias)


def flat_width(shape) -> int:
    return math.prod(shape)


__all__ = [
    "NormSpec",
    "extract_module_kwargs",
    "channel_norm_factors",
    "channel_norm_spec",
    "final_embedding",
    "final_linear",
    "fold_norm_rows",
    "norm_spec",
    "preprocess_factorized",
    "preprocess_factors",
    "to_3d",
]
_ = dtypes  # re-exported policy lives next door
