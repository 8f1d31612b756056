"""Layer-type constants and predicates.

The strings are the reference's canonical class names
(``dattri_llm/gradient/ops/types.py:14-47``): they are keys stored with every
captured gradient, so they must be identical for a drop-in.
"""

from __future__ import annotations

LINEAR_TYPES = frozenset(
    {
        "nn.Linear",
        "nn.Bilinear",
        "nn.NonDynamicallyQuantizableLinear",
        "transformers.pytorch_utils.Conv1D",
    }
)
CONV_TYPES = frozenset({"nn.Conv1d", "nn.Conv2d", "nn.Conv3d"})
CONV_TRANSPOSE_TYPES = frozenset({"nn.ConvTranspose1d", "nn.ConvTranspose2d", "nn.ConvTranspose3d"})
NORM_TYPES = frozenset(
    {"nn.LayerNorm", "nn.RMSNorm", "nn.GroupNorm", "nn.InstanceNorm1d", "nn.InstanceNorm2d", "nn.InstanceNorm3d"}
)
TOKEN_NORM_TYPES = frozenset({"nn.LayerNorm", "nn.RMSNorm"})
EMBEDDING_TYPES = frozenset({"nn.Embedding", "nn.EmbeddingBag"})
PARAM_GRAD_TYPES = "param_grad_layers"
ALL_LAYER_TYPES = LINEAR_TYPES | CONV_TYPES | CONV_TRANSPOSE_TYPES | NORM_TYPES | EMBEDDING_TYPES


def is_linear(layer_type: str) -> bool:
    return layer_type in LINEAR_TYPES


def is_conv(layer_type: str) -> bool:
    return layer_type in CONV_TYPES


def is_conv_transpose(layer_type: str) -> bool:
    return layer_type in CONV_TRANSPOSE_TYPES


def is_norm(layer_type: str) -> bool:
    return layer_type in NORM_TYPES


def is_embedding(layer_type: str) -> bool:
    return layer_type in EMBEDDING_TYPES


def is_kfac_eligible(layer_type: str) -> bool:
    return is_linear(layer_type) or is_conv(layer_type) or is_conv_transpose(layer_type)


def canonical_class_name(module) -> str:
    """Canonical string for a module class, e.g. ``'nn.Linear'``."""
    mod = type(module).__module__
    name = type(module).__name__
    return f"nn.{name}" if mod.startswith("torch.nn") else f"{mod}.{name}"


def require_supported(layer_type: str, what: str) -> None:
    """Raise for layer families the HIP kernels do not cover."""
    if is_linear(layer_type) or layer_type in TOKEN_NORM_TYPES:
        return
    raise NotImplementedError(
        f"{what}: layer type {layer_type!r} is not covered by this operation on the MI355X kernels "
        "(the inner products and materialization cover linear, convolution, embedding and "
        "RMSNorm/LayerNorm layers; channel norms are not implemented)."
    )
