"""Convolution layers (``nn.Conv1d/2d/3d``, ``nn.ConvTranspose1d/2d/3d``, grouped).

A convolution's weight gradient is a linear layer's over unfolded patches
(``dattri_llm/gradient/ops/preprocess.py:301-439``):

* Conv: the input unfolded to ``(N, L, C_in*prod(k))`` (features in the
  weight's ``(channel, taps)`` order), the output gradient flattened to
  ``(N, L, C_out)``; ``dW = sum_l g_l a_l^T`` as for a linear layer, the bias a
  ones column;
* ConvTranspose: roles reversed -- the input flattened to ``(N, L, C_in)`` and
  the output gradient unfolded to ``(N, L, C_out*prod(k))``, ``dW = sum_l a_l
  g_l^T`` laid out ``(C_in, C_out*prod(k))``; the bias rides on one extra
  location and feature block (:171-228);
* groups > 1: both factors get a group axis ``(N, L, G, W/G)``; every product
  pairs group e with group e only.

The unfolding is layout work done with tensor views (a zero pad, one strided
window per spatial axis, a permute): the arithmetic then runs on the linear
kernels -- the ghost engine, the dW kernel, the score GEMM -- per group.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from dattri_llm_amd.gradient.ops.types import is_conv, is_conv_transpose


def _tuple(v, rank: int) -> tuple[int, ...]:
    return tuple(v) if isinstance(v, (tuple, list)) else (int(v),) * rank


def _pads(padding, kernel, dilation, rank: int) -> list[tuple[int, int]]:
    """(before, after) zero padding per spatial axis; 'valid' is none and
    'same' splits the window's reach with the odd element after, as torch does."""
    if padding == "valid":
        return [(0, 0)] * rank
    if padding == "same":
        out = []
        for k, d in zip(kernel, dilation):
            total = d * (k - 1)
            out.append((total // 2, total - total // 2))
        return out
    return [(p, p) for p in _tuple(padding, rank)]


def unfold_patches(x: torch.Tensor, kernel_size, stride, padding, dilation) -> torch.Tensor:
    """``(N, C, *spatial) -> (N, L, C*prod(kernel))``: every output location's
    receptive field, features ordered ``(channel, tap_1, ..., tap_r)`` and
    locations row-major over the output grid (the order of ``g.flatten(2)``).
    Zero padding (the reference pads with zeros whatever the padding mode)."""
    rank = x.dim() - 2
    kernel, step, dil = _tuple(kernel_size, rank), _tuple(stride, rank), _tuple(dilation, rank)
    pads = _pads(padding, kernel, dil, rank)
    flat = [p for pair in reversed(pads) for p in pair]  # F.pad lists the last axis first
    if any(flat):
        x = F.pad(x, flat)
    for ax in range(rank):
        reach = dil[ax] * (kernel[ax] - 1) + 1
        x = x.unfold(2 + ax, reach, step[ax])  # the window becomes the last axis
        if dil[ax] > 1:
            x = x[..., :: dil[ax]]
    n, c = x.shape[:2]
    grid = x.shape[2:2 + rank]
    order = (0, *range(2, 2 + rank), 1, *range(2 + rank, 2 + 2 * rank))
    return x.permute(order).reshape(n, math.prod(grid), c * math.prod(kernel))


def _split(x: torch.Tensor, groups: int) -> torch.Tensor:
    """Channel-major features: the groups are consecutive width blocks."""
    return x if groups == 1 else x.reshape(*x.shape[:-1], groups, x.shape[-1] // groups)


@dataclass
class ConvFactors:
    """Kernel operands of one convolution side.

    ``a`` / ``g`` are ``(B, L, Wa)`` / ``(B, L, Wg)``, or with a group axis
    ``(B, L, G, Wa)`` / ``(B, L, G, Wg)``.  ``bias``: an implicit ones column
    follows ``a`` (in every group).  ``transpose``: the weight is laid out
    ``(Wa, Wg)`` per group (ConvTranspose) instead of ``(Wg, Wa)``."""

    a: torch.Tensor
    g: torch.Tensor
    bias: bool
    transpose: bool

    @property
    def groups(self) -> int:
        return self.a.shape[2] if self.a.dim() == 4 else 1

    def group(self, e: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Group e's (B, L, W) factors (views)."""
        if self.a.dim() == 3:
            return self.a, self.g
        return self.a[:, :, e], self.g[:, :, e]


def _transpose_bias(a_flat: torch.Tensor, g_unf: torch.Tensor, g_raw: torch.Tensor, groups: int):
    """A transposed convolution's bias folded into its factors
    (preprocess.py:171-228): one extra location whose activation is a lone 1
    in an extra feature and whose gradient carries the per-channel bias
    gradient in an extra block of C_out/G features per group."""
    n, c_out = g_raw.shape[:2]
    bias_grad = g_raw.reshape(n, c_out, -1).sum(dim=2)
    grouped = a_flat.dim() == 4
    cg = c_out // groups
    lead = a_flat.shape[:2]
    shape_a = (*lead[:1], lead[1] + 1, *a_flat.shape[2:-1], a_flat.shape[-1] + 1)
    a_aug = a_flat.new_zeros(shape_a)
    a_aug[:, :-1, ..., :-1] = a_flat
    a_aug[:, -1, ..., -1] = 1
    shape_g = (*lead[:1], lead[1] + 1, *g_unf.shape[2:-1], g_unf.shape[-1] + cg)
    g_aug = g_unf.new_zeros(shape_g)
    g_aug[:, :-1, ..., :-cg] = g_unf
    g_aug[:, -1, ..., -cg:] = bias_grad.reshape(n, groups, cg) if grouped else bias_grad
    return a_aug, g_aug


def final(a, g, layer_type: str, module_kwargs: dict | None, include_bias: bool) -> ConvFactors:
    """Kernel operands of a raw capture (``module_kwargs`` given) or of final
    factors (``module_kwargs=None``: ``a``/``g`` already unfolded, 3-D or with a
    group axis, any bias already folded in)."""
    transpose = is_conv_transpose(layer_type)
    if module_kwargs is None:
        return ConvFactors(a, g, False, transpose)
    mk = module_kwargs
    groups = int(mk.get("groups", 1))
    has_bias = bool(mk["has_bias"] and include_bias)
    window = (mk["kernel_size"], mk["stride"], mk["padding"], mk["dilation"])
    n = a.shape[0]
    if transpose:
        a_flat = _split(a.reshape(n, a.shape[1], -1).transpose(1, 2), groups)
        g_unf = _split(unfold_patches(g, *window), groups)
        if a_flat.shape[1] != g_unf.shape[1]:
            raise ValueError(
                f"{layer_type}: the output gradient unfolds to {g_unf.shape[1]} locations, the input has "
                f"{a_flat.shape[1]} (output_padding is not modelled)"
            )
        if has_bias:
            a_flat, g_unf = _transpose_bias(a_flat, g_unf, g, groups)
        return ConvFactors(a_flat, g_unf, False, True)
    if not is_conv(layer_type):
        raise ValueError(f"{layer_type!r} is not a convolution")
    a_unf = _split(unfold_patches(a, *window), groups)
    g_out = _split(g.reshape(n, g.shape[1], -1).transpose(1, 2), groups)
    if a_unf.shape[1] != g_out.shape[1]:
        raise ValueError(f"{layer_type}: {a_unf.shape[1]} unfolded locations against {g_out.shape[1]} outputs")
    return ConvFactors(a_unf, g_out, has_bias, False)


def preprocess(a, g, layer_type: str, module_kwargs: dict, include_bias: bool):
    """The reference's preprocessed ``(a, g)`` tensors (explicit ones column)."""
    f = final(a, g, layer_type, module_kwargs, include_bias)
    x, y = f.a.contiguous(), f.g.contiguous()
    if f.bias:
        x = torch.cat([x, torch.ones_like(x[..., :1])], dim=-1)
    return x, y
