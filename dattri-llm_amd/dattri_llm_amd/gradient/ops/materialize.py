"""Per-sample weight gradients of factorized captures (materialized form).

Mirrors ``dattri_llm/gradient/ops/materialize.py:22-146`` for linear layers
(``bmm(g^T, a)`` flattened to ``(B, out*in)``, index ``o*K + i``, with the bias
column last), convolutions (per group, the transposed layout for
ConvTranspose, :100-114), token norms (``sum_t x_hat * g``, and ``[dgamma, dbeta]`` with
a bias) and embeddings (the scatter-add into ``(B, vocab*E)``, run by
``da_materialize_embedding``).  The linear case runs the ``da_materialize_linear`` MFMA kernel; the
norm case runs ``da_norm_weight_grad``, which normalises in registers and never
forms x_hat.  Results are in the resolved compute dtype with fp32 accumulation.
"""

from __future__ import annotations

import warnings

import torch

from dattri_llm_amd import kernels
from dattri_llm_amd.gradient.ops import conv, dtypes
from dattri_llm_amd.gradient.ops import embedding as emb
from dattri_llm_amd.gradient.ops.preprocess import (
    channel_norm_factors,
    channel_norm_spec,
    final_linear,
    fold_norm_rows,
    norm_spec,
    to_3d,
)
from dattri_llm_amd.gradient.ops.types import (
    TOKEN_NORM_TYPES,
    is_conv,
    is_conv_transpose,
    is_embedding,
    is_linear,
    is_norm,
    require_supported,
)


def _operands(*tensors):
    """Align to the compute dtype; kernels read fp32 for a float64 policy."""
    aligned = dtypes.align(*tensors)
    out_dtype = aligned[0].dtype
    kd = dtypes.kernel_dtype(out_dtype)
    return tuple(t.to(kd) for t in aligned), out_dtype


def norm_grad_from_raw(x, g, layer_type: str, module_kwargs: dict, include_bias: bool = True, fp32: bool = False):
    """Fused preprocess + token sum of a raw norm capture -> (B, d[*2]):
    token norms normalise each row in registers (``da_norm_weight_grad``);
    channel norms take their (sample, group) statistics first
    (``da_channel_norm_weight_grad``).  ``fp32`` keeps the sums in fp32 (for
    an inner product that follows) instead of the compute dtype."""
    if layer_type not in TOKEN_NORM_TYPES:
        groups, eps = channel_norm_spec(layer_type, module_kwargs)
        bias = bool(module_kwargs["has_bias"] and include_bias)
        (xo, go), out_dtype = _operands(x, g)
        out = kernels.channel_norm_weight_grad(xo, go, groups=groups, eps=eps, bias=bias,
                                               out_dtype=torch.float32 if fp32 else dtypes.kernel_dtype(out_dtype))
        return out if fp32 else out.to(out_dtype)
    spec = norm_spec(x, layer_type, module_kwargs, include_bias)
    x3 = fold_norm_rows(x, spec.width)
    g3 = fold_norm_rows(g, spec.width)
    (xo, go), out_dtype = _operands(x3, g3)
    out = kernels.norm_weight_grad(xo, go, kind=spec.kind, eps=spec.eps, bias=spec.has_bias,
                                   out_dtype=torch.float32 if fp32 else dtypes.kernel_dtype(out_dtype))
    return out if fp32 else out.to(out_dtype)


def norm_grad_from_final(a, g, fp32: bool = False):
    """Token sum ``(a * g).sum(1)`` of already-preprocessed norm factors
    (kept in fp32 with ``fp32``)."""
    (ao, go), out_dtype = _operands(to_3d(a), to_3d(g))
    out = kernels.norm_weight_grad(ao, go, kind=kernels.NORM_KIND_GIVEN, eps=0.0, bias=False,
                                   out_dtype=torch.float32 if fp32 else dtypes.kernel_dtype(out_dtype))
    return out if fp32 else out.to(out_dtype)


def linear_dense(a, g, bias: bool) -> torch.Tensor:
    """(B, D*(K+bias)) per-sample dW of linear factors, in the compute dtype."""
    (ao, go), out_dtype = _operands(to_3d(a), to_3d(g))
    out = kernels.materialize_linear(ao, go, bias=bias, out_dtype=dtypes.kernel_dtype(out_dtype))
    return out.to(out_dtype)


def conv_dense(c) -> torch.Tensor:
    """(B, d) per-sample weight gradient of convolution factors in the kernel
    dtype of their operands (materialize.py:100-114): per group a (Wg, Wa(+1))
    block -- (Wa, Wg) for a transposed convolution -- groups in order."""
    b = c.a.shape[0]
    if c.a.dim() == 3:
        if c.transpose:
            return kernels.materialize_linear(c.g, c.a)
        return kernels.materialize_linear(c.a, c.g, bias=c.bias)
    wa, wg = c.a.shape[-1] + int(c.bias), c.g.shape[-1]
    out = torch.empty(b, c.groups, wa * wg, dtype=c.a.dtype, device=c.a.device)
    for e in range(c.groups):
        x, y = c.group(e)
        out[:, e] = kernels.materialize_linear(y, x) if c.transpose else kernels.materialize_linear(x, y, bias=c.bias)
    return out.reshape(b, -1)


def norm_token_rows(a, g, layer_type: str, module_kwargs: dict | None = None,
                    include_bias: bool = True) -> torch.Tensor:
    """(B, T, d') per-token norm gradients x_hat * g (with a bias, [x_hat * g, g]):
    the terms whose token sum is the norm weight gradient (materialize.py:96-98).
    A channel norm's rows are its spatial positions, (B, S, C)."""
    if module_kwargs is not None and layer_type not in TOKEN_NORM_TYPES:
        x3, g3 = channel_norm_factors(a, g, layer_type, module_kwargs, include_bias)
    elif module_kwargs is not None:
        spec = norm_spec(a, layer_type, module_kwargs, include_bias)
        x_hat = kernels.norm_xhat(a, kind=spec.kind, eps=spec.eps)
        x3, g3 = fold_norm_rows(x_hat, spec.width), fold_norm_rows(g, spec.width)
        if spec.has_bias:
            x3 = torch.cat([x3, torch.ones_like(x3)], dim=-1)
            g3 = torch.cat([g3, g3], dim=-1)
    else:
        x3, g3 = to_3d(a), to_3d(g)
    x3, g3 = dtypes.align(x3, g3)
    return x3 * g3


def materialize_factors(
    a: torch.Tensor,
    g: torch.Tensor,
    layer_type: str,
    module_kwargs: dict | None = None,
    include_bias: bool = True,
    per_token: bool = False,
) -> torch.Tensor:
    """Per-sample weight gradient ``(B, d)`` (materialize.py:56-116)."""
    if is_embedding(layer_type):
        if module_kwargs is None:
            raise ValueError(
                "Materializing an embedding gradient requires module_kwargs with 'num_embeddings' "
                "(the weight's vocab size cannot be inferred from the captured factors)."
            )
        vocab = int(module_kwargs["num_embeddings"])
        emb.check_ids(a, vocab=vocab)
        return emb.materialize(emb.side(a, g, layer_type, module_kwargs), vocab)
    if is_norm(layer_type):
        if per_token:
            return norm_token_rows(a, g, layer_type, module_kwargs, include_bias).flatten(1)
        if module_kwargs is not None:
            return norm_grad_from_raw(a, g, layer_type, module_kwargs, include_bias)
        return norm_grad_from_final(a, g)
    if is_conv(layer_type) or is_conv_transpose(layer_type) or (module_kwargs is None and a.ndim == 4):
        c = conv.final(a, g, layer_type, module_kwargs, include_bias)
        (x, y), out_dtype = _operands(c.a, c.g)
        return conv_dense(conv.ConvFactors(x, y, c.bias, c.transpose)).to(out_dtype)
    if not is_linear(layer_type):
        require_supported(layer_type, "materialize_factors")
    a, g, bias = final_linear(a, g, layer_type, module_kwargs, include_bias)
    return linear_dense(a, g, bias)


def materialize_blocked(f, layer_type: str, include_bias: bool = True) -> torch.Tensor:
    """:func:`materialize` for a dense copy that only the score kernel reads.

    Linear layers without a bias column whose input width is a multiple of 64
    come back in the k-blocked layout -- the ``(B, W/64, 64)`` view of a
    buffer in which block j of every sample is one contiguous run, which the
    score GEMM streams at full HBM rate.  Other layers are materialized as
    usual.  ``x.reshape(B, -1)`` recovers the reference's ``(B, d)`` matrix."""
    if isinstance(f, torch.Tensor) or not is_linear(layer_type):
        return materialize(f, layer_type, include_bias)
    bf = f.as_batch_first()
    a, g, bias = final_linear(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs,
                              include_bias)
    if bias or a.ndim == 4 or to_3d(a).shape[-1] % 64:
        return materialize(f, layer_type, include_bias)
    (ao, go), out_dtype = _operands(to_3d(a), to_3d(g))
    out = kernels.materialize_linear(ao, go, out_dtype=dtypes.kernel_dtype(out_dtype), blocked=True)
    return out.to(out_dtype)


_UNBLOCKED_GROUP_WARNED = False


def _warn_unblocked_group() -> None:
    global _UNBLOCKED_GROUP_WARNED
    if not _UNBLOCKED_GROUP_WARNED:
        _UNBLOCKED_GROUP_WARNED = True
        warnings.warn("materialize_group: the blocks of a linear layer differ in form (a dense block, a bias "
                      "column, other widths or dtypes), so the group is concatenated row-major instead of "
                      "written k-blocked; scores are unchanged, the score GEMM reads it more slowly",
                      RuntimeWarning, stacklevel=3)


def materialize_group(values: list, layer_type: str, include_bias: bool = True) -> torch.Tensor:
    """The dense form of one layer over several train blocks, stacked along the batch.

    Linear layers that :func:`materialize_blocked` writes k-blocked go block
    by block into row slices of one k-blocked buffer, so the score GEMM reads
    the stacked rows as one block with no copy; other layers are materialized
    and concatenated."""
    if len(values) == 1:
        return materialize_blocked(values[0], layer_type, include_bias)
    prepared = []
    if is_linear(layer_type):
        for f in values:
            if isinstance(f, torch.Tensor):
                break
            bf = f.as_batch_first()
            a, g, bias = final_linear(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs,
                                      include_bias)
            if bias or a.ndim == 4:
                break
            (ao, go), out_dtype = _operands(to_3d(a), to_3d(g))
            b, t, k = ao.shape
            d = go.shape[-1]
            if (k % 64 or d % (16 // ao.element_size()) or b == 0 or t == 0
                    or dtypes.kernel_dtype(out_dtype) != out_dtype):
                break
            prepared.append((ao, go, out_dtype))
    shapes = {(ao.shape[-1], go.shape[-1], ao.dtype, od) for ao, go, od in prepared}
    if len(prepared) != len(values) or len(shapes) != 1:
        if is_linear(layer_type):
            _warn_unblocked_group()
        return torch.cat([materialize(f, layer_type, include_bias) for f in values])
    k, d, _dt, out_dtype = shapes.pop()
    rows = sum(ao.shape[0] for ao, _go, _od in prepared)
    buf = kernels.blocked_storage(rows, d * k, out_dtype, prepared[0][0].device)
    r = 0
    for ao, go, _od in prepared:
        kernels.materialize_linear(ao, go, out_dtype=out_dtype, blocked=True, out=buf[r:r + ao.shape[0]])
        r += ao.shape[0]
    return buf


def materialize(f, layer_type: str, include_bias: bool = True, per_token: bool = False) -> torch.Tensor:
    """Per-sample weight gradient of one layer, whatever its form (materialize.py:119-146)."""
    if isinstance(f, torch.Tensor):
        return f.reshape(f.shape[0], -1)
    bf = f.as_batch_first()
    return materialize_factors(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs,
                               include_bias, per_token)
