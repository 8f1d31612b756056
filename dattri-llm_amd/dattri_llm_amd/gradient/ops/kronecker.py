"""K-FAC / EK-FAC preconditioning and empirical-Fisher ops on the MI355X kernels.

Same names, signatures and errors as ``dattri_llm/gradient/ops/kronecker.py``
for the K-FAC-eligible families: linear, convolution and transposed
convolution layers, a grouped convolution with one covariance per group
(``(G, K, K)`` factors).  Where the arithmetic lives:

* token-axis contractions -- the K-FAC covariances ``a^T a`` / ``g^T g`` over
  every token row, the empirical Fisher ``grad^T grad`` over samples, the
  EK-FAC eigenbasis coordinates -- run the symmetric row-Gram kernel or the
  per-sample dW kernel (``da_materialize_linear``) with the whole row set as
  one sample (a grouped convolution: each group as one sample), fp32 out;
* the whitened cross-gram runs ``cross_gram`` (ghost / materialized kernels);
* right-multiplications by a ``(K, K)`` inverse or eigenbasis are plain
  library GEMMs (``torch.matmul``), eigendecompositions and Cholesky factors
  are ``torch.linalg`` -- one-off per fit, not on the scoring loop.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import TYPE_CHECKING

import torch

from dattri_llm_amd import kernels
from dattri_llm_amd.gradient.ops import dtypes
from dattri_llm_amd.gradient.ops.dot import cross_gram
from dattri_llm_amd.gradient.ops.materialize import materialize, materialize_factors
from dattri_llm_amd.gradient.ops.preprocess import preprocess_factors
from dattri_llm_amd.gradient.ops.types import (
    is_conv,
    is_conv_transpose,
    is_embedding,
    is_linear,
    is_norm,
    require_supported,
)

if TYPE_CHECKING:
    from collections.abc import Iterable

    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

# rows per call of the row-Gram kernel: keeps each operand under 1 GiB
_GRAM_BYTES = 1 << 30


def _require_kfac_eligible(layer_type: str) -> None:
    if is_norm(layer_type):
        raise NotImplementedError("K-FAC is not defined for normalization layers")
    if is_embedding(layer_type):
        raise NotImplementedError("K-FAC is not defined for embedding layers")
    if not (is_linear(layer_type) or is_conv(layer_type) or is_conv_transpose(layer_type)):
        require_supported(layer_type, "K-FAC")


def _flatten_for_kfac(a: torch.Tensor, g: torch.Tensor, layer_type: str):
    """kronecker.py:33-53: token rows ``(N, K)``, ``(N, D)`` in the aligned
    dtype; a grouped convolution's ``(B, L, G, K)`` factors give ``(G, N, K)``
    rows, one row set per group."""
    _require_kfac_eligible(layer_type)
    a, g = dtypes.align(a, g)
    if a.ndim == 4:
        groups = a.shape[2]
        return (a.permute(2, 0, 1, 3).reshape(groups, -1, a.shape[-1]).contiguous(),
                g.permute(2, 0, 1, 3).reshape(groups, -1, g.shape[-1]).contiguous())
    return a.reshape(-1, a.shape[-1]), g.reshape(-1, g.shape[-1])


def _sequence_rows(layer_type: str) -> bool:
    """Gradient-free rows are padding only for sequence layers; a convolution's
    zero-gradient positions are architectural and stay (kronecker.py:104-108)."""
    return not (is_conv(layer_type) or is_conv_transpose(layer_type))


def _right_multiply(x: torch.Tensor, matrix: torch.Tensor) -> torch.Tensor:
    """kronecker.py:56-62: ``x @ matrix`` on the feature axis (a plain GEMM);
    per group when *matrix* is a ``(G, K, J)`` stack and *x* a grouped
    ``(..., G, K)`` factor."""
    if matrix.ndim == 3:
        return torch.matmul(x.unsqueeze(-2), matrix).squeeze(-2)
    return x @ matrix


def _drop_gradient_free_rows(a_f: torch.Tensor, g_f: torch.Tensor):
    """kronecker.py:65-81: drop token rows whose output gradient is exactly zero."""
    keep = kernels.nonzero_rows(g_f) if g_f.dtype in (torch.bfloat16, torch.float16, torch.float32) \
        else (g_f != 0).any(dim=1)
    if bool(keep.all()):
        return a_f, g_f
    return a_f[keep], g_f[keep]


def row_gram(x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 ``x^T y`` over the rows of ``x (N, p)`` and ``y (N, q)`` -> ``(p, q)``.

    ``y`` omitted (``x^T x``, 16-bit rows): ``da_row_gram``, which computes the
    tiles on or above the diagonal once and mirrors them.  Otherwise the
    per-sample dW kernel with all N rows as one sample (it computes
    ``sum_t y[t, o] x[t, k]`` into index ``o*p + k``), in row chunks below
    1 GiB that are added in fp32."""
    y = x if y is None else y
    if x.ndim != 2 or y.ndim != 2 or x.shape[0] != y.shape[0]:
        raise ValueError("row_gram expects (N, p) and (N, q) with the same N")
    same = y is x
    x, y = dtypes.align(x, y)
    kd = dtypes.kernel_dtype(x.dtype)
    x, y = x.to(kd), y.to(kd)
    if same and kd in (torch.bfloat16, torch.float16):
        return kernels.row_gram(x)  # the symmetric kernel: tiles on or above the diagonal, mirrored
    n, p, q = x.shape[0], x.shape[1], y.shape[1]
    out = torch.zeros(q, p, dtype=torch.float32, device=x.device)
    if n == 0 or p == 0 or q == 0:
        return out.t()
    rows = max(1, _GRAM_BYTES // (max(p, q) * x.element_size()))
    for r0 in range(0, n, rows):
        xs, ys = x[r0:r0 + rows], y[r0:r0 + rows]
        part = kernels.materialize_linear(xs.unsqueeze(0), ys.unsqueeze(0), out_dtype=torch.float32)
        out += part.view(q, p)
    # symmetric when y is x; otherwise out is y^T x, so transpose to x^T y
    return out.t()


def _grams(x: torch.Tensor) -> torch.Tensor:
    """fp32 ``x^T x`` of ``(N, p)`` rows, or per group of ``(G, N, p)`` rows
    -> ``(G, p, p)``: the dW kernel with each group as one sample, in row
    chunks below 1 GiB added in fp32."""
    if x.ndim == 2:
        return row_gram(x)
    kd = dtypes.kernel_dtype(x.dtype)
    x = x.to(kd)
    groups, n, p = x.shape
    out = torch.zeros(groups, p * p, dtype=torch.float32, device=x.device)
    if n == 0 or p == 0:
        return out.view(groups, p, p)
    rows = max(1, _GRAM_BYTES // max(1, groups * p * x.element_size()))
    for r0 in range(0, n, rows):
        xs = x[:, r0:r0 + rows]
        out += kernels.materialize_linear(xs, xs, out_dtype=torch.float32)
    return out.view(groups, p, p)


def kfac_factors(
    a: torch.Tensor,
    g: torch.Tensor,
    layer_type: str,
    module_kwargs: dict | None = None,
    include_bias: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return the fp32 K-FAC covariances ``(A, G)`` (kronecker.py:84-118):
    ``a^T a / N`` and ``g^T g / N`` over the token rows that carry a gradient."""
    a, g = preprocess_factors(a, g, layer_type, module_kwargs, include_bias)
    a_f, g_f = _flatten_for_kfac(a, g, layer_type)
    if _sequence_rows(layer_type):
        a_f, g_f = _drop_gradient_free_rows(a_f, g_f)
    n = a_f.shape[-2]
    if n == 0:
        raise ValueError(
            "K-FAC factors are undefined: every token row carries a zero "
            "gradient (fully padded / masked input).",
        )
    return _grams(a_f) / n, _grams(g_f) / n


def fim_factors(
    a: torch.Tensor,
    g: torch.Tensor,
    layer_type: str,
    module_kwargs: dict | None = None,
    include_bias: bool = True,
) -> torch.Tensor:
    """The fp32 ``(d, d)`` empirical Fisher ``grad^T grad / B`` of the
    per-sample gradients (kronecker.py:121-141)."""
    grad = materialize_factors(a, g, layer_type, module_kwargs, include_bias)  # (B, d)
    return row_gram(grad) / grad.shape[0]


def sym_inverse(matrix: torch.Tensor, damping: float = 0.0) -> torch.Tensor:
    """Damped symmetric inverse through the eigendecomposition (kronecker.py:144-152)."""
    evals, evecs = torch.linalg.eigh(matrix.float())
    return (evecs / (evals + damping).unsqueeze(-2)) @ evecs.transpose(-1, -2)


def dense_inverse(matrix: torch.Tensor, damping: float = 0.0) -> torch.Tensor:
    """Damped inverse through Cholesky, falling back to :func:`sym_inverse`
    (kronecker.py:155-175)."""
    m = matrix.float()
    damped = m + damping * torch.eye(m.shape[-1], device=m.device, dtype=m.dtype)
    try:
        return torch.cholesky_inverse(torch.linalg.cholesky(damped))
    except RuntimeError:
        return sym_inverse(matrix, damping)


def kfac_cross_factors(
    a1: torch.Tensor,
    g1: torch.Tensor,
    a2: torch.Tensor,
    g2: torch.Tensor,
    layer_type: str,
    A_inv: torch.Tensor,  # noqa: N803
    G_inv: torch.Tensor,  # noqa: N803
    module_kwargs1: dict | None = None,
    module_kwargs2: dict | None = None,
    include_bias: bool = True,
) -> torch.Tensor:
    """``K[i, j] = vec(dW1_i)^T (A^-1 (x) G^-1) vec(dW2_j)`` (kronecker.py:178-202):
    side 1's factors whitened by the inverses, then :func:`cross_gram`."""
    _require_kfac_eligible(layer_type)
    a1, g1 = preprocess_factors(a1, g1, layer_type, module_kwargs1, include_bias)
    a2, g2 = preprocess_factors(a2, g2, layer_type, module_kwargs2, include_bias)
    a1 = _right_multiply(a1.float(), A_inv.float())
    g1 = _right_multiply(g1.float(), G_inv.float())
    return cross_gram(a1, g1, a2, g2, layer_type)


def kfac_eigh(A: torch.Tensor, G: torch.Tensor):  # noqa: N803
    """Eigendecompose both K-FAC factors: ``(s_A, U_A, s_G, U_G)`` (kronecker.py:205-212)."""
    s_a, u_a = torch.linalg.eigh(A.float())
    s_g, u_g = torch.linalg.eigh(G.float())
    return s_a, u_a, s_g, u_g


def ekfac_materialize_factors(
    a: torch.Tensor,
    g: torch.Tensor,
    layer_type: str,
    U_A: torch.Tensor,  # noqa: N803
    U_G: torch.Tensor,  # noqa: N803
    module_kwargs: dict | None = None,
    include_bias: bool = True,
) -> torch.Tensor:
    """``(B, d_out*d_in)`` of ``U_G^T dW U_A``: the factors rotated into the
    eigenbasis, then the per-sample dW kernel (kronecker.py:215-233)."""
    _require_kfac_eligible(layer_type)
    a, g = preprocess_factors(a, g, layer_type, module_kwargs, include_bias)
    a = _right_multiply(a.float(), U_A.float())
    g = _right_multiply(g.float(), U_G.float())
    return materialize_factors(a, g, layer_type)


def kfac(f: Factorized, layer_type: str, include_bias: bool = True):
    """:func:`kfac_factors` on a :class:`Factorized` (kronecker.py:236-249)."""
    bf = f.as_batch_first()
    return kfac_factors(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs, include_bias)


def fim(f: Factorized, layer_type: str, include_bias: bool = True) -> torch.Tensor:
    """:func:`fim_factors` on a :class:`Factorized` (kronecker.py:252-265)."""
    bf = f.as_batch_first()
    return fim_factors(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs, include_bias)


def kfac_cross(
    f1: Factorized,
    f2: Factorized,
    layer_type: str,
    A_inv: torch.Tensor,  # noqa: N803
    G_inv: torch.Tensor,  # noqa: N803
    include_bias: bool = True,
) -> torch.Tensor:
    """:func:`kfac_cross_factors` on two :class:`Factorized` (kronecker.py:268-289)."""
    b1, b2 = f1.as_batch_first(), f2.as_batch_first()
    return kfac_cross_factors(
        b1.activation, b1.pre_activation_grad, b2.activation, b2.pre_activation_grad, layer_type,
        A_inv, G_inv, b1.module_kwargs, b2.module_kwargs, include_bias,
    )


def ekfac_materialize(
    f,
    layer_type: str,
    U_A: torch.Tensor,  # noqa: N803
    U_G: torch.Tensor,  # noqa: N803
    include_bias: bool = True,
) -> torch.Tensor:
    """:func:`ekfac_materialize_factors` on a :class:`Factorized`, or the same
    rotation of an already materialized ``(B, d_out*d_in)`` block
    (kronecker.py:292-320)."""
    if isinstance(f, torch.Tensor):
        return _ekfac_rotate_materialized(f, layer_type, U_A, U_G)
    bf = f.as_batch_first()
    return ekfac_materialize_factors(
        bf.activation, bf.pre_activation_grad, layer_type, U_A, U_G, bf.module_kwargs, include_bias,
    )


def _t(u: torch.Tensor) -> torch.Tensor:
    """fp32 transpose of the last two axes, as a contiguous operand."""
    return u.float().transpose(-1, -2).contiguous()


def _layout(block: torch.Tensor, layer_type: str, U_A: torch.Tensor, U_G: torch.Tensor):  # noqa: N803
    """The rows of a materialized block as matrices, and the bases on their
    left and right: linear and conv blocks are ``(d_out, d_in)``-major (U_G on
    the left), conv-transpose blocks ``(C_in, P)``-major (U_A on the left); a
    grouped block holds one such matrix per group (materialize.py:100-114)."""
    left, right = (U_A, U_G) if is_conv_transpose(layer_type) else (U_G, U_A)
    batch = block.shape[0]
    if U_A.ndim == 3:
        shape = (batch, U_A.shape[0], left.shape[-2], right.shape[-2])
    else:
        shape = (batch, left.shape[-2], right.shape[-2])
    return block.reshape(shape).float(), left.float(), right.float()


def _ekfac_rotate_materialized(block, layer_type, U_A, U_G):  # noqa: N803
    """``vec(U_G^T dW U_A)`` per row of a materialized ``(B, D)`` block
    (kronecker.py:323-354; ``U_A^T dW U_G`` for a conv-transpose block, per
    group for a grouped one), as two fp32 GEMMs."""
    d_w, left, right = _layout(block, layer_type, U_A, U_G)
    return (torch.matmul(_t(left), d_w) @ right).reshape(block.shape[0], -1)


def kfac_precondition(
    f: Factorized,
    layer_type: str,
    A_inv: torch.Tensor,  # noqa: N803
    G_inv: torch.Tensor,  # noqa: N803
    include_bias: bool = True,
):
    """The preprocessed ``(a @ A^-1, g @ G^-1)`` of one side (kronecker.py:357-383):
    a cross-gram of these against a raw side equals :func:`kfac_cross`."""
    bf = f.as_batch_first()
    _require_kfac_eligible(layer_type)
    a, g = preprocess_factors(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs,
                              include_bias)
    return _right_multiply(a.float(), A_inv.float()), _right_multiply(g.float(), G_inv.float())


def kfac_precondition_materialized(block, A_inv, G_inv):  # noqa: N803
    """``vec(G^-1 dW A^-1)`` per row of a ``(B, k_g*k_a)`` block (kronecker.py:386-410)."""
    batch = block.shape[0]
    k_g, k_a = G_inv.shape[-1], A_inv.shape[-1]
    shape = (batch, A_inv.shape[0], k_g, k_a) if A_inv.ndim == 3 else (batch, k_g, k_a)
    d_w = block.reshape(shape).float()
    return (torch.matmul(G_inv.float(), d_w) @ A_inv.float()).reshape(batch, -1)


def ekfac_precondition(M, U_A, U_G, lam, layer_type: str):  # noqa: N803
    """``U_G (M / lam) U_A^T`` back in the original basis, flattened like
    :func:`materialize_factors` (kronecker.py:413-458; ``U_A (M / lam) U_G^T``
    for a conv-transpose block, per group for a grouped one)."""
    m3, left, right = _layout(M / lam, layer_type, U_A, U_G)
    return (torch.matmul(left, m3) @ _t(right)).reshape(M.shape[0], -1)


def _all_reduce_sum(t: torch.Tensor) -> torch.Tensor:
    """A no-op in a single process (``utils/distributed.py``'s contract outside a
    distributed context); this build runs on one GPU and has no collective path."""
    dist = torch.distributed
    if dist.is_available() and dist.is_initialized() and dist.get_world_size() > 1:
        raise NotImplementedError("cross-rank reduction is outside this one-GPU build")
    return t


# ---------------------------------------------------------------------------
# streaming accumulators (kronecker.py:460-748)
# ---------------------------------------------------------------------------


def _accumulate_gram(acc: torch.Tensor | None, x: torch.Tensor) -> torch.Tensor:
    """``acc + x^T x`` in fp32: the product itself when ``acc`` is None (no
    zero fill), else added into ``acc`` -- in the kernel's epilogue for 16-bit
    rows."""
    if acc is None:
        return _grams(x)
    if x.ndim == 3:
        acc += _grams(x)
        return acc
    if x.dtype in (torch.bfloat16, torch.float16) and acc.dtype == torch.float32 and acc.is_contiguous():
        kernels.row_gram(x, out=acc, accumulate=True)
    else:
        acc += row_gram(x)
    return acc


@dataclass
class LayerKroneckerAccumulator:
    """Streaming K-FAC covariance sums of one layer (kronecker.py:460-550)."""

    _A: torch.Tensor | None = field(default=None, init=False, repr=False)
    _G: torch.Tensor | None = field(default=None, init=False, repr=False)
    _n: int = field(default=0, init=False, repr=False)

    def update(self, a, g, layer_type: str, module_kwargs: dict | None = None, include_bias: bool = True):
        a, g = preprocess_factors(a, g, layer_type, module_kwargs, include_bias)
        a_f, g_f = _flatten_for_kfac(a, g, layer_type)
        if _sequence_rows(layer_type):
            a_f, g_f = _drop_gradient_free_rows(a_f, g_f)
        self._A = _accumulate_gram(self._A, a_f)
        self._G = _accumulate_gram(self._G, g_f)
        self._n += a_f.shape[-2]

    def all_reduce(self) -> None:
        if self._A is None:
            raise RuntimeError("No gradient-carrying data has been accumulated")
        _all_reduce_sum(self._A)
        _all_reduce_sum(self._G)

    def result(self, *, consume: bool = False):
        if self._A is None or self._n == 0:
            raise RuntimeError("No gradient-carrying data has been accumulated")
        if not consume:
            return self._A / self._n, self._G / self._n
        a, g = self._A.div_(self._n), self._G.div_(self._n)
        self.reset()
        return a, g

    def reset(self) -> None:
        self._A = None
        self._G = None
        self._n = 0


@dataclass
class LayerFisherAccumulator:
    """Streaming empirical Fisher of one layer (kronecker.py:553-620)."""

    _F: torch.Tensor | None = field(default=None, init=False, repr=False)
    _n: int = field(default=0, init=False, repr=False)

    def update(self, a, g, layer_type: str, module_kwargs: dict | None = None, include_bias: bool = True):
        self.update_from_grad(materialize_factors(a, g, layer_type, module_kwargs, include_bias))

    def update_from_grad(self, grad: torch.Tensor) -> None:
        if self._F is None:
            self._F = torch.zeros(grad.shape[-1], grad.shape[-1], dtype=grad.dtype, device=grad.device)
        self._F += row_gram(grad).to(self._F.dtype)
        self._n += grad.shape[0]

    def all_reduce(self) -> None:
        if self._F is None:
            raise RuntimeError("No data has been accumulated")
        _all_reduce_sum(self._F)

    def result(self) -> torch.Tensor:
        if self._F is None:
            raise RuntimeError("No data has been accumulated")
        return self._F / self._n

    def reset(self) -> None:
        self._F = None
        self._n = 0


class KroneckerAccumulator:
    """K-FAC covariance accumulators across layers (kronecker.py:625-688)."""

    def __init__(self) -> None:
        self._layers: dict[str, LayerKroneckerAccumulator] = {}

    def update(self, gradient: Gradient, layers: Iterable[str]) -> None:
        for name in layers:
            value = gradient.data[name]
            if isinstance(value, torch.Tensor):
                raise TypeError(
                    f"K-FAC covariances need factorized (activation, output-gradient) factors, but layer "
                    f"{name!r} holds a materialized tensor (e.g. a TRAK-projected or param_grad capture). "
                    "Exclude it from the K-FAC layer set.",
                )
            bf = value.as_batch_first()
            self._layers.setdefault(name, LayerKroneckerAccumulator()).update(
                bf.activation, bf.pre_activation_grad, gradient.layer_types[name], bf.module_kwargs,
            )

    def all_reduce(self) -> None:
        for name in sorted(self._layers):
            self._layers[name].all_reduce()

    def result(self, *, consume: bool = False):
        out = {name: acc.result(consume=consume) for name, acc in self._layers.items()}
        if consume:
            self._layers = {}
        return out


class FisherAccumulator:
    """Empirical-Fisher accumulators across layers, with a parameter cap
    (kronecker.py:691-748)."""

    def __init__(self, max_params: int | None = None) -> None:
        self._max_params = max_params
        self._layers: dict[str, LayerFisherAccumulator] = {}
        self._skipped: dict[str, int] = {}

    def update(self, gradient: Gradient, layers: Iterable[str]) -> None:
        for name in layers:
            if name in self._skipped:
                continue
            value = gradient.data[name]
            if isinstance(value, torch.Tensor):
                g = value.reshape(value.shape[0], -1).float()
            else:
                g = materialize(value, gradient.layer_types[name])
            if self._max_params is not None and g.shape[-1] > self._max_params:
                self._skipped[name] = g.shape[-1]
                self._layers.pop(name, None)
                continue
            self._layers.setdefault(name, LayerFisherAccumulator()).update_from_grad(g)

    def all_reduce(self) -> None:
        for name in sorted(self._layers):
            self._layers[name].all_reduce()

    def result(self) -> dict[str, torch.Tensor]:
        return {name: acc.result() for name, acc in self._layers.items()}

    @property
    def skipped(self) -> dict[str, int]:
        return dict(self._skipped)


__all__ = [
    "FisherAccumulator",
    "KroneckerAccumulator",
    "LayerFisherAccumulator",
    "LayerKroneckerAccumulator",
    "dense_inverse",
    "ekfac_materialize",
    "ekfac_materialize_factors",
    "ekfac_precondition",
    "fim",
    "fim_factors",
    "kfac",
    "kfac_cross",
    "kfac_cross_factors",
    "kfac_eigh",
    "kfac_factors",
    "kfac_precondition",
    "kfac_precondition_materialized",
    "row_gram",
    "sym_inverse",
]
