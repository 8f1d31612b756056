"""numpy restatement of dattri-llm's gradient-scoring ops (TEST INFRASTRUCTURE ONLY).

Reference: TRAIS-Lab/dattri-llm 0.1.0, paths relative to its repository root.
Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.

Each function below says which reference lines it restates and how it is
pinned (tests/test_oracle.py):

=============================  =============================================  ===========================================
function                       reference                                      pinned by
=============================  =============================================  ===========================================
cross_gram_factorized          gradient/ops/dot.py:115-118                    brute-force loops; torch autograd per-sample
                                                                              grads (linear layer, with bias)
cross_gram_materialized        gradient/ops/dot.py:110-114                    equals the factorized form; autograd
cross_gram                     gradient/ops/dot.py:36-118 (linear, norm)      the two above + norm branch vs autograd
cross_gram_per_token           gradient/ops/dot.py:171-222 (linear, norm)     brute-force loops over (i, t, j, s); the
                                                                              sum over t equals cross_gram (dot.py:181-183)
cross_gram_per_token_dense     gradient/ops/dot.py:225-263 (linear, norm)     equals cross_gram_per_token with m2 =
                                                                              materialize_linear of side 2
materialize_linear             gradient/ops/materialize.py:114-116,           torch autograd weight.grad (+ bias.grad)
                               preprocess.py:436-437                          flattened o*K+i layout
rms_x_hat / layer_norm_x_hat   gradient/ops/norm.py:25-41, :10-22             torch.nn.functional.rms_norm / layer_norm
                                                                              (eps=None -> machine eps special case)
norm_weight_grad               materialize.py:96-98 + preprocess.py:366-384   autograd of nn.RMSNorm / nn.LayerNorm
                               + norm.py:95-110
project                        gradient/ops/projection.py:363-370            ones-column identity: addmm(bias) ==
                                                                              cat([x,1]) @ P
project_outer                  hooks/hooks.py:631-648, projection.py:423-489  Kronecker identity
                                                                              vec(P_out^T dW P_in) vs materialize_linear
score_gemm                     gradient/ops/dot.py:114, :505, :599-604        brute-force loops
cost rules                     dot.py:728-753, projection.py:846-899          the reference's own known-answer tables
moe_router_topk                transformers MixtralTopKRouter.forward         torch.topk(torch.softmax(x.float())) on
                               (installed transformers, a library routine);   thousands of rows with tied, NaN, +-inf
                               tie order: ATen TopKImpl.h + libstdc++         logits (both selection branches)
moe_segments                   hooks/override_layers/fused_experts.py:219-228 torch.where(one_hot(idx).permute(2,1,0)[e])
moe_regroup_dense              hooks/routing.py:71-86                         explicit scatter check
moe_segment_ghost              dense-with-zeros cross_gram (routing.py:17-23) equals cross_gram on the regrouped
                                                                              zero-filled (B, T, d) factors
moe_segment_ghost_compact      the same without the zero rows                 equals moe_segment_ghost (empty experts,
                                                                              bias, one sample); brute force
match_rows                     gradient/hooks/routing.py:300-333              a gather by torch.where(mask) is recovered;
                                                                              repeated rows in ascending order; absent
                                                                              rows, surplus copies and NaN rows fail
kfac_factors                   gradient/ops/kronecker.py:65-118               brute-force sums of row outer products over
                                                                              the rows with a non-zero gradient
fim_factors                    gradient/ops/kronecker.py:121-141              brute-force sum of per-sample outer products
sym_inverse                    gradient/ops/kronecker.py:144-152              (M + damping I) @ result == I
kfac_cross_factors             gradient/ops/kronecker.py:178-202              vec(dW1)^T kron(G^-1, A^-1) vec(dW2) with the
                                                                              Kronecker matrix formed explicitly; identity
                                                                              inverses reduce to cross_gram
ekfac_materialize_factors      gradient/ops/kronecker.py:215-233              U_G^T (g^T a) U_A from materialize_linear
ekfac_rotate_materialized      gradient/ops/kronecker.py:323-354              equals ekfac_materialize_factors
ekfac_precondition             gradient/ops/kronecker.py:413-458              lam = 1 undoes the rotation (U orthogonal);
                                                                              score == vec(dW1)^T (U (x) U) diag(1/lam)
                                                                              (U (x) U)^T vec(dW2), matrices formed
kfac_precondition_materialized gradient/ops/kronecker.py:386-410              kron(G^-1, A^-1) @ vec(dW)
conv_unfold                    gradient/ops/preprocess.py:33-106 (im2col)     materialized through conv_preprocess:
conv_preprocess                gradient/ops/preprocess.py:171-228, :417-433   autograd weight.grad (+ bias.grad) of
conv_materialize               gradient/ops/materialize.py:100-114            nn.Conv1d/2d/3d and nn.ConvTranspose1d/2d
                                                                              (stride, padding, dilation, groups, bias)
grouped_cross_gram             gradient/ops/dot.py:100-109                    equals conv_materialize M1 @ M2^T
grouped_cross_gram_per_token   gradient/ops/dot.py:216-218                    sums over t to grouped_cross_gram; brute force
group_norm_x_hat               gradient/ops/norm.py:44-62                     torch.nn.functional.group_norm (no affine),
                                                                              InstanceNorm as one group per channel
channel_norm_preprocess        gradient/ops/norm.py:120-141,                  token sum of a * g equals autograd
                               preprocess.py:386-401                          [weight.grad, bias.grad] of nn.GroupNorm /
                                                                              nn.InstanceNorm2d(affine=True) per sample
embedding_materialize          gradient/ops/materialize.py:22-48              torch autograd weight.grad of nn.Embedding
                                                                              (f64); torch's CPU scatter_add_ in bf16 /
                                                                              fp16 / fp32, bit for bit (per-add rounding)
embedding_bag_expand           gradient/ops/preprocess.py:126-169             materialized: autograd of nn.EmbeddingBag
                                                                              (sum / mean, with and without padding_idx)
embedding_cross_gram           gradient/ops/dot.py:58-74                      brute-force loops; M1 @ M2^T of autograd
                                                                              per-sample weight grads
embedding_cross_gram_per_token gradient/ops/dot.py:189-203                    brute-force loops; the sum over t equals
                                                                              embedding_cross_gram
embedding_per_token_dense      gradient/ops/dot.py:239-245                    equals embedding_cross_gram_per_token with
                                                                              m2 = embedding_materialize of side 2
=============================  =============================================  ===========================================
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "cross_gram",
    "cross_gram_factorized",
    "cross_gram_materialized",
    "cross_gram_per_token",
    "cross_gram_per_token_dense",
    "conv_materialize",
    "conv_preprocess",
    "conv_unfold",
    "channel_norm_preprocess",
    "group_norm_x_hat",
    "grouped_cross_gram",
    "grouped_cross_gram_per_token",
    "ekfac_materialize_factors",
    "embedding_bag_expand",
    "embedding_cross_gram",
    "embedding_cross_gram_per_token",
    "embedding_materialize",
    "embedding_per_token_dense",
    "ekfac_precondition",
    "ekfac_rotate_materialized",
    "fim_factors",
    "kfac_cross_factors",
    "kfac_factors",
    "kfac_precondition_materialized",
    "sym_inverse",
    "layer_norm_x_hat",
    "materialize_linear",
    "match_rows",
    "maybe_materialize_projected",
    "maybe_use_materialized_gram",
    "maybe_use_materialized_norm",
    "moe_regroup_dense",
    "moe_router_topk",
    "moe_segment_ghost",
    "moe_segment_ghost_compact",
    "moe_segments",
    "norm_weight_grad",
    "preprocess",
    "project",
    "project_outer",
    "rms_x_hat",
    "score_gemm",
    "should_materialize",
    "BF16_EPS",
    "F32_EPS",
    "F16_EPS",
]

# torch.finfo(dtype).eps, the RMSNorm eps=None special case (norm.py:38-39).
F32_EPS = float(np.finfo(np.float32).eps)  # 2**-23
F16_EPS = float(np.finfo(np.float16).eps)  # 2**-10
BF16_EPS = 2.0**-7


def _with_ones(a: np.ndarray) -> np.ndarray:
    """Linear bias fold: append a ones column (preprocess.py:436-437)."""
    return np.concatenate([a, np.ones(a.shape[:-1] + (1,), dtype=a.dtype)], axis=-1)


def _to_3d(x: np.ndarray) -> np.ndarray:
    """(B, D) -> (B, 1, D) (preprocess.py:447-455)."""
    return x[:, None, :] if x.ndim == 2 else x


# ---------------------------------------------------------------------------
# cross-gram
# ---------------------------------------------------------------------------


def cross_gram_factorized(a1, g1, a2, g2, bias: bool = False) -> np.ndarray:
    """Ghost route of cross_gram (dot.py:115-118): K_a = A1 A2^T, K_g = G1 G2^T
    over the flattened (B*S) rows, Hadamard product summed per sample block.
    ``bias`` folds a ones column into both activations first."""
    a1, g1, a2, g2 = (_to_3d(x) for x in (a1, g1, a2, g2))
    if bias:
        a1, a2 = _with_ones(a1), _with_ones(a2)
    b1, s1, k = a1.shape
    b2, s2, _ = a2.shape
    d = g1.shape[-1]
    ka = a1.reshape(b1 * s1, k) @ a2.reshape(b2 * s2, k).T
    kg = g1.reshape(b1 * s1, d) @ g2.reshape(b2 * s2, d).T
    return (ka * kg).reshape(b1, s1, b2, s2).sum(axis=(1, 3))


def cross_gram_materialized(a1, g1, a2, g2, bias: bool = False) -> np.ndarray:
    """Materialized route of cross_gram (dot.py:110-114): per-sample
    ``bmm(a^T, g)`` flattened, then one GEMM."""
    a1, g1, a2, g2 = (_to_3d(x) for x in (a1, g1, a2, g2))
    if bias:
        a1, a2 = _with_ones(a1), _with_ones(a2)
    m1 = np.matmul(a1.transpose(0, 2, 1), g1).reshape(a1.shape[0], -1)
    m2 = np.matmul(a2.transpose(0, 2, 1), g2).reshape(a2.shape[0], -1)
    return m1 @ m2.T


def cross_gram(a1, g1, a2, g2, layer_type: str, mode: str = "auto", bias: bool = False):
    """cross_gram (dot.py:36-118) on preprocessed factors, for the linear and
    norm families.  Norm layers contract positions first (dot.py:80-86)."""
    if layer_type in NORM_TYPES:
        grad1 = (_to_3d(a1) * _to_3d(g1)).sum(axis=1)
        grad2 = (_to_3d(a2) * _to_3d(g2)).sum(axis=1)
        return grad1 @ grad2.T
    a1_3, a2_3 = _to_3d(a1), _to_3d(a2)
    b1, s, k = a1_3.shape
    d = _to_3d(g1).shape[-1]
    if mode == "auto":
        mode = (
            "materialized"
            if maybe_use_materialized_gram(b1, a2_3.shape[0], s, k + int(bias), d)
            else "factorized"
        )
    if mode == "materialized":
        return cross_gram_materialized(a1, g1, a2, g2, bias)
    return cross_gram_factorized(a1, g1, a2, g2, bias)


def cross_gram_per_token(a1, g1, a2, g2, layer_type: str = "nn.Linear", bias: bool = False) -> np.ndarray:
    """cross_gram_per_token (dot.py:171-222) on preprocessed factors, (B1, T1, B2):
    side 2's per-sample gradient M2_j = sum_s a2_js (x) g2_js, then
    K[i, t, j] = a1_it^T M2_j g1_it (einsum "btk,btd,ckd->btc", :220-222).  Norm
    layers: (a1 * g1) against sum_s a2 * g2 (:209-214).  ``bias`` folds the
    ones column into both activations (the preprocessed linear factors)."""
    a1, g1, a2, g2 = (_to_3d(x) for x in (a1, g1, a2, g2))
    if layer_type in NORM_TYPES:
        grad2 = (a2 * g2).sum(axis=1)
        return np.einsum("btd,cd->btc", a1 * g1, grad2)
    if bias:
        a1, a2 = _with_ones(a1), _with_ones(a2)
    m2 = np.einsum("csk,csd->ckd", a2, g2)
    return np.einsum("btk,btd,ckd->btc", a1, g1, m2, optimize=True)


def cross_gram_per_token_dense(a1, g1, m2, layer_type: str = "nn.Linear", bias: bool = False) -> np.ndarray:
    """cross_gram_per_token_dense (dot.py:225-263): side 2 dense, ``m2`` (B2, D*K')
    in materialize's o*K' + i layout (K' = K + bias), reshaped to (B2, D, K');
    K[i, t, j] = einsum("btk,btd,cdk->btc") (:260-263).  Norm layers:
    einsum("btd,cd->btc", a1 * g1, m2) (:246-247)."""
    a1, g1 = _to_3d(a1), _to_3d(g1)
    b2 = m2.shape[0]
    if layer_type in NORM_TYPES:
        return np.einsum("btd,cd->btc", a1 * g1, m2.reshape(b2, -1))
    if bias:
        a1 = _with_ones(a1)
    m2 = m2.reshape(b2, g1.shape[-1], a1.shape[-1])
    return np.einsum("btk,btd,cdk->btc", a1, g1, m2, optimize=True)


# ---------------------------------------------------------------------------
# materialization and norm preprocessing
# ---------------------------------------------------------------------------


def materialize_linear(a, g, bias: bool = False) -> np.ndarray:
    """Per-sample weight gradient of a linear layer, ``bmm(g^T, a)`` flattened
    to (B, D*K) with index o*K + i (materialize.py:114-116); with ``bias`` the
    activation carries the ones column so the layout is (B, D*(K+1))."""
    a, g = _to_3d(a), _to_3d(g)
    if bias:
        a = _with_ones(a)
    return np.matmul(g.transpose(0, 2, 1), a).reshape(a.shape[0], -1)


NORM_TYPES = frozenset(
    {
        "nn.LayerNorm",
        "nn.RMSNorm",
        "nn.GroupNorm",
        "nn.InstanceNorm1d",
        "nn.InstanceNorm2d",
        "nn.InstanceNorm3d",
    }
)


def rms_x_hat(x, eps) -> np.ndarray:
    """x * rsqrt(mean(x^2) + eps) over the last axis (norm.py:25-41)."""
    mean_sq = (x * x).mean(axis=-1, keepdims=True)
    return x / np.sqrt(mean_sq + eps)


def layer_norm_x_hat(x, eps) -> np.ndarray:
    """(x - mu) / sqrt(var + eps), biased variance, last axis (norm.py:10-22)."""
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps)


def preprocess(a, g, layer_type: str, module_kwargs: dict | None, include_bias: bool = True):
    """preprocess_factors (preprocess.py:301-439) for linear, RMSNorm and
    LayerNorm over the last axis.  ``module_kwargs['eps'] is None`` must be
    resolved by the caller to the raw activation dtype's machine eps."""
    if module_kwargs is None:
        return a, g
    has_bias = module_kwargs["has_bias"] and include_bias
    if layer_type in ("nn.RMSNorm", "nn.LayerNorm"):
        fn = rms_x_hat if layer_type == "nn.RMSNorm" else layer_norm_x_hat
        x_hat = fn(a, module_kwargs["eps"])
        if has_bias:  # norm.py:95-110
            return (
                np.concatenate([x_hat, np.ones_like(x_hat)], axis=-1),
                np.concatenate([g, g], axis=-1),
            )
        return x_hat, g
    if layer_type in LINEAR_TYPES and has_bias:
        return _with_ones(a), g
    return a, g


LINEAR_TYPES = frozenset(
    {
        "nn.Linear",
        "nn.Bilinear",
        "nn.NonDynamicallyQuantizableLinear",
        "transformers.pytorch_utils.Conv1D",
    }
)


def norm_weight_grad(x, g, layer_type: str, eps: float, has_bias: bool = False) -> np.ndarray:
    """Per-sample norm weight gradient: preprocess then ``(a*g).sum(1)``
    (materialize.py:96-98).  Returns (B, d), or (B, 2d) = [dgamma, dbeta]."""
    a, gg = preprocess(x, g, layer_type, {"has_bias": has_bias, "eps": eps})
    return (_to_3d(a) * _to_3d(gg)).sum(axis=1)


# ---------------------------------------------------------------------------
# projection
# ---------------------------------------------------------------------------


def project(x, matrix, bias_row=None) -> np.ndarray:
    """ProjectionMatrix.__call__ (projection.py:363-370): ``x @ P`` over the
    last axis, plus the bias row broadcast when the layer has a bias."""
    flat = x.reshape(-1, x.shape[-1])
    out = flat @ matrix
    if bias_row is not None:
        out = out + bias_row[None, :]
    return out.reshape(*x.shape[:-1], matrix.shape[1])


def project_outer(a, g, p_in, p_out, bias: bool = False) -> np.ndarray:
    """Capture-time LoGRA projection then materialization
    (hooks.py:631-648): a_p = a @ P_in (+ bias row, P_in is (K+1, k_a) when
    ``bias``), g_p = g @ P_out, result ``bmm(g_p^T, a_p)`` flattened to
    (B, k_g*k_a) with index o*k_a + i."""
    if bias:
        a_p = project(a, p_in[:-1], p_in[-1])
    else:
        a_p = project(a, p_in)
    g_p = project(g, p_out)
    return materialize_linear(a_p, g_p)


# ---------------------------------------------------------------------------
# score GEMM
# ---------------------------------------------------------------------------


def score_gemm(m1_list, m2_list) -> np.ndarray:
    """Dense-side layer products summed over layers (dot.py:114, :505,
    :599-604): sum_L M1_L @ M2_L^T."""
    total = None
    for m1, m2 in zip(m1_list, m2_list, strict=True):
        part = m1.reshape(m1.shape[0], -1) @ m2.reshape(m2.shape[0], -1).T
        total = part if total is None else total + part
    return total


# ---------------------------------------------------------------------------
# cost rules (exact restatements; pinned by the reference's known-answer tests)
# ---------------------------------------------------------------------------


def maybe_use_materialized_gram(b1, b2, s, k, d, kappa: float = 1.0) -> bool:
    """dot.py:728-745."""
    cost_f = b1 * b2 * s * s * (d + k)
    cost_m = (b1 + b2) * s * d * k + b1 * b2 * d * k
    return kappa * cost_f >= cost_m


def maybe_use_materialized_norm(s, k, d) -> bool:
    """dot.py:748-753."""
    return s * (d + k) >= d * k


def maybe_materialize_projected(seq_len, k_a, k_g, kappa: float = 1.0) -> bool:
    """projection.py:846-874."""
    denom = k_a + k_g
    if denom <= 0:
        return False
    return seq_len >= kappa * (k_a * k_g) / denom


def should_materialize(capture_style, seq_len, k_a, k_g) -> bool:
    """projection.py:877-899."""
    if capture_style == "factorized":
        return False
    if capture_style == "materialized":
        return True
    if capture_style != "auto":
        raise ValueError(f"capture_style must be one of ('factorized', 'materialized', 'auto'), got {capture_style!r}.")
    return maybe_materialize_projected(seq_len, k_a, k_g)


# ---------------------------------------------------------------------------
# MoE routing
# ---------------------------------------------------------------------------


def _softmax_f32(logits: np.ndarray) -> np.ndarray:
    """softmax over the last axis in float32; a NaN anywhere in a row makes its
    maximum NaN (numpy's max propagates NaN, as torch's does)."""
    x = logits.astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        m = x.max(axis=-1, keepdims=True)
        e = np.exp(x - m, dtype=np.float32)
        return e / e.sum(axis=-1, keepdims=True, dtype=np.float32)


def _before(x, y) -> bool:
    """ATen's top-k order (largest first): NaN before any number, then larger
    first (torch/include/ATen/native/TopKImpl.h, topk_impl_loop)."""
    xn, yn = x[0] != x[0], y[0] != y[0]
    return (xn and not yn) or x[0] > y[0]


def _insertion_sort(q, lo, hi):
    """libstdc++ __insertion_sort / __unguarded_linear_insert on q[lo:hi]."""
    for i in range(lo + 1, hi):
        v = q[i]
        if _before(v, q[lo]):
            q[lo + 1 : i + 1] = q[lo:i]
            q[lo] = v
            continue
        j = i
        while _before(v, q[j - 1]):
            q[j] = q[j - 1]
            j -= 1
        q[j] = v


def _adjust_heap(q, first, hole, length, v):
    """libstdc++ __adjust_heap + __push_heap (root = the entry returned last)."""
    top = child = hole
    while child < (length - 1) // 2:
        child = 2 * (child + 1)
        if _before(q[first + child], q[first + child - 1]):
            child -= 1
        q[first + hole] = q[first + child]
        hole = child
    if length % 2 == 0 and child == (length - 2) // 2:
        child = 2 * (child + 1)
        q[first + hole] = q[first + child - 1]
        hole = child - 1
    while hole > top and _before(q[first + (hole - 1) // 2], v):
        q[first + hole] = q[first + (hole - 1) // 2]
        hole = (hole - 1) // 2
    q[first + hole] = v


def _heap_select(q, first, middle, last):
    """libstdc++ __heap_select: __make_heap on [first, middle), then every later
    entry that comes before the root replaces it (__pop_heap)."""
    size = middle - first
    if size >= 2:
        for parent in range((size - 2) // 2, -1, -1):
            _adjust_heap(q, first, parent, size, q[first + parent])
    for i in range(middle, last):
        if _before(q[i], q[first]):
            v = q[i]
            q[i] = q[first]
            _adjust_heap(q, first, 0, size, v)


def _sort_heap(q, first, last):
    """libstdc++ __sort_heap."""
    while last - first > 1:
        last -= 1
        v = q[last]
        q[last] = q[first]
        _adjust_heap(q, first, 0, last - first, v)


def _nth_element(q, nth):
    """libstdc++ std::nth_element (__introselect: median-of-three pivot moved to
    the front, unguarded Hoare partition, depth limit 2*floor(log2 n), then an
    insertion sort of the last range of at most 3)."""
    first, last = 0, len(q)
    if last == 0 or nth == last:
        return
    depth = 2 * (last.bit_length() - 1)
    while last - first > 3:
        if depth == 0:
            _heap_select(q, first, nth + 1, last)
            q[first], q[nth] = q[nth], q[first]
            return
        depth -= 1
        a, b, c = first + 1, first + (last - first) // 2, last - 1
        if _before(q[a], q[b]):
            m = b if _before(q[b], q[c]) else (c if _before(q[a], q[c]) else a)
        else:
            m = a if _before(q[a], q[c]) else (c if _before(q[b], q[c]) else b)
        q[first], q[m] = q[m], q[first]
        pivot, lo, hi = q[first], first + 1, last
        while True:
            while _before(q[lo], pivot):
                lo += 1
            hi -= 1
            while _before(pivot, q[hi]):
                hi -= 1
            if not lo < hi:
                break
            q[lo], q[hi] = q[hi], q[lo]
            lo += 1
        if lo <= nth:
            first = lo
        else:
            last = lo
    _insertion_sort(q, first, last)


def _topk_order(probs_row, k: int) -> list[int]:
    """The indices torch.topk(row, k) returns on the CPU: ATen's topk_impl_loop
    runs std::partial_sort when k * 64 <= n, else std::nth_element at k - 1 and
    std::sort of the first k - 1 (an insertion sort for k <= 16).  Equal values
    keep the order those algorithms leave them in."""
    q = [(float(v), j) for j, v in enumerate(probs_row)]
    if k * 64 <= len(q):
        _heap_select(q, 0, k, len(q))
        _sort_heap(q, 0, k)
    else:
        _nth_element(q, k - 1)
        _insertion_sort(q, 0, k - 1)
    return [j for _v, j in q[:k]]


def moe_router_topk(logits, k: int):
    """Mixtral top-k router (installed transformers 5.15.0,
    MixtralTopKRouter.forward): torch.topk(softmax(logits.float()), k) with the
    weights renormalised over the k.  Indices follow torch.topk's CPU order,
    ties and NaN rows included (:func:`_topk_order`).  A row holding a NaN or
    +inf logit, or only -inf logits, has NaN probabilities, as torch's softmax
    gives.  Returns (weights (N,k) float32, indices (N,k) int64)."""
    probs = _softmax_f32(np.asarray(logits))
    n = probs.shape[0]
    order = np.array([_topk_order(probs[r], k) for r in range(n)], dtype=np.int64).reshape(n, k)
    top = np.take_along_axis(probs, order, axis=-1)
    with np.errstate(invalid="ignore"):
        weights = top / top.sum(axis=-1, keepdims=True, dtype=np.float32)
    return weights.astype(np.float32), order


def moe_segments(top_idx, n_experts: int):
    """Per-expert routed rows in the reference loop's order
    (fused_experts.py:219-228): ``torch.where(one_hot(idx).permute(2,1,0)[e])``
    enumerates (top_k_pos, token_idx) slot-major, token ascending.
    Returns a list of (top_k_pos, token_idx) int64 arrays, one per expert."""
    top_idx = np.asarray(top_idx)
    out = []
    for e in range(n_experts):
        mask = (top_idx == e).T  # (k, tokens): mask[pos, token]
        pos, tok = np.nonzero(mask)  # row-major: pos-major, token ascending
        out.append((pos.astype(np.int64), tok.astype(np.int64)))
    return out


def moe_regroup_dense(rows, token_idx, batch: int, tokens: int) -> np.ndarray:
    """RowLayout.regroup (routing.py:71-86): scatter routed rows back to a
    zero-filled (B, T, d) tensor at their (sample, position)."""
    out = np.zeros((batch, tokens) + rows.shape[1:], dtype=rows.dtype)
    tok = np.asarray(token_idx)
    out[tok // tokens, tok % tokens] = rows
    return out


def moe_segment_ghost(a1, g1, tok1, a2, g2, tok2, batch1, batch2, tokens1, tokens2, bias=False):
    """One expert's factorized cross-gram under the reference's layout:
    regroup both sides' routed rows to zero-filled (B, T, d) factors
    (routing.py:71-86) and apply the ghost route (dot.py:115-118)."""
    A1 = moe_regroup_dense(a1, tok1, batch1, tokens1)
    G1 = moe_regroup_dense(g1, tok1, batch1, tokens1)
    A2 = moe_regroup_dense(a2, tok2, batch2, tokens2)
    G2 = moe_regroup_dense(g2, tok2, batch2, tokens2)
    return cross_gram_factorized(A1, G1, A2, G2, bias)


def moe_segment_ghost_compact(a1, g1, tok1, a2, g2, tok2, batch1, batch2, tokens1, tokens2, bias=False):
    """moe_segment_ghost without forming the zero rows (they are inert,
    routing.py:17-23): K_a = A1 A2^T and K_g = G1 G2^T over the routed rows
    only, their Hadamard product summed into (sample of row p, sample of row q)
    bins.  Same value, ~(B*T / rows)^2 fewer flops."""
    a1, g1, a2, g2 = (np.asarray(x, np.float64) for x in (a1, g1, a2, g2))
    if bias:
        a1, a2 = _with_ones(a1), _with_ones(a2)
    prod = (a1 @ a2.T) * (g1 @ g2.T)
    bins1 = np.zeros((batch1, len(a1)))
    bins1[np.asarray(tok1) // tokens1, np.arange(len(a1))] = 1.0
    bins2 = np.zeros((batch2, len(a2)))
    bins2[np.asarray(tok2) // tokens2, np.arange(len(a2))] = 1.0
    return bins1 @ prod @ bins2.T


# ---------------------------------------------------------------------------
# K-FAC / EK-FAC (gradient/ops/kronecker.py), on preprocessed linear factors
# ---------------------------------------------------------------------------


def kfac_factors(a, g):
    """kronecker.py:84-118 for a linear layer: over the flattened token rows
    whose output gradient is not exactly zero (:65-81), A = a^T a / N and
    G = g^T g / N.  Raises ValueError when every row is gradient-free."""
    a_f = np.asarray(a, np.float64).reshape(-1, np.shape(a)[-1])
    g_f = np.asarray(g, np.float64).reshape(-1, np.shape(g)[-1])
    keep = ~(g_f == 0).all(axis=1)
    a_f, g_f = a_f[keep], g_f[keep]
    n = a_f.shape[0]
    if n == 0:
        raise ValueError("K-FAC factors are undefined: every token row carries a zero gradient")
    return a_f.T @ a_f / n, g_f.T @ g_f / n


def fim_factors(grad):
    """kronecker.py:121-141: the empirical Fisher grad^T grad / B of per-sample
    gradients (B, d)."""
    grad = np.asarray(grad, np.float64)
    return grad.T @ grad / grad.shape[0]


def sym_inverse(m, damping: float = 0.0):
    """kronecker.py:144-152: (m + damping I)^-1 through the eigendecomposition."""
    w, v = np.linalg.eigh(np.asarray(m, np.float64))
    return (v / (w + damping)[None, :]) @ v.T


def kfac_cross_factors(a1, g1, a2, g2, a_inv, g_inv):
    """kronecker.py:178-202: side 1's preprocessed factors right-multiplied by
    A^-1 and G^-1, then the factorized cross-gram against side 2."""
    a1w = _to_3d(np.asarray(a1, np.float64)) @ np.asarray(a_inv, np.float64)
    g1w = _to_3d(np.asarray(g1, np.float64)) @ np.asarray(g_inv, np.float64)
    return cross_gram_factorized(a1w, g1w, a2, g2)


def ekfac_materialize_factors(a, g, u_a, u_g):
    """kronecker.py:215-233: per-sample dW rotated into the K-FAC eigenbasis,
    (B, D*K) of U_G^T dW U_A, from the rotated factors."""
    a = _to_3d(np.asarray(a, np.float64)) @ np.asarray(u_a, np.float64)
    g = _to_3d(np.asarray(g, np.float64)) @ np.asarray(u_g, np.float64)
    return materialize_linear(a, g)


def ekfac_rotate_materialized(block, u_a, u_g):
    """kronecker.py:323-354 (linear): U_G^T dW U_A per row of a (B, d_out*d_in) block."""
    u_a, u_g = np.asarray(u_a, np.float64), np.asarray(u_g, np.float64)
    d_w = np.asarray(block, np.float64).reshape(len(block), u_g.shape[0], u_a.shape[0])
    return np.einsum("oe,boi,if->bef", u_g, d_w, u_a).reshape(len(block), -1)


def ekfac_precondition(m, u_a, u_g, lam):
    """kronecker.py:413-458 (linear): U_G (M / lam) U_A^T, back in the original basis."""
    u_a, u_g = np.asarray(u_a, np.float64), np.asarray(u_g, np.float64)
    md = (np.asarray(m, np.float64) / np.asarray(lam, np.float64)).reshape(len(m), u_g.shape[1], u_a.shape[1])
    return np.einsum("oe,bef,if->boi", u_g, md, u_a).reshape(len(m), -1)


def kfac_precondition_materialized(block, a_inv, g_inv):
    """kronecker.py:386-410: G^-1 dW A^-1 per row of a (B, k_g*k_a) block."""
    a_inv, g_inv = np.asarray(a_inv, np.float64), np.asarray(g_inv, np.float64)
    d_w = np.asarray(block, np.float64).reshape(len(block), g_inv.shape[0], a_inv.shape[0])
    return (g_inv @ d_w @ a_inv).reshape(len(block), -1)


# ---------------------------------------------------------------------------
# embedding layers
# ---------------------------------------------------------------------------


def _round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 values rounded to ``dtype`` ("bf16", "f16", "f32") with
    round-to-nearest-even, returned as float32 (NaN stays NaN)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def embedding_materialize(tok, g, vocab: int, dtype: str = "f64") -> np.ndarray:
    """Per-sample embedding weight gradient (materialize.py:22-48): a zero
    (B, vocab, E) table, ``scatter_add_`` of the (B, T, E) gradient rows at the
    token ids along the vocab axis, flattened to (B, vocab*E).

    ``dtype`` "f64" sums exactly (float64); "f32", "bf16" and "f16" restate the
    CPU scatter_add_ in that dtype: rows are summed in fp32 in ascending t and
    the sum is rounded once to the dtype (torch's reduced-precision scatter
    accumulates in fp32).  Ids must lie in [0, vocab) (the reference raises
    ValueError above it)."""
    tok = np.asarray(tok, dtype=np.int64)
    g = np.asarray(g)
    b, t = tok.shape
    e = g.shape[-1]
    if tok.size and (tok.min() < 0 or tok.max() >= vocab):
        raise ValueError("token id out of range")
    rows = np.arange(b)
    if dtype == "f64":
        out = np.zeros((b, vocab, e), dtype=np.float64)
        for s in range(t):
            np.add.at(out, (rows, tok[:, s]), g[:, s].astype(np.float64))
        return out.reshape(b, -1)
    out = np.zeros((b, vocab, e), dtype=np.float32)
    g32 = _round_to(g.astype(np.float32), dtype)
    for s in range(t):  # one (b, id) pair per sample and step: no index collides
        out[rows, tok[:, s]] = out[rows, tok[:, s]] + g32[:, s]
    return _round_to(out, dtype).reshape(b, -1)


def embedding_bag_expand(a, g, mode: str, padding_idx=None):
    """EmbeddingBag per-bag gradients spread over the bag's tokens
    (preprocess.py:126-169): g (N, E) -> (N, T, E), divided by T for 'mean';
    with a padding_idx the pad positions get zero and the 'mean' divisor is the
    bag's non-pad count (at least 1)."""
    a = np.asarray(a, dtype=np.int64)
    g = np.asarray(g)
    n, t = a.shape
    rows = np.repeat(g[:, None, :], t, axis=1).astype(g.dtype)
    if padding_idx is not None:
        pad = a == padding_idx
        rows = np.where(pad[..., None], 0, rows)
        if mode == "mean":
            rows = rows / np.maximum((~pad).sum(axis=1), 1)[:, None, None]
    elif mode == "mean":
        rows = rows / t
    return a, rows


def embedding_cross_gram(tok1, g1, tok2, g2) -> np.ndarray:
    """Embedding branch of cross_gram (dot.py:58-74), (B1, B2):
    K[i, j] = sum_t g1_i[t] . G2_sum_j[tok1_i[t]] with
    G2_sum_j[v] = sum over s with tok2_j[s] == v of g2_j[s], i.e. the sum over
    token pairs with equal ids of g1_it . g2_js."""
    tok1, tok2 = np.asarray(tok1, dtype=np.int64), np.asarray(tok2, dtype=np.int64)
    b1, b2 = tok1.shape[0], tok2.shape[0]
    out = np.zeros((b1, b2), dtype=np.result_type(g1, g2))
    for i in range(b1):
        for j in range(b2):
            eq = tok1[i][:, None] == tok2[j][None, :]
            out[i, j] = ((g1[i] @ g2[j].T) * eq).sum()
    return out


def embedding_cross_gram_per_token(tok1, g1, tok2, g2) -> np.ndarray:
    """Embedding branch of cross_gram_per_token (dot.py:189-203), (B1, T1, B2):
    out[i, t, j] = g1_i[t] . G2_sum_j[tok1_i[t]]."""
    tok1, tok2 = np.asarray(tok1, dtype=np.int64), np.asarray(tok2, dtype=np.int64)
    b1, t1 = tok1.shape
    b2 = tok2.shape[0]
    out = np.zeros((b1, t1, b2), dtype=np.result_type(g1, g2))
    for i in range(b1):
        for j in range(b2):
            eq = tok1[i][:, None] == tok2[j][None, :]
            out[i, :, j] = ((g1[i] @ g2[j].T) * eq).sum(axis=1)
    return out


def embedding_per_token_dense(tok1, g1, m2, vocab: int) -> np.ndarray:
    """Embedding branch of cross_gram_per_token_dense (dot.py:239-245): the rows
    of side 2's (B2, vocab, E) dense gradients at side 1's ids, dotted with
    side 1's gradient rows, (B1, T1, B2)."""
    tok1 = np.asarray(tok1, dtype=np.int64)
    e = g1.shape[-1]
    m2 = np.asarray(m2).reshape(m2.shape[0], vocab, e)
    rows = m2[:, tok1.reshape(-1)].reshape(m2.shape[0], *tok1.shape, e)
    return np.einsum("bte,cbte->btc", g1, rows)


# ---------------------------------------------------------------------------
# convolutions and grouped factors
# ---------------------------------------------------------------------------


def conv_unfold(x, kernel_size, stride, padding, dilation) -> np.ndarray:
    """im2col of preprocess.py:33-106, one output location at a time:
    (N, C, *spatial) -> (N, L, C*prod(k)), zero padding, features ordered
    (channel, taps) and locations row-major over the output grid."""
    import itertools

    x = np.asarray(x)
    rank = x.ndim - 2
    ks, ss, ps, ds = (tuple(v) for v in (kernel_size, stride, padding, dilation))
    xp = np.pad(x, [(0, 0), (0, 0)] + [(p, p) for p in ps])
    outs = [(xp.shape[2 + i] - ds[i] * (ks[i] - 1) - 1) // ss[i] + 1 for i in range(rank)]
    n, c = x.shape[:2]
    cols = []
    for loc in itertools.product(*(range(o) for o in outs)):
        pos = [loc[i] * ss[i] + np.arange(ks[i]) * ds[i] for i in range(rank)]
        patch = xp[(slice(None), slice(None)) + np.ix_(*pos)]  # (N, C, k_1, ..., k_r)
        cols.append(patch.reshape(n, -1))
    return np.stack(cols, axis=1)


def conv_preprocess(a, g, transpose: bool, kernel_size, stride, padding, dilation, groups: int = 1,
                    has_bias: bool = False):
    """The preprocessed factors of a convolution (preprocess.py:417-433) or a
    transposed convolution (:171-228): 3-D, or 4-D (N, L, G, W/G) with groups;
    the conv bias a ones column per group, the transposed conv's bias an extra
    location and feature block."""
    a, g = np.asarray(a), np.asarray(g)
    n = a.shape[0]
    win = (kernel_size, stride, padding, dilation)

    def split(x):
        return x if groups == 1 else x.reshape(*x.shape[:-1], groups, x.shape[-1] // groups)

    if not transpose:
        a_f = split(conv_unfold(a, *win))
        g_f = split(g.reshape(n, g.shape[1], -1).transpose(0, 2, 1))
        if has_bias:
            a_f = np.concatenate([a_f, np.ones(a_f.shape[:-1] + (1,), dtype=a_f.dtype)], axis=-1)
        return a_f, g_f
    a_f = split(a.reshape(n, a.shape[1], -1).transpose(0, 2, 1))
    g_f = split(conv_unfold(g, *win))
    if not has_bias:
        return a_f, g_f
    c_out = g.shape[1]
    cg = c_out // groups
    bias_grad = g.reshape(n, c_out, -1).sum(axis=2)
    if groups > 1:
        bias_grad = bias_grad.reshape(n, groups, cg)
    zeros_a = np.zeros(a_f.shape[:-1] + (1,), dtype=a_f.dtype)
    a_pad = np.concatenate([a_f, zeros_a], axis=-1)
    a_row = np.zeros_like(a_pad[:, :1])
    a_row[..., -1] = 1.0
    g_pad = np.concatenate([g_f, np.zeros(g_f.shape[:-1] + (cg,), dtype=g_f.dtype)], axis=-1)
    g_row = np.zeros_like(g_pad[:, :1])
    g_row[:, 0, ..., -cg:] = bias_grad
    return np.concatenate([a_pad, a_row], axis=1), np.concatenate([g_pad, g_row], axis=1)


def conv_materialize(a, g, transpose: bool = False) -> np.ndarray:
    """Per-sample weight gradient of preprocessed convolution factors
    (materialize.py:100-114): per group (D, K) = g^T a, or (C, P) = a^T g for a
    transposed convolution, groups in order, flattened to (B, d)."""
    a, g = np.asarray(a), np.asarray(g)
    if a.ndim == 3:
        a, g = a[:, :, None], g[:, :, None]
    if transpose:
        return np.einsum("btgc,btgp->bgcp", a, g).reshape(a.shape[0], -1)
    return np.einsum("btgk,btgd->bgdk", a, g).reshape(a.shape[0], -1)


def grouped_cross_gram(a1, g1, a2, g2) -> np.ndarray:
    """Grouped factorized cross_gram (dot.py:100-109): the group axis is a batch
    axis aligned on both sides, K[i, j] = sum_{g,t,s} (a1 . a2)(g1 . g2)."""
    ka = np.einsum("btgk,csgk->bcgts", a1, a2)
    kg = np.einsum("btgd,csgd->bcgts", g1, g2)
    return (ka * kg).sum(axis=(2, 3, 4))


def grouped_cross_gram_per_token(a1, g1, a2, g2) -> np.ndarray:
    """Grouped cross_gram_per_token (dot.py:216-218): side 2's per-group weight
    gradients, then each side-1 token's per-group rank-1 term against them."""
    m2 = np.einsum("csgk,csgd->cgkd", a2, g2)
    return np.einsum("btgk,btgd,cgkd->btc", a1, g1, m2)


# ---------------------------------------------------------------------------
# channel norms
# ---------------------------------------------------------------------------


def group_norm_x_hat(x, groups: int, eps: float) -> np.ndarray:
    """GroupNorm x_hat (norm.py:44-62): x (N, C, *spatial) split into `groups`
    blocks of consecutive channels, each normalised over its channels and
    positions with the biased variance; groups == C is InstanceNorm."""
    x = np.asarray(x)
    n, c = x.shape[:2]
    blk = x.reshape(n, groups, -1)
    mean = blk.mean(axis=2, keepdims=True)
    var = ((blk - mean) ** 2).mean(axis=2, keepdims=True)
    return ((blk - mean) / np.sqrt(var + eps)).reshape(x.shape)


def channel_norm_preprocess(x, g, groups: int, eps: float, has_bias: bool = False):
    """A channel norm's factors (norm.py:120-141, preprocess.py:386-401): x_hat
    and g laid out (N, S, C) with the positions as tokens; with a bias,
    [x_hat, 1] and [g, g] so that a * g summed over S is [dgamma, dbeta]."""
    x_hat = group_norm_x_hat(x, groups, eps)
    n, c = x_hat.shape[:2]
    a = x_hat.reshape(n, c, -1).transpose(0, 2, 1)
    gg = np.asarray(g).reshape(n, c, -1).transpose(0, 2, 1)
    if has_bias:
        return np.concatenate([a, np.ones_like(a)], axis=-1), np.concatenate([gg, gg], axis=-1)
    return a, gg


# ---------------------------------------------------------------------------
# routed-row location
# ---------------------------------------------------------------------------


def match_rows(x, src):
    """RoutedTokenTracker._match (routing.py:300-333) by exact grouping: the
    k-th occurrence of a row value in x takes the k-th token (ascending) of src
    whose row has the same bits, then the pair must compare equal as floats
    (torch.equal: a NaN fails).  Returns the int64 tokens, or None."""
    x, src = np.asarray(x), np.asarray(src)
    groups: dict[bytes, list[int]] = {}
    for t in range(src.shape[0]):
        groups.setdefault(src[t].tobytes(), []).append(t)
    used: dict[bytes, int] = {}
    out = np.empty(x.shape[0], dtype=np.int64)
    for r in range(x.shape[0]):
        key = x[r].tobytes()
        k = used.get(key, 0)
        cand = groups.get(key, [])
        if k >= len(cand):
            return None
        used[key] = k + 1
        t = cand[k]
        if not np.array_equal(x[r].astype(np.float64), src[t].astype(np.float64)):
            return None
        out[r] = t
    return out

