"""Gradient inner products on the MI355X kernels.

Mirrors ``dattri_llm/gradient/ops/dot.py``:

* :func:`cross_gram` (dot.py:36-118) -- per-layer ``K[i, j] = <dW1_i, dW2_j>``;
  the factorized route is the fused ghost kernel (``da_ghost_gram``), the
  materialized route is the dW kernel on both sides plus the score GEMM, the
  norm route is the fused norm-gradient kernel plus the score GEMM.
* :func:`cross_dot` / :func:`cross_dot_factors` (dot.py:121-146, :478-517) --
  raw captures are preprocessed *inside* the kernels (implicit bias column,
  x_hat in registers) instead of by concatenation copies.
* :func:`layerwise_cross_dot` (dot.py:532-604) -- all dense layer pairs of a
  block go through ONE multi-layer score-GEMM launch and factorized pairs
  accumulate into the same fp32 total.
* the routing rules (dot.py:686-753), looked up through this module's globals
  so the reference's ``pin_route`` monkeypatching still steers ``cross_gram``.

Every product accumulates in fp32; results are returned in the resolved
compute dtype (the reference's contract).
"""

from __future__ import annotations

import math
import weakref
from typing import TYPE_CHECKING

import torch

from dattri_llm_amd import kernels
from dattri_llm_amd.gradient.ops import conv, cost, dtypes
from dattri_llm_amd.gradient.ops import embedding as emb
from dattri_llm_amd.gradient.ops.materialize import (
    conv_dense,
    linear_dense,
    materialize,
    materialize_blocked,
    norm_token_rows,
    norm_grad_from_final,
    norm_grad_from_raw,
)
from dattri_llm_amd.gradient.ops.preprocess import final_linear, to_3d
from dattri_llm_amd.gradient.ops.types import (
    PARAM_GRAD_TYPES,
    is_conv,
    is_conv_transpose,
    is_embedding,
    is_linear,
    is_norm,
    require_supported,
)

if TYPE_CHECKING:
    from collections.abc import Iterable


def _kernel_operands(*tensors):
    aligned = dtypes.align(*tensors)
    out_dtype = aligned[0].dtype
    kd = dtypes.kernel_dtype(out_dtype)
    return tuple(t.to(kd) for t in aligned), out_dtype


def _rows(m: torch.Tensor) -> torch.Tensor:
    """A dense layer as the score kernel takes it: k-blocked views as they are
    (reshaping one would copy it), anything else flattened to (B, d)."""
    return m if kernels.is_blocked(m) else m.reshape(m.shape[0], -1)


def _dense_gram(m1: torch.Tensor, m2: torch.Tensor, out=None, accumulate=False) -> torch.Tensor:
    """fp32 ``m1 @ m2.T`` of two dense (B, d) blocks via the score kernel."""
    (m1, m2), _ = _kernel_operands(_rows(m1), _rows(m2))
    return kernels.score_gemm([(m1, m2)], out=out, accumulate=accumulate)


def _route(b1: int, b2: int, s: int, k: int, d: int) -> str:
    # looked up through module globals (pin_route contract, run_ours.py:61-86)
    return "materialized" if maybe_use_materialized_gram(b1, b2, s, k, d) else "factorized"


def _explicit_bias(x: torch.Tensor) -> torch.Tensor:
    """``x`` with its ones column appended (the preprocessed form of a bias)."""
    return torch.cat([x, torch.ones_like(x[..., :1])], dim=-1)


def _agree_bias(x1, bias1, x2, bias2):
    """One layer's activation factors where one side still applies its bias
    column implicitly (a raw capture) and the other holds it explicitly
    (already preprocessed, utils.py:180-236): the implicit one is appended, so
    both sides read the same K + 1 columns."""
    if bias1 == bias2:
        return x1, bias1, x2, bias2
    if bias1:
        return _explicit_bias(x1), False, x2, False
    return x1, False, _explicit_bias(x2), False


def _linear_gram32(a1, g1, bias1, a2, g2, bias2, mode, out=None, accumulate=False):
    """fp32 (B1, B2) cross-gram of linear factors with implicit bias columns."""
    a1, bias1, a2, bias2 = _agree_bias(a1, bias1, a2, bias2)
    (a1, g1, a2, g2), _ = _kernel_operands(to_3d(a1), to_3d(g1), to_3d(a2), to_3d(g2))
    if a1.shape[-1] != a2.shape[-1] or g1.shape[-1] != g2.shape[-1]:
        raise ValueError("the two sides disagree on the layer widths")
    b1, s, k = a1.shape
    b2 = a2.shape[0]
    d = g1.shape[-1]
    if mode == "auto":
        mode = _route(b1, b2, s, k + int(bias1), d)
    if mode == "materialized":
        m1 = kernels.materialize_linear(a1, g1, bias=bias1, blocked=True)
        m2 = kernels.materialize_linear(a2, g2, bias=bias2, blocked=True)
        return kernels.score_gemm([(m1, m2)], out=out, accumulate=accumulate)
    if mode != "factorized":
        raise ValueError("mode must be 'factorized', 'materialized', or 'auto'")
    if out is None:
        out = torch.zeros(b1, b2, dtype=torch.float32, device=a1.device)
    elif not accumulate:
        out.zero_()
    _ghost_pairs([(a1, g1, a2, g2, bias1)], out)
    return out


# ---------------------------------------------------------------------------
# The factorized route over packed rows when most rows carry no gradient
# ---------------------------------------------------------------------------

# Take the packed route when side 2's live rows are under this share of its
# B2*T2 rows (so the live pairs are under it of the dense ghost's (B1*T1) x
# (B2*T2)): the packed kernel bins its products by sample pair and runs at
# ~3/4 of the dense engine's rate, so it pays from about half the work down.
_PACKED_SHARE = 0.5


def _live_rows(x3: torch.Tensor, y3: torch.Tensor):
    """Per-sample ``(seg, rows)`` of the rows whose gradient row is non-zero: the
    rows a routed expert's zero-filled (B, T, d) capture actually holds
    (routing.py:17-23, :71-86)."""
    b, t = y3.shape[:2]
    return kernels.compact_rows(kernels.nonzero_rows(y3.reshape(b * t, y3.shape[-1])), b, t)


# Live-row probes per gradient factor, keyed by the identity of the tensor a
# factor is a view of (an entry leaves with that tensor) and checked against
# the view's address, shape, strides and version: a query block scored
# against every train block is read and counted once.
_PROBES: dict[int, tuple] = {}


def _probe_key(y3: torch.Tensor):
    root = y3._base if y3._base is not None else y3
    return root, (y3.data_ptr(), tuple(y3.shape), y3.stride(), y3._version)


def _probe_get(root: torch.Tensor, sig):
    hit = _PROBES.get(id(root))
    return hit[2] if hit is not None and hit[0]() is root and hit[1] == sig else None


def _probe_put(root: torch.Tensor, sig, entry) -> None:
    key = id(root)

    def drop(ref, key=key):
        if _PROBES.get(key, (None,))[0] is ref:
            del _PROBES[key]

    _PROBES[key] = (weakref.ref(root, drop), sig, entry)


# Uniform per-sample offsets (sample b's rows b*T .. b*T+T-1) of fully live
# sides, per (B, T, device); made outside graph capture only, so a cached
# tensor always holds its values.
_UNIFORM_SEGS: dict[tuple, torch.Tensor] = {}


def _uniform_segments(b: int, t: int, device) -> torch.Tensor:
    key = (b, t, str(device))
    seg = _UNIFORM_SEGS.get(key)
    if seg is None:
        seg = torch.arange(0, b * t + 1, t, dtype=torch.int32, device=device)
        if not torch.cuda.is_current_stream_capturing():
            _UNIFORM_SEGS[key] = seg
    return seg


def _ghost_pairs(pairs, out: torch.Tensor) -> None:
    """Add the factorized cross-gram of every ``(a1, g1, a2, g2, bias)`` kernel
    operand pair (3-D, one dtype per pair) into ``out`` (fp32, (B1, B2)).

    Side 2 (the query side, scored against every train block) decides the
    route: its gradient-carrying rows are found on the device and counted on
    the host once per tensor.  When under ``_PACKED_SHARE`` of its rows live,
    the pair's products are under that share of the dense ghost's for any
    side 1, so side 1 is packed on the device too (no host read) and the
    packed grouped kernel runs every such pair of a dtype in ONE launch;
    otherwise the dense ghost kernel runs and side 1 is never probed, so a
    dense train block costs no extra read and no host sync.  Both kernels give
    the same sums -- zero rows contribute nothing -- so the choice changes
    speed only.  The packed kernel's grid is sized for all B*T rows; tiles
    past the live rows return at once.

    Pairs left to the dense kernel whose 256 x 128-token tiles would hold
    under ``cost.PACKED_RELATIVE_RATE`` of live row pairs -- short sequences,
    single-token rows -- take the packed kernel too, with every row live
    (uniform segments, no probe): it packs several samples into each tile
    (measured at K = D = 4096: 1069 against 193 TFLOP/s at T = 64, 972
    against 646 at T = 128)."""
    probed, plain = [], []
    for pair in pairs:
        a1, _g1, a2, _g2, _bias = pair
        (plain if a1.shape[1] <= 1 and a2.shape[1] <= 1 else probed).append(pair)
    side2, misses = [], []
    for _a1, _g1, a2, g2, _b in probed:
        root, sig = _probe_key(g2)
        hit = _probe_get(root, sig)
        if hit is not None:
            side2.append(hit)
        else:
            seg, rows = _live_rows(a2, g2)
            side2.append([seg, rows, None])
            misses.append((root, sig, side2[-1]))
    if misses:  # one host read for every newly probed side
        counts = torch.stack([entry[0][-1] for _r, _s, entry in misses]).tolist()
        for (root, sig, entry), n in zip(misses, counts):
            entry[2] = int(n)
            _probe_put(root, sig, entry)
    packed: dict[torch.dtype, tuple[list, list, list]] = {}
    for pair, (seg2, rows2, n2) in zip(probed, side2):
        a1, g1, a2, g2, bias = pair
        rows_1, rows_2 = a1.shape[0] * a1.shape[1], a2.shape[0] * a2.shape[1]
        if n2 >= _PACKED_SHARE * rows_2:
            plain.append(pair)
            continue
        seg1, rows1 = _live_rows(a1, g1)
        g_1, g_2, flags = packed.setdefault(a1.dtype, ([], [], []))
        g_1.append((a1.reshape(rows_1, -1), g1.reshape(rows_1, -1), seg1, rows1))
        g_2.append((a2.reshape(rows_2, -1), g2.reshape(rows_2, -1), seg2, rows2))
        flags.append(bias)
    for pair in plain:
        a1, g1, a2, g2, bias = pair
        (b1, t1), (b2, t2) = a1.shape[:2], a2.shape[:2]
        if t1 >= 1 and t2 >= 1 and cost.ghost_tile_share(t1, t2) < cost.PACKED_RELATIVE_RATE:
            g_1, g_2, flags = packed.setdefault(a1.dtype, ([], [], []))
            g_1.append((a1.reshape(b1 * t1, -1), g1.reshape(b1 * t1, -1), _uniform_segments(b1, t1, a1.device), None))
            g_2.append((a2.reshape(b2 * t2, -1), g2.reshape(b2 * t2, -1), _uniform_segments(b2, t2, a2.device), None))
            flags.append(bias)
            continue
        kernels.ghost_gram(a1, g1, a2, g2, bias=bias, out=out, accumulate=True)
    for g_1, g_2, flags in packed.values():
        kernels.ghost_gram_grouped(g_1, g_2, bias=flags, out=out, accumulate=True)


# ---------------------------------------------------------------------------
# Convolutions and grouped (4-D) factors: the linear kernels, per group
# ---------------------------------------------------------------------------


def _is_conv_family(layer_type: str, a) -> bool:
    """Conv / ConvTranspose layers, and any factors with a group axis."""
    return is_conv(layer_type) or is_conv_transpose(layer_type) or to_3d(a).ndim == 4


def _conv_pair(c1, c2):
    """The two sides of one convolution, checked and with one bias form (a
    raw side's implicit ones column made explicit against a preprocessed
    side's)."""
    if c1.bias != c2.bias:
        if c1.bias:
            c1 = conv.ConvFactors(_explicit_bias(c1.a), c1.g, False, c1.transpose)
        else:
            c2 = conv.ConvFactors(_explicit_bias(c2.a), c2.g, False, c2.transpose)
    if c1.groups != c2.groups or c1.a.dim() != c2.a.dim():
        raise ValueError(f"the two sides disagree on the group count ({c1.groups} vs {c2.groups})")
    if c1.a.shape[-1] != c2.a.shape[-1] or c1.g.shape[-1] != c2.g.shape[-1]:
        raise ValueError("the two sides disagree on the layer widths")
    return c1, c2


def _conv_operands(c):
    (a, g), _ = _kernel_operands(c.a, c.g)
    return conv.ConvFactors(a, g, c.bias, c.transpose)


def _group_rows(c, e: int):
    """Group e of a side as the grouped kernel's (rows, width) operands: all
    B*L rows, sample b's rows b*L .. b*L+L-1."""
    a, g = c.group(e)
    b, length = a.shape[:2]
    seg = torch.arange(0, b * length + 1, max(length, 1), dtype=torch.int32, device=a.device)[: b + 1]
    return a.reshape(b * length, a.shape[-1]), g.reshape(b * length, g.shape[-1]), seg, None


def _conv_gram32(c1, c2, mode, out=None, accumulate=False):
    """fp32 (B1, B2) cross-gram of two convolution sides (dot.py:88-118): the
    ungrouped case is the linear layer's; groups pair with their own group
    only -- one grouped ghost launch over all groups, or each group's dW."""
    c1, c2 = _conv_pair(c1, c2)
    if c1.groups == 1 and c1.a.dim() == 3:
        return _linear_gram32(c1.a, c1.g, c1.bias, c2.a, c2.g, c2.bias, mode, out=out, accumulate=accumulate)
    c1, c2 = _conv_operands(c1), _conv_operands(c2)
    b1, s, _g, k = c1.a.shape
    b2, d = c2.a.shape[0], c1.g.shape[-1]
    if mode == "auto":  # per-group widths: the group count scales both costs alike
        mode = _route(b1, b2, s, k + int(c1.bias), d)
    if mode == "materialized":
        return kernels.score_gemm([(conv_dense(c1), conv_dense(c2))], out=out, accumulate=accumulate)
    if mode != "factorized":
        raise ValueError("mode must be 'factorized', 'materialized', or 'auto'")
    if out is None:
        out = torch.zeros(b1, b2, dtype=torch.float32, device=c1.a.device)
    elif not accumulate:
        out.zero_()
    groups1 = [_group_rows(c1, e) for e in range(c1.groups)]
    groups2 = [_group_rows(c2, e) for e in range(c2.groups)]
    return kernels.ghost_gram_grouped(groups1, groups2, bias=c1.bias, out=out, accumulate=True)


def _conv_diag32(c1, c2) -> torch.Tensor:
    """fp32 (B,) per-sample dots (squared norms for one side with itself)."""
    same = c1 is c2
    c1, c2 = _conv_pair(c1, c2)
    if c1.a.shape[0] != c2.a.shape[0]:
        raise ValueError("per-sample dots need two blocks of one batch size")
    c1 = _conv_operands(c1)
    c2 = c1 if same else _conv_operands(c2)
    out = torch.zeros(c1.a.shape[0], dtype=torch.float32, device=c1.a.device)
    for e in range(c1.groups):
        (x1, y1), (x2, y2) = c1.group(e), c2.group(e)
        if same:
            x2, y2 = x1, y1
        kernels.ghost_gram_diag(x1, y1, x2, y2, bias=c1.bias, out=out, accumulate=True)
    return out


def _conv_norm32(c, mode) -> torch.Tensor:
    """fp32 (B,) squared norms, routed by the norm rule on per-group widths
    (dot.py:386-405)."""
    s, k, d = c.a.shape[1], c.a.shape[-1] + int(c.bias), c.g.shape[-1]
    if mode == "auto":
        mode = "materialized" if maybe_use_materialized_norm(s, k, d) else "factorized"
    if mode == "materialized":
        return _sq_row_norms(conv_dense(_conv_operands(c)))
    if mode != "factorized":
        raise ValueError("mode must be 'factorized', 'materialized', or 'auto'")
    return _conv_diag32(c, c)


def _conv_per_token32(c1, c2) -> torch.Tensor:
    """fp32 (B1, T1, B2): side 1's location t against side 2's whole gradient,
    summed over the groups (dot.py:216-222)."""
    c1, c2 = _conv_pair(c1, c2)
    c1, c2 = _conv_operands(c1), _conv_operands(c2)
    out = None
    for e in range(c1.groups):
        (x1, y1), (x2, y2) = c1.group(e), c2.group(e)
        out = kernels.ghost_gram_per_token(x1, y1, x2, y2, bias=c1.bias, out=out, accumulate=out is not None)
    return out


def _conv_dense_per_token32(c1, m2: torch.Tensor) -> torch.Tensor:
    """fp32 (B1, T1, B2) against dense per-sample gradients in materialize's
    layout (dot.py:248-263): per group, (Wg, Wa) blocks -- (Wa, Wg) for a
    transposed convolution, whose roles the kernel then swaps."""
    c1 = _conv_operands(c1)
    (m2,), _ = _kernel_operands(m2.reshape(m2.shape[0], -1))
    groups = c1.groups
    per = m2.reshape(m2.shape[0], groups, -1)
    out = None
    for e in range(groups):
        x1, y1 = c1.group(e)
        if c1.transpose:  # block (Wa, Wg): sum_c a[c] (M g)[c]
            x1, y1 = y1, x1
        out = kernels.dense_per_token(x1, y1, per[:, e], bias=c1.bias, out=out, accumulate=out is not None)
    return out


def cross_gram(a1, g1, a2, g2, layer_type: str, mode: str = "auto") -> torch.Tensor:
    """Cross-gram ``K[i, j] = <dW1_i, dW2_j>`` on already-preprocessed factors
    (dot.py:36-118)."""
    out_dtype = dtypes.resolve(a1, g1, a2, g2)
    if is_embedding(layer_type):
        # K[i,j] = sum over equal ids of g1_it . g2_js (dot.py:58-74)
        emb.check_ids(a1, a2)
        return emb.gram32(emb.side(a1, g1, layer_type, None), emb.side(a2, g2, layer_type, None)).to(out_dtype)
    if is_norm(layer_type):  # final factors: the token sum of a * g, whatever the norm
        return _dense_gram(norm_grad_from_final(a1, g1, fp32=True), norm_grad_from_final(a2, g2, fp32=True)).to(
            out_dtype)
    if _is_conv_family(layer_type, a1):
        c1, c2 = conv.final(a1, g1, layer_type, None, False), conv.final(a2, g2, layer_type, None, False)
        return _conv_gram32(c1, c2, mode).to(out_dtype)
    if not is_linear(layer_type):
        require_supported(layer_type, "cross_gram")
    return _linear_gram32(a1, g1, False, a2, g2, False, mode).to(out_dtype)


def _side(a, g, layer_type, module_kwargs, include_bias):
    """('norm', (B, d) fp32 dense) | ('linear', (a, g, bias)) | ('embedding', (ids, g))
    | ('conv', ConvFactors) for one raw side.  A norm layer's per-sample
    gradient stays in fp32 on its way into the inner product."""
    if is_embedding(layer_type):
        return "embedding", emb.side(a, g, layer_type, module_kwargs)
    if is_conv(layer_type) or is_conv_transpose(layer_type) or (module_kwargs is None and a.ndim == 4):
        return "conv", conv.final(a, g, layer_type, module_kwargs, include_bias)
    if is_norm(layer_type):
        if module_kwargs is not None:
            return "norm", norm_grad_from_raw(a, g, layer_type, module_kwargs, include_bias, fp32=True)
        return "norm", norm_grad_from_final(a, g, fp32=True)
    if not is_linear(layer_type):
        require_supported(layer_type, "cross_dot")
    return "linear", final_linear(a, g, layer_type, module_kwargs, include_bias)


def _cross_factors32(a1, g1, a2, g2, layer_type, mk1, mk2, include_bias, mode, out=None, accumulate=False):
    if is_embedding(layer_type):
        emb.check_ids(a1, a2)
    kind, s1 = _side(a1, g1, layer_type, mk1, include_bias)
    _, s2 = _side(a2, g2, layer_type, mk2, include_bias)
    if kind == "embedding":
        return emb.gram32(s1, s2, out=out, accumulate=accumulate)
    if kind == "conv":
        return _conv_gram32(s1, s2, mode, out=out, accumulate=accumulate)
    if kind == "norm":
        return _dense_gram(s1, s2, out=out, accumulate=accumulate)
    return _linear_gram32(*s1, *s2, mode, out=out, accumulate=accumulate)


def cross_dot_factors(a1, g1, a2, g2, layer_type: str, module_kwargs1: dict | None = None,
                      module_kwargs2: dict | None = None, include_bias: bool = True,
                      mode: str = "auto") -> torch.Tensor:
    """(B1, B2) cross-gram of two raw factor pairs (dot.py:121-146)."""
    out_dtype = dtypes.resolve(a1, g1, a2, g2)
    return _cross_factors32(a1, g1, a2, g2, layer_type, module_kwargs1, module_kwargs2,
                            include_bias, mode).to(out_dtype)


def pairwise_dot_factors(a, g, layer_type: str, module_kwargs: dict | None = None,
                         include_bias: bool = True, mode: str = "auto") -> torch.Tensor:
    """(B, B) pairwise Gram of one block (dot.py:149-163)."""
    return cross_dot_factors(a, g, a, g, layer_type, module_kwargs, module_kwargs, include_bias, mode)


def dot_factors(a1, g1, a2, g2, layer_type: str, module_kwargs1: dict | None = None,
                module_kwargs2: dict | None = None, include_bias: bool = True) -> torch.Tensor:
    """(B,) per-sample dots ``<dW1_i, dW2_i>`` (dot.py:307-357): one launch of
    the ghost kernel on the diagonal pairs (linear layers) or of the row-dot
    kernel (norm layers)."""
    out_dtype = dtypes.resolve(a1, g1, a2, g2)
    if a1.shape[0] != g2.shape[0]:
        raise ValueError("dot_factors needs two blocks of one batch size")
    if is_embedding(layer_type):
        emb.check_ids(a1, a2)
    kind, s1 = _side(a1, g1, layer_type, module_kwargs1, include_bias)
    _, s2 = _side(a2, g2, layer_type, module_kwargs2, include_bias)
    if kind == "embedding":
        return emb.diag32(s1, s2).to(out_dtype)
    if kind == "conv":
        return _conv_diag32(s1, s2).to(out_dtype)
    if kind == "norm":
        (m1, m2), _ = _kernel_operands(_rows(s1), _rows(s2))
        return kernels.row_dots([(m1, m2)]).to(out_dtype)
    (x1, y1, bias1), (x2, y2, bias2) = s1, s2
    x1, bias1, x2, bias2 = _agree_bias(x1, bias1, x2, bias2)
    (x1, y1, x2, y2), _ = _kernel_operands(to_3d(x1), to_3d(y1), to_3d(x2), to_3d(y2))
    return kernels.ghost_gram_diag(x1, y1, x2, y2, bias=bias1).to(out_dtype)


def _sq_row_norms(m: torch.Tensor) -> torch.Tensor:
    """fp32 squared row norms of a dense (B, d) block (k-blocked views are
    read in place), one launch."""
    (m,), _ = _kernel_operands(_rows(m))
    return kernels.row_dots([(m, None)])


def grad_norm_sq_factors(a, g, layer_type: str, module_kwargs: dict | None = None,
                         include_bias: bool = True, mode: str = "auto") -> torch.Tensor:
    """(B,) squared per-sample gradient norms (dot.py:365-411), one launch:
    the ghost kernel on the diagonal pairs of the block with itself
    (factorized), or the row-dot kernel on the per-sample gradients
    (materialized, and norm layers)."""
    out_dtype = dtypes.resolve(a, g)
    if is_embedding(layer_type):
        emb.check_ids(a)
    kind, side = _side(a, g, layer_type, module_kwargs, include_bias)
    if kind == "embedding":  # the diagonal of the pairwise gram (dot.py:383-384)
        return emb.diag32(side, side).to(out_dtype)
    if kind == "conv":
        return _conv_norm32(side, mode).to(out_dtype)
    if kind == "norm":
        return _sq_row_norms(side).to(out_dtype)
    x, y, bias = side
    (x3, y3), _ = _kernel_operands(to_3d(x), to_3d(y))
    s, k, d = x3.shape[1], x3.shape[-1] + int(bias), y3.shape[-1]
    if mode == "auto":
        mode = "materialized" if maybe_use_materialized_norm(s, k, d) else "factorized"
    if mode == "materialized":
        return _sq_row_norms(linear_dense(x3, y3, bias)).to(out_dtype)
    if mode != "factorized":
        raise ValueError("mode must be 'factorized', 'materialized', or 'auto'")
    return kernels.ghost_gram_diag(x3, y3, x3, y3, bias=bias).to(out_dtype)


def grad_norm_sq(f, layer_type: str, include_bias: bool = True, mode: str = "auto") -> torch.Tensor:
    """(B,) squared norms of one layer, whatever its form (dot.py:414-437)."""
    if isinstance(f, torch.Tensor):
        return _sq_row_norms(f).to(dtypes.resolve(f))
    bf = f.as_batch_first()
    return grad_norm_sq_factors(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs,
                                include_bias, mode)


def block_grad_norm_sq(rep, layers, dense_cache=None) -> torch.Tensor:
    """fp32 (B,) per-sample squared gradient norms summed over ``layers`` of a
    block -- the whole-model norm of GradCos (tracin.py:129-148).  Every dense
    layer of full batch (held dense, or already in ``dense_cache``) is summed
    in ONE row-dot launch; factorized layers take :func:`grad_norm_sq`; a
    broadcast batch-1 layer counts for every sample."""
    b = rep.batch_size
    total = torch.zeros(b, dtype=torch.float32, device=rep.device)
    dense = []
    for name in layers:
        value = rep.data[name]
        if dense_cache is not None and name in dense_cache:
            value = dense_cache.get(name)
        if isinstance(value, torch.Tensor) and value.shape[0] == b and b > 1:
            dense.append(_rows(value))
            continue
        sq = grad_norm_sq(value, rep.layer_types[name]).float()
        total += sq.expand(b) if sq.shape[0] == 1 else sq
    by_dtype: dict[torch.dtype, list] = {}
    for m in dense:
        (m,), _ = _kernel_operands(m)
        by_dtype.setdefault(m.dtype, []).append((m, None))
    for group in by_dtype.values():
        kernels.row_dots(group, out=total, accumulate=True)
    return total


def pairwise_dot(f, layer_type: str, include_bias: bool = True, mode: str = "auto") -> torch.Tensor:
    bf = f.as_batch_first()
    return pairwise_dot_factors(bf.activation, bf.pre_activation_grad, layer_type, bf.module_kwargs,
                                include_bias, mode)


def dot(f1, f2, layer_type: str, include_bias: bool = True) -> torch.Tensor:
    b1, b2 = f1.as_batch_first(), f2.as_batch_first()
    return dot_factors(b1.activation, b1.pre_activation_grad, b2.activation, b2.pre_activation_grad,
                       layer_type, b1.module_kwargs, b2.module_kwargs, include_bias)


def _cross_dot32(f1, f2, layer_type, include_bias=True, mode="auto", out=None, accumulate=False):
    if isinstance(f1, torch.Tensor) or isinstance(f2, torch.Tensor):
        m1 = materialize(f1, layer_type, include_bias)
        m2 = materialize(f2, layer_type, include_bias)
        return _dense_gram(m1, m2, out=out, accumulate=accumulate)
    b1, b2 = f1.as_batch_first(), f2.as_batch_first()
    return _cross_factors32(b1.activation, b1.pre_activation_grad, b2.activation, b2.pre_activation_grad,
                            layer_type, b1.module_kwargs, b2.module_kwargs, include_bias, mode,
                            out=out, accumulate=accumulate)


def _payload_dtype(f) -> torch.dtype:
    if isinstance(f, torch.Tensor):
        return dtypes.resolve(f)
    return dtypes.resolve(f.activation, f.pre_activation_grad)


def cross_dot(f1, f2, layer_type: str, include_bias: bool = True, mode: str = "auto") -> torch.Tensor:
    """(B1, B2) cross-gram of one layer in whatever form each side holds
    (dot.py:478-517)."""
    out_dtype = torch.promote_types(_payload_dtype(f1), _payload_dtype(f2)) \
        if dtypes.get_compute_dtype() == "auto" else dtypes.resolve(torch.empty(0))
    return _cross_dot32(f1, f2, layer_type, include_bias, mode).to(out_dtype)


def _expand_broadcast(m: torch.Tensor, b1: int, b2: int) -> torch.Tensor:
    return m.expand(b1 if m.shape[0] == 1 else m.shape[0], b2 if m.shape[1] == 1 else m.shape[1])


def _batch(f) -> int:
    if isinstance(f, torch.Tensor):
        return f.shape[0]
    return f.activation.shape[0 if f.batch_first else 1]


def layerwise_cross_dot(train, test, *, layers: Iterable[str] | None = None, mode: str = "auto",
                        dense_cache=None, reduce: str = "sum"):
    """Layer-by-layer cross-gram of two gradient blocks, summed over layers
    (dot.py:532-604)."""
    if reduce not in {"sum", "none"}:
        raise ValueError("reduce must be 'sum' or 'none'")
    names = list(train.data) if layers is None else list(layers)
    pairs = []  # (name, layer_type, train payload, test payload)
    for name in names:
        if name not in train.data or name not in test.data:
            continue
        layer_type = train.layer_types[name]
        if layer_type == PARAM_GRAD_TYPES:
            continue
        tr, te = train.data[name], test.data[name]
        if isinstance(te, torch.Tensor) and not isinstance(tr, torch.Tensor):
            tr = (dense_cache.get_or_compute(name, lambda tr=tr, lt=layer_type: materialize_blocked(tr, lt))
                  if dense_cache is not None else materialize_blocked(tr, layer_type))
        pairs.append((name, layer_type, tr, te))
    if reduce == "none":
        return {n: cross_dot(tr, te, lt, mode=mode) for n, lt, tr, te in pairs}
    if not pairs:
        raise ValueError("No shared layers between the two gradient blocks.")
    b_tr, b_te = train.batch_size, test.batch_size
    out_dtype = None
    for _n, _lt, tr, te in pairs:
        d = torch.promote_types(_payload_dtype(tr), _payload_dtype(te))
        out_dtype = d if out_dtype is None else torch.promote_types(out_dtype, d)
    if dtypes.get_compute_dtype() != "auto":
        out_dtype = dtypes.resolve(torch.empty(0))
    device = next(p.device if isinstance(p, torch.Tensor) else p.activation.device
                  for _n, _lt, tr, _te in pairs for p in (tr,))
    total = torch.zeros(b_tr, b_te, dtype=torch.float32, device=device)
    # Dense x dense pairs of full batch: one multi-layer score GEMM per dtype.
    dense_groups: dict[torch.dtype, list] = {}
    rest = []
    for name, lt, tr, te in pairs:
        full = _batch(tr) == b_tr and _batch(te) == b_te
        if full and isinstance(tr, torch.Tensor) and isinstance(te, torch.Tensor):
            (m1, m2), _ = _kernel_operands(_rows(tr), _rows(te))
            dense_groups.setdefault(m1.dtype, []).append((m1, m2))
        else:
            rest.append((name, lt, tr, te, full))
    for group in dense_groups.values():
        kernels.score_gemm(group, out=total, accumulate=True)
    ghost = []  # factorized-route linear pairs: probed together, packed ones in one launch
    for _name, lt, tr, te, full in rest:
        if not full:  # a broadcast (batch-1) layer's shared row counts for every sample
            total += _expand_broadcast(_cross_dot32(tr, te, lt, mode=mode), b_tr, b_te)
            continue
        pair = _factorized_linear_pair(tr, te, lt, mode)
        if pair is not None:
            ghost.append(pair)
        else:
            _cross_dot32(tr, te, lt, mode=mode, out=total, accumulate=True)
    if ghost:
        _ghost_pairs(ghost, total)
    return total.to(out_dtype)


def _factorized_linear_pair(f1, f2, layer_type: str, mode: str, include_bias: bool = True):
    """Kernel operands ``(a1, g1, a2, g2, bias)`` of a factorized linear layer
    pair the route sends to the ghost product, else None (dense sides, other
    layer families, the materialized route, grouped factors)."""
    if isinstance(f1, torch.Tensor) or isinstance(f2, torch.Tensor) or not is_linear(layer_type):
        return None
    b1, b2 = f1.as_batch_first(), f2.as_batch_first()
    x1, y1, bias1 = final_linear(b1.activation, b1.pre_activation_grad, layer_type, b1.module_kwargs, include_bias)
    x2, y2, bias2 = final_linear(b2.activation, b2.pre_activation_grad, layer_type, b2.module_kwargs, include_bias)
    if any(to_3d(t).ndim == 4 for t in (x1, y1, x2, y2)):
        return None
    x1, bias1, x2, bias2 = _agree_bias(x1, bias1, x2, bias2)
    (x1, y1, x2, y2), _ = _kernel_operands(to_3d(x1), to_3d(y1), to_3d(x2), to_3d(y2))
    if x1.shape[-1] != x2.shape[-1] or y1.shape[-1] != y2.shape[-1]:
        raise ValueError("the two sides disagree on the layer widths")
    route = mode if mode != "auto" else _route(x1.shape[0], x2.shape[0], x1.shape[1], x1.shape[-1] + int(bias1),
                                               y1.shape[-1])
    if route not in ("factorized", "materialized"):
        raise ValueError("mode must be 'factorized', 'materialized', or 'auto'")
    return (x1, y1, x2, y2, bias1) if route == "factorized" else None


# ---------------------------------------------------------------------------
# Per-token decomposition (dot.py:166-299, :607-669)
# ---------------------------------------------------------------------------


def _norm_per_token32(rows1: torch.Tensor, m2: torch.Tensor) -> torch.Tensor:
    """fp32 (B1, T1, B2): every token row of side 1 against side 2's (B2, d')
    norm gradients, through the score kernel."""
    b1, t1, d = rows1.shape
    return _dense_gram(rows1.reshape(b1 * t1, d), m2.reshape(m2.shape[0], -1)).reshape(b1, t1, m2.shape[0])


def _linear_operands(*tensors):
    (ts), _ = _kernel_operands(*(to_3d(t) for t in tensors))
    if any(t.ndim == 4 for t in ts):
        raise NotImplementedError("grouped (4-D) factors are conv-only and outside this path")
    return ts


def cross_gram_per_token(a1, g1, a2, g2, layer_type: str) -> torch.Tensor:
    """Per-token cross-gram ``K[i, t, j]`` on preprocessed factors
    (dot.py:171-222): side 1's token t against side 2's whole per-sample
    gradient; summing over t gives :func:`cross_gram`.  ``(B1, T1, B2)``."""
    out_dtype = dtypes.resolve(a1, g1, a2, g2)
    if is_embedding(layer_type):
        emb.check_ids(a1, a2)
        return emb.per_token32(emb.side(a1, g1, layer_type, None), emb.side(a2, g2, layer_type, None)).to(out_dtype)
    if is_norm(layer_type):  # final factors: the token sum of a * g, whatever the norm
        x1, y1, x2, y2 = dtypes.align(to_3d(a1), to_3d(g1), to_3d(a2), to_3d(g2))
        return _norm_per_token32(x1 * y1, norm_grad_from_final(x2, y2, fp32=True)).to(out_dtype)
    if _is_conv_family(layer_type, a1):
        c1, c2 = conv.final(a1, g1, layer_type, None, False), conv.final(a2, g2, layer_type, None, False)
        return _conv_per_token32(c1, c2).to(out_dtype)
    if not is_linear(layer_type):
        require_supported(layer_type, "cross_gram_per_token")
    a1, g1, a2, g2 = _linear_operands(a1, g1, a2, g2)
    return kernels.ghost_gram_per_token(a1, g1, a2, g2).to(out_dtype)


def cross_gram_per_token_dense(a1, g1, m2, layer_type: str) -> torch.Tensor:
    """:func:`cross_gram_per_token` with side 2 dense (dot.py:225-263): ``m2`` is
    the (B2, D) per-sample gradient block in materialize's layout."""
    out_dtype = dtypes.resolve(a1, g1, m2)
    if is_embedding(layer_type):
        emb.check_ids(a1)
        return emb.dense_per_token32(emb.side(a1, g1, layer_type, None), m2).to(out_dtype)
    m2 = m2.reshape(m2.shape[0], -1)
    if is_norm(layer_type):  # final factors: the token sum of a * g, whatever the norm
        x1, y1 = dtypes.align(to_3d(a1), to_3d(g1))
        return _norm_per_token32(x1 * y1, m2).to(out_dtype)
    if _is_conv_family(layer_type, a1):
        return _conv_dense_per_token32(conv.final(a1, g1, layer_type, None, False), m2).to(out_dtype)
    if not is_linear(layer_type):
        require_supported(layer_type, "cross_gram_per_token_dense")
    a1, g1, m2 = _linear_operands(a1, g1, m2)
    return kernels.dense_per_token(a1, g1, m2.reshape(m2.shape[0], -1)).to(out_dtype)


def cross_dot_per_token(f1, f2, layer_type: str, include_bias: bool = True) -> torch.Tensor:
    """Per-token cross-gram of a factorized side 1 against side 2 in whatever
    form it holds (dot.py:266-299); ``(B1, T1, B2)``.  Raw captures are
    preprocessed inside the kernels (implicit bias column)."""
    b1 = f1.as_batch_first()
    a1, g1, mk1 = b1.activation, b1.pre_activation_grad, b1.module_kwargs
    dense2 = isinstance(f2, torch.Tensor)
    out_dtype = dtypes.resolve(a1, g1, f2) if dense2 else dtypes.resolve(a1, g1, f2.activation, f2.pre_activation_grad)
    if is_norm(layer_type):
        rows1 = norm_token_rows(a1, g1, layer_type, mk1, include_bias)
        m2 = f2.reshape(f2.shape[0], -1) if dense2 else materialize(f2, layer_type, include_bias)
        return _norm_per_token32(rows1, m2).to(out_dtype)
    if is_embedding(layer_type):
        emb.check_ids(a1, None if dense2 else f2.as_batch_first().activation)
        s1 = emb.side(a1, g1, layer_type, mk1)
        if dense2:
            return emb.dense_per_token32(s1, f2).to(out_dtype)
        b2 = f2.as_batch_first()
        s2 = emb.side(b2.activation, b2.pre_activation_grad, layer_type, b2.module_kwargs)
        return emb.per_token32(s1, s2).to(out_dtype)
    if is_conv(layer_type) or is_conv_transpose(layer_type) or (mk1 is None and a1.ndim == 4):
        c1 = conv.final(a1, g1, layer_type, mk1, include_bias)
        if dense2:
            return _conv_dense_per_token32(c1, f2).to(out_dtype)
        b2 = f2.as_batch_first()
        c2 = conv.final(b2.activation, b2.pre_activation_grad, layer_type, b2.module_kwargs, include_bias)
        return _conv_per_token32(c1, c2).to(out_dtype)
    if not is_linear(layer_type):
        require_supported(layer_type, "cross_dot_per_token")
    x1, y1, bias1 = final_linear(a1, g1, layer_type, mk1, include_bias)
    if dense2:
        x1, y1, m2 = _linear_operands(x1, y1, f2.reshape(f2.shape[0], -1))
        return kernels.dense_per_token(x1, y1, m2.reshape(m2.shape[0], -1), bias=bias1).to(out_dtype)
    b2 = f2.as_batch_first()
    x2, y2, bias2 = final_linear(b2.activation, b2.pre_activation_grad, layer_type, b2.module_kwargs, include_bias)
    x1, bias1, x2, bias2 = _agree_bias(x1, bias1, x2, bias2)
    x1, y1, x2, y2 = _linear_operands(x1, y1, x2, y2)
    return kernels.ghost_gram_per_token(x1, y1, x2, y2, bias=bias1).to(out_dtype)


def layerwise_cross_dot_per_token(train, test, *, layers: Iterable[str] | None = None, reduce: str = "sum"):
    """Layer-by-layer per-token cross-gram (dot.py:607-669): the
    ``(B_train, T_train, B_test)`` contribution of every train token position to
    :func:`layerwise_cross_dot`, which it sums back to exactly over ``T``.  The
    train side must hold every scored layer factorized with a token axis; the
    test side may be factorized or dense per layer."""
    if reduce not in {"sum", "none"}:
        raise ValueError("reduce must be 'sum' or 'none'")
    names = list(train.data) if layers is None else list(layers)
    per_layer: dict[str, torch.Tensor] = {}
    for name in names:
        if name not in train.data or name not in test.data:
            continue
        if train.layer_types[name] == PARAM_GRAD_TYPES:
            continue  # a batch-level gradient: no per-sample rows to score
        tr = train.data[name]
        if isinstance(tr, torch.Tensor) or train.indexing[name] != "batch_token":
            raise ValueError(
                f"layer {name!r} has no token axis on the train side "
                f"(stored {train.representation[name]}, indexing {train.indexing[name]!r}); token-level "
                "attribution needs the train gradients captured factorized."
            )
        per_layer[name] = cross_dot_per_token(tr, test.data[name], train.layer_types[name])
    if reduce == "none":
        return per_layer
    if not per_layer:
        raise ValueError("No shared layers between the two gradient blocks.")
    shapes = {tuple(v.shape) for v in per_layer.values()}
    if len(shapes) > 1:
        raise ValueError(
            "Layers disagree on the token axis, so their per-token contributions cannot be summed: "
            f"{sorted(shapes)}.  Use reduce='none'."
        )
    total = None
    for v in per_layer.values():
        total = v.float() if total is None else total + v.float()
    return total.to(next(iter(per_layer.values())).dtype)


# ---------------------------------------------------------------------------
# Routing (dot.py:686-753)
# ---------------------------------------------------------------------------


def effective_dims(f, layer_type: str) -> tuple[int, int, int, int]:
    """``(B, S, K, D)`` read from the raw factor shapes (dot.py:686-725)."""
    bf = f.as_batch_first()
    a, g = bf.activation, bf.pre_activation_grad
    if bf.module_kwargs is None:
        if a.ndim == 4:
            return a.shape[0], a.shape[1], a.shape[-1], g.shape[-1]
        return a.shape[0], math.prod(a.shape[1:-1]), a.shape[-1], g.shape[-1]
    mk = bf.module_kwargs
    groups = mk.get("groups", 1)
    if is_conv(layer_type):
        kprod = math.prod(mk["kernel_size"]) if "kernel_size" in mk else 1
        return a.shape[0], math.prod(g.shape[2:]), a.shape[1] // groups * kprod, g.shape[1] // groups
    if is_conv_transpose(layer_type):
        kprod = math.prod(mk["kernel_size"]) if "kernel_size" in mk else 1
        return a.shape[0], math.prod(a.shape[2:]), a.shape[1] // groups, g.shape[1] // groups * kprod
    return a.shape[0], math.prod(a.shape[1:-1]), a.shape[-1], g.shape[-1]


def route_flops(b1: int, b2: int, s: int, k: int, d: int) -> tuple[int, int]:
    """The flop counts the reference's rule compares (dot.py:728-745):
    ``(B1*B2*S^2*(D+K), (B1+B2)*S*D*K + B1*B2*D*K)`` for (factorized,
    materialized)."""
    return b1 * b2 * s * s * (d + k), (b1 + b2) * s * d * k + b1 * b2 * d * k


def maybe_use_materialized_gram(B1: int, B2: int, S: int, K: int, D: int, kappa: float = 1.0) -> bool:  # noqa: N803
    """``True`` when materialize-then-GEMM is the cheaper cross-gram.

    Under the default ``"flops"`` policy this is the reference's rule
    (dot.py:728-745): materialize iff ``kappa * B1*B2*S^2*(D+K) >=
    (B1+B2)*S*D*K + B1*B2*D*K``.  Under ``set_routing_policy("calibrated")``
    the two routes are compared by their predicted MI355X time instead
    (:mod:`dattri_llm_amd.gradient.ops.cost`).
    """
    if cost.get_routing_policy() == "calibrated":
        return cost.calibrated_model().prefers_materialized(B1, B2, S, S, K, D, kappa)
    cost_f, cost_m = route_flops(B1, B2, S, K, D)
    return kappa * cost_f >= cost_m


def maybe_use_materialized_norm(S: int, K: int, D: int) -> bool:  # noqa: N803
    """Per-sample norms: materialize iff ``S*(D+K) >= D*K`` (dot.py:748-753)."""
    if cost.get_routing_policy() == "calibrated":
        return cost.calibrated_model().prefers_materialized(1, 1, S, S, K, D, 1.0)
    return S * (D + K) >= D * K
