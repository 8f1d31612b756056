"""MoE routed layers: router top-k, expert segments, segment-summed ghost products.

The reference captures fused experts through per-expert proxies
(``dattri_llm/gradient/hooks/override_layers/fused_experts.py:210-237``): the
router is ``softmax(logits.float()) -> topk -> / sum`` (transformers'
MixtralTopKRouter), expert ``e`` receives the rows
``torch.where(one_hot(idx).permute(2,1,0)[e])`` -- top-k slot major, token
ascending -- and each proxy's rows are scattered back into a zero-filled
``(B, T, d)`` tensor (``hooks/routing.py:71-86``), so an expert's ghost
product runs over all ``B*T`` rows although only its routed rows are non-zero.

Here the rows stay compact: :func:`expert_segments` reproduces the reference
enumeration with a stable device counting sort, :func:`segment_by_sample`
groups an expert's rows by sample, and :func:`expert_cross_gram` runs the
ghost kernel over those per-sample segments -- the same sum without the zero
rows (``routing.py:17-23`` explains why zero rows are inert).  Segment-summing
over experts accumulates into one fp32 matrix.
"""

from __future__ import annotations

import torch

from dattri_llm_amd import kernels
from dattri_llm_amd.gradient.ops import dtypes

_KERNEL_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def router_topk(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(weights, indices)`` of the top-k router; indices int64 (N, k)."""
    logits = logits.reshape(-1, logits.shape[-1])
    return kernels.moe_topk(logits, k)


def expert_segments(top_idx: torch.Tensor, n_experts: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Expert segments of a (N, k) top-k index matrix.

    Returns ``(offsets, entries)``: expert ``e`` owns ``entries[offsets[e]:offsets[e+1]]``,
    each entry ``p = slot * N + token`` -- in the reference's order."""
    offsets, perm = kernels.counting_sort(top_idx.to(torch.int64), n_experts, slot_major=True)
    return offsets, perm


def expert_rows(top_idx: torch.Tensor, n_experts: int) -> list[tuple[torch.Tensor, torch.Tensor]]:
    """Per expert ``(top_k_pos, token_idx)`` exactly as ``torch.where(mask[e])``."""
    n = top_idx.shape[0]
    offsets, entries = expert_segments(top_idx, n_experts)
    off = offsets.cpu().tolist()
    entries = entries.to(torch.int64)
    return [(entries[off[e]:off[e + 1]] // n, entries[off[e]:off[e + 1]] % n) for e in range(n_experts)]


def segment_by_sample(token_idx: torch.Tensor, batch: int, tokens: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Group routed rows by sample (flat token ``b*T + t`` -> sample ``b``):
    ``(offsets (B+1) int32, rows int32)``, sample ``b`` owning
    ``rows[offsets[b]:offsets[b+1]]`` (stable: routed order kept)."""
    return kernels.counting_sort(token_idx, batch, key_div=tokens)


def expert_cross_gram(a1, g1, tok1, a2, g2, tok2, *, batch1: int, tokens1: int, batch2: int, tokens2: int,
                      bias: bool = False, out: torch.Tensor | None = None, accumulate: bool = False):
    """One expert's factorized cross-gram over compact routed rows.

    ``a*``/``g*`` are the expert's (rows, width) captures in routed order and
    ``tok*`` the flat token index of every row; equals the reference's ghost
    product on the zero-filled ``(B, T, d)`` regroup."""
    return moe_cross_gram([(a1, g1, tok1, a2, g2, tok2)], batch1=batch1, tokens1=tokens1, batch2=batch2,
                          tokens2=tokens2, bias=bias, out=out, accumulate=accumulate)


def route_segments(top_idx: torch.Tensor, n_experts: int, batch: int, tokens: int,
                   rows_per_expert=None) -> list[tuple[torch.Tensor, torch.Tensor]]:
    """Per-sample segments of every expert straight from the top-k indices, in
    one launch: ``(seg, rows)`` per expert, the same as
    ``segment_experts([tok of expert_rows(top_idx)], batch, tokens)``.

    ``rows_per_expert`` (host ints, e.g. the captures' row counts) avoids
    reading the expert sizes back from the device."""
    offsets, _entries, seg, rows = kernels.moe_route(top_idx.reshape(-1, top_idx.shape[-1]).to(torch.int64),
                                                     n_experts, batch, tokens)
    if rows_per_expert is None:
        rows_per_expert = (offsets[1:] - offsets[:-1]).cpu().tolist()
    out, start = [], 0
    for e, r in enumerate(rows_per_expert):
        out.append((seg[e], rows[start:start + int(r)]))
        start += int(r)
    return out


def segment_experts(expert_tokens, batch: int, tokens: int) -> list[tuple[torch.Tensor, torch.Tensor]]:
    """Per-sample segments of every expert of one side: ``expert_tokens[e]`` is
    expert e's flat token index per routed row; returns ``(seg, rows)`` per
    expert (see :func:`segment_by_sample`).  The routing is shared by every
    routed layer, so this runs once per routing, not per layer."""
    return [segment_by_sample(tok, batch, tokens) for tok in expert_tokens]


def moe_layers_cross_gram(layers, segs1, segs2, *, out: torch.Tensor | None = None, accumulate: bool = False):
    """Cross-gram summed over experts AND routed layers in one grouped launch.

    ``layers`` is a list of ``(experts, bias)`` with ``experts[e] = (a1, g1,
    a2, g2)`` -- expert e's (rows, width) captures of that layer on both
    sides, in routed order -- and ``segs*[e] = (seg, rows)`` the per-sample
    segments of expert e's rows (:func:`segment_experts`), shared by all
    layers.  Groups are ordered widest layer first so the longest tiles are
    scheduled first."""
    groups1, groups2, biases, widths = [], [], [], []
    auto = dtypes.get_compute_dtype() == "auto"
    for experts, bias in layers:
        if len(experts) != len(segs1) or len(experts) != len(segs2):
            raise ValueError("one (a1, g1, a2, g2) per expert, matching the segment lists")
        for e, (a1, g1, a2, g2) in enumerate(experts):
            dt = a1.dtype
            # operands already in one kernel dtype under the "auto" policy
            # pass as they are (a model's many experts: no per-expert casts)
            if not (auto and g1.dtype == dt and a2.dtype == dt and g2.dtype == dt and dt in _KERNEL_DTYPES):
                a1, g1, a2, g2 = dtypes.align(a1, g1, a2, g2)
                kd = dtypes.kernel_dtype(a1.dtype)
                a1, g1, a2, g2 = a1.to(kd), g1.to(kd), a2.to(kd), g2.to(kd)
            groups1.append((a1, g1, *segs1[e]))
            groups2.append((a2, g2, *segs2[e]))
            biases.append(bool(bias))
            widths.append(a1.shape[-1] + g1.shape[-1])
    if not groups1:
        raise ValueError("moe_layers_cross_gram needs at least one layer with experts")
    order = sorted(range(len(groups1)), key=lambda i: -widths[i])
    return kernels.ghost_gram_grouped([groups1[i] for i in order], [groups2[i] for i in order],
                                      bias=[biases[i] for i in order], out=out, accumulate=accumulate)


def moe_cross_gram(experts, *, batch1: int, tokens1: int, batch2: int, tokens2: int, bias: bool = False,
                   out: torch.Tensor | None = None, accumulate: bool = False):
    """Segment-sum over experts: ``experts`` yields ``(a1, g1, tok1, a2, g2, tok2)``
    per expert; returns the fp32 ``(B1, B2)`` total.

    All experts go to one grouped launch: each expert's rows are grouped by
    sample (stable counting sort of ``tok // tokens``) and tiled as packed
    rows, so no tile is spent on the zero rows of the reference's regroup."""
    experts = list(experts)
    if not experts:
        raise ValueError("moe_cross_gram needs at least one expert")
    segs1 = segment_experts([x[2] for x in experts], batch1, tokens1)
    segs2 = segment_experts([x[5] for x in experts], batch2, tokens2)
    layer = ([(a1, g1, a2, g2) for a1, g1, _t1, a2, g2, _t2 in experts], bias)
    return moe_layers_cross_gram([layer], segs1, segs2, out=out, accumulate=accumulate)
