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
    seg1, rows1 = segment_by_sample(tok1, batch1, tokens1)
    seg2, rows2 = segment_by_sample(tok2, batch2, tokens2)
    (a1, g1, a2, g2) = dtypes.align(a1, g1, a2, g2)
    kd = dtypes.kernel_dtype(a1.dtype)
    return kernels.ghost_gram_segmented(
        a1.to(kd), g1.to(kd), seg1, rows1, tokens1, a2.to(kd), g2.to(kd), seg2, rows2, tokens2,
        bias=bias, out=out, accumulate=accumulate)


def moe_cross_gram(experts, *, batch1: int, tokens1: int, batch2: int, tokens2: int, bias: bool = False):
    """Segment-sum over experts: ``experts`` yields ``(a1, g1, tok1, a2, g2, tok2)``
    per expert; returns the fp32 ``(B1, B2)`` total."""
    out = None
    for a1, g1, tok1, a2, g2, tok2 in experts:
        if out is None:
            out = torch.zeros(batch1, batch2, dtype=torch.float32, device=a1.device)
        if a1.shape[0] == 0 or a2.shape[0] == 0:
            continue
        expert_cross_gram(a1, g1, tok1, a2, g2, tok2, batch1=batch1, tokens1=tokens1, batch2=batch2,
                          tokens2=tokens2, bias=bias, out=out, accumulate=True)
    if out is None:
        raise ValueError("moe_cross_gram needs at least one expert")
    return out
