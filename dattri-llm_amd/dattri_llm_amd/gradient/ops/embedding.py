"""Embedding layers (``nn.Embedding``, ``nn.EmbeddingBag``) on the MI355X kernels.

An embedding's per-sample weight gradient is ``dW = sum_t e_{tok_t} g_t^T``: the
activation factor is a one-hot row per token, so every product of two such
gradients only pairs tokens with equal ids.  The reference builds a
``(vocab, E)`` scatter-add table per side-2 sample and gathers from it
(``dattri_llm/gradient/ops/dot.py:58-74``, ``:189-203``, ``:325-337``); here
side 2 is compacted to each sample's distinct ids (fp32 row sums, sorted ids)
and every side-1 token is looked up in it, so no vocabulary-sized table is
formed and no token pair is multiplied:

* :func:`gram32` / :func:`diag32` -- ``da_embedding_cross_gram`` (all pairs, or
  the diagonal pairs for per-sample dots and squared norms);
* :func:`per_token32` -- ``da_embedding_cross_gram_per_token``;
* :func:`dense_per_token32` -- ``da_dense_per_token_embedding``, side 2 dense;
* :func:`materialize` -- ``da_materialize_embedding``, the deterministic
  scatter-add of ``materialize.py:22-48``.

Operands are ``(ids, g)`` pairs from :func:`side`: int64 ids with padding
positions set to -1 (they match and scatter nothing, as the reference's
zeroed gradient rows contribute nothing) and the per-token gradient rows.
"""

from __future__ import annotations

import torch

from dattri_llm_amd import kernels
from dattri_llm_amd.gradient.ops import dtypes
from dattri_llm_amd.gradient.ops.preprocess import final_embedding


def check_ids(*toks: torch.Tensor, vocab: int | None = None) -> None:
    """Raise ``ValueError`` for a negative id, or one at or above ``vocab``
    (materialize.py:37-44): one host read of every tensor's min and max."""
    live = [t for t in toks if t is not None and t.numel() > 0]
    if not live:
        return
    bounds = torch.stack([torch.stack([t.min(), t.max()]).to(torch.int64) for t in live]).tolist()
    lo = min(b[0] for b in bounds)
    hi = max(b[1] for b in bounds)
    if lo < 0:
        raise ValueError(f"Embedding token id {lo} is negative; token ids index the embedding table.")
    if vocab is not None and hi >= vocab:
        raise ValueError(
            f"Embedding token id {hi} is out of range for the declared num_embeddings={vocab}; the "
            "module_kwargs do not match the captured data."
        )


def side(a, g, layer_type: str, module_kwargs: dict | None):
    """Kernel operands ``(ids, g)`` of one raw or preprocessed embedding side."""
    ids, rows = final_embedding(a, g, layer_type, module_kwargs)
    if ids.dim() != 2 or rows.dim() != 3:
        raise ValueError(f"{layer_type} factors must be (B, T) ids and (B, T, E) gradients")
    return ids, rows


def _rows(*gs):
    (out), _ = _kernel_rows(*gs)
    return out


def _kernel_rows(*gs):
    aligned = dtypes.align(*gs)
    out_dtype = aligned[0].dtype
    kd = dtypes.kernel_dtype(out_dtype)
    return tuple(t.to(kd) for t in aligned), out_dtype


def gram32(s1, s2, out=None, accumulate=False) -> torch.Tensor:
    """fp32 (B1, B2) cross-gram of two embedding sides."""
    (ids1, g1), (ids2, g2) = s1, s2
    if s1 is s2:
        (g1,) = _rows(g1)
        return kernels.embedding_cross_gram(ids1, g1, ids1, g1, out=out, accumulate=accumulate)
    g1, g2 = _rows(g1, g2)
    return kernels.embedding_cross_gram(ids1, g1, ids2, g2, out=out, accumulate=accumulate)


def diag32(s1, s2) -> torch.Tensor:
    """fp32 (B,) per-sample dots of two embedding sides of one batch size (the
    squared norms when both are the same side)."""
    (ids1, g1), (ids2, g2) = s1, s2
    if s1 is s2:
        (g1,) = _rows(g1)
        return kernels.embedding_cross_gram(ids1, g1, ids1, g1, diag=True)
    g1, g2 = _rows(g1, g2)
    return kernels.embedding_cross_gram(ids1, g1, ids2, g2, diag=True)


def per_token32(s1, s2) -> torch.Tensor:
    """fp32 (B1, T1, B2): side 1's token t against side 2's whole gradient."""
    (ids1, g1), (ids2, g2) = s1, s2
    g1, g2 = _rows(g1, g2)
    return kernels.embedding_cross_gram_per_token(ids1, g1, ids2, g2)


def dense_per_token32(s1, m2: torch.Tensor) -> torch.Tensor:
    """fp32 (B1, T1, B2) against dense per-sample gradients ``m2 (B2, vocab*E)``
    (materialize's layout); the vocab is ``m2``'s width over E."""
    ids1, g1 = s1
    e = g1.shape[-1]
    m2 = m2.reshape(m2.shape[0], -1)
    if m2.shape[1] % e:
        raise ValueError(f"dense embedding gradient width {m2.shape[1]} is not a multiple of E={e}")
    vocab = m2.shape[1] // e
    check_ids(ids1.masked_fill(ids1 < 0, 0), vocab=vocab)
    g1, m2 = _rows(g1, m2)
    return kernels.dense_per_token_embedding(ids1, g1, m2, vocab)


def materialize(s, vocab: int) -> torch.Tensor:
    """(B, vocab*E) per-sample weight gradient in the compute dtype."""
    ids, g = s
    (g,), out_dtype = _kernel_rows(g)
    return kernels.materialize_embedding(ids, g, vocab).to(out_dtype)
