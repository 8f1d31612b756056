"""Where routed token rows came from: the per-sample layout of a Mixture-of-
Experts expert's 2-D capture (``dattri_llm/gradient/hooks/routing.py``).

An expert sees ``(n, d)`` rows gathered from its block's ``(B*T, d)`` input.
:func:`locate_rows` finds each row's token -- the k-th occurrence of a row
value takes the k-th token (ascending) holding it, verified exactly -- with
the ``da_match_rows`` kernels (fingerprints, stable sorts, one comparison per
row), and returns the reference's :class:`RowLayout` (routing.py:52-86), whose
:meth:`RowLayout.regroup` scatters a capture back to ``(B, T, ...)`` with zero
rows where a sample's token was not routed.  ``locate_rows`` is the drop-in
for ``RoutedTokenTracker._match`` (routing.py:300-333).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from dattri_llm_amd import kernels


@dataclass(frozen=True)
class RowLayout:
    """Sample and sequence position of each row of a routed 2-D capture;
    ``sample is None`` when the rows are the block's tokens in order."""

    batch: int
    tokens: int
    rows: int
    sample: torch.Tensor | None = None
    position: torch.Tensor | None = None

    def regroup(self, t: torch.Tensor) -> torch.Tensor:
        """``t``'s ``(rows, ...)`` rows laid out as ``(batch, tokens, ...)``
        (zero where no row lands).  Raises ``ValueError`` on a row-count mismatch."""
        if t.shape[0] != self.rows:
            raise ValueError(f"routed capture has {t.shape[0]} rows but the layout holds {self.rows}.")
        if self.sample is None:
            return t.reshape(self.batch, self.tokens, *t.shape[1:])
        out = t.new_zeros((self.batch, self.tokens, *t.shape[1:]))
        out[self.sample.to(t.device), self.position.to(t.device)] = t
        return out


def locate_rows(x: torch.Tensor, src_flat: torch.Tensor, batch: int, tokens: int) -> RowLayout | None:
    """Layout of ``x``'s rows within the block input ``src_flat (batch*tokens,
    d)``, or None when they are not its rows (a value it does not hold, or more
    copies of a value than it holds)."""
    n = x.shape[0]
    if src_flat.shape[0] != batch * tokens:
        raise ValueError(f"block input has {src_flat.shape[0]} rows, expected {batch} x {tokens}")
    # The block's own rows in order (routing.py:303-304): float equality, so
    # rows that differ only in the sign of a zero still match here.
    if n == batch * tokens and x.shape == src_flat.shape and bool(torch.equal(x, src_flat)):
        return RowLayout(batch, tokens, n)
    token = kernels.match_rows(src_flat, x)
    if token is None:
        return None
    if n == batch * tokens and bool(torch.equal(token, torch.arange(n, device=token.device))):
        return RowLayout(batch, tokens, n)
    sample = torch.div(token, tokens, rounding_mode="floor")
    return RowLayout(batch, tokens, n, sample, token - sample * tokens)


__all__ = ["RowLayout", "locate_rows"]
