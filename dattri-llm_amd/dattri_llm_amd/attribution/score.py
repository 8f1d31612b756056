"""Attribution scores keyed by sample hash, trajectory-aware.

The container of ``dattri_llm/attribution/score.py:49-470``: a
``(num_rows, num_test)`` fp32 matrix whose row ``r`` is training sample
``row_train_ids[r]`` at step ``row_steps[r]`` (optionally token position
``row_token_ids[r]``), columns keyed by ``test_ids``.  The on-disk format --
``scores.pt`` (a plain tensor) plus ``metadata.json`` with the same keys --
is the reference's, so scores written by either implementation load in the
other.
"""

from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import torch


@dataclass
class AttributionScore:
    scores: torch.Tensor
    row_train_ids: list[str]
    row_steps: list[int]
    test_ids: list[str]
    algorithm: str
    algorithm_meta: dict[str, Any]
    layer_name: list[str] | None
    row_token_ids: list[int] | None = None

    train_index: dict[str, list[tuple[int, int]]] = field(init=False, repr=False)
    test_index: dict[str, int] = field(init=False, repr=False)

    _SCORES_FILE = "scores.pt"
    _META_FILE = "metadata.json"

    def __post_init__(self) -> None:
        n_rows = self.scores.shape[0]
        if not (len(self.row_train_ids) == len(self.row_steps) == n_rows):
            raise ValueError(
                f"row_train_ids ({len(self.row_train_ids)}) and row_steps ({len(self.row_steps)}) "
                f"must both equal num_rows ({n_rows})."
            )
        if len(self.test_ids) != self.scores.shape[1]:
            raise ValueError(f"test_ids ({len(self.test_ids)}) must equal num_test ({self.scores.shape[1]}).")
        if self.row_token_ids is not None and len(self.row_token_ids) != n_rows:
            raise ValueError(f"row_token_ids ({len(self.row_token_ids)}) must equal num_rows ({n_rows}).")
        index: dict[str, list[tuple[int, int]]] = {}
        for r, (h, step) in enumerate(zip(self.row_train_ids, self.row_steps, strict=True)):
            index.setdefault(h, []).append((step, r))
        for entries in index.values():
            entries.sort()
        self.train_index = index
        self.test_index = {h: c for c, h in enumerate(self.test_ids)}

    @property
    def granularity(self) -> str:
        return "instance" if self.row_token_ids is None else "token"

    @property
    def train_ids(self) -> list[str]:
        """Distinct training hashes in row order."""
        return list(dict.fromkeys(self.row_train_ids))

    @property
    def num_rows(self) -> int:
        return self.scores.shape[0]

    @property
    def num_train(self) -> int:
        return len(self.train_index)

    @property
    def num_test(self) -> int:
        return self.scores.shape[1]

    def _require_train(self, h: str):
        if h not in self.train_index:
            raise KeyError(f"train hash {h[:16]}... not in scores.")
        return self.train_index[h]

    def _require_test(self, h: str) -> int:
        if h not in self.test_index:
            raise KeyError(f"test hash {h[:16]}... not in scores.")
        return self.test_index[h]

    def trajectory_aware(self, train_hash: str) -> tuple[list[int], torch.Tensor]:
        """(steps, (len(steps), num_test)) per-step rows; token rows summed per step."""
        entries = self._require_train(train_hash)
        by_step: dict[int, list[int]] = {}
        for step, r in entries:
            by_step.setdefault(step, []).append(r)
        steps = sorted(by_step)
        return steps, torch.stack([self.scores[by_step[s]].sum(dim=0) for s in steps])

    def token_scores(self, train_hash: str, step: int | None = None) -> tuple[list[int], torch.Tensor]:
        """(positions, (len(positions), num_test)) per-token-position scores of one
        training sample (score.py:185-226); ``step=None`` sums the positions over
        every step the sample appears at."""
        if self.row_token_ids is None:
            raise ValueError("token_scores() needs a token-level score; attribute with "
                             "attribution_granularity='token'.")
        entries = self._require_train(train_hash)
        rows = [r for s, r in entries if step is None or s == step]
        if not rows:
            known = sorted({s for s, _ in entries})
            raise KeyError(f"train sample {train_hash[:16]}... has no row at step {step}; known steps: {known}")
        by_pos: dict[int, list[int]] = {}
        for r in rows:
            by_pos.setdefault(self.row_token_ids[r], []).append(r)
        positions = sorted(by_pos)
        return positions, torch.stack([self.scores[by_pos[p]].sum(dim=0) for p in positions])

    def trajectory_agnostic(self, train_hash: str) -> torch.Tensor:
        return self.trajectory_aware(train_hash)[1].sum(dim=0)

    def agnostic_matrix(self) -> tuple[list[str], torch.Tensor]:
        ids = self.train_ids
        out = self.scores.new_zeros(len(ids), self.num_test)
        for i, h in enumerate(ids):
            for _, r in self.train_index[h]:
                out[i] += self.scores[r]
        return ids, out

    def column(self, test_hash: str) -> torch.Tensor:
        return self.scores[:, self._require_test(test_hash)]

    def step_matrix(self, step: int) -> tuple[list[str], torch.Tensor]:
        """The rows recorded at ``step`` (score.py:278-304): instance rows as
        stored, in row order (a sample stored twice at one step keeps both
        rows); token rows summed per sample, in first-seen order."""
        rows = [i for i, s in enumerate(self.row_steps) if s == step]
        if not rows:
            raise KeyError(f"step {step} not present in scores.")
        if self.row_token_ids is None:
            return [self.row_train_ids[i] for i in rows], self.scores[rows]
        ids = list(dict.fromkeys(self.row_train_ids[i] for i in rows))
        pos = {h: i for i, h in enumerate(ids)}
        out = self.scores.new_zeros(len(ids), self.num_test)
        for i in rows:
            out[pos[self.row_train_ids[i]]] += self.scores[i]
        return ids, out

    def step_matrices(self) -> dict[int, tuple[list[str], torch.Tensor]]:
        """``{step: step_matrix(step)}`` for every recorded step, ascending (score.py:306-318)."""
        return {step: self.step_matrix(step) for step in sorted(set(self.row_steps))}

    def score_at(self, train_hash: str, step: int, test_hash: str) -> torch.Tensor:
        col = self._require_test(test_hash)
        rows = [r for s, r in self._require_train(train_hash) if s == step]
        if not rows:
            known = sorted({s for s, _ in self.train_index[train_hash]})
            raise KeyError(f"train sample {train_hash[:16]}... has no row at step {step}; known steps: {known}")
        return self.scores[rows, col].sum() if len(rows) > 1 else self.scores[rows[0], col]

    def query(self, train_hashes=None, test_hashes=None, trajectory: str = "agnostic") -> torch.Tensor:
        if trajectory not in ("aware", "agnostic"):
            raise ValueError(f"trajectory must be 'aware' or 'agnostic', got {trajectory!r}.")
        train_hashes = list(train_hashes) if train_hashes is not None else self.train_ids
        cols = list(range(self.num_test)) if test_hashes is None else [self._require_test(h) for h in test_hashes]
        if trajectory == "agnostic":
            return torch.stack([self.trajectory_agnostic(h) for h in train_hashes])[:, cols]
        rows = [r for h in train_hashes for _, r in self._require_train(h)]
        return self.scores[rows][:, cols]

    def save(self, out_dir) -> Path:
        out = Path(out_dir)
        out.mkdir(parents=True, exist_ok=True)
        torch.save(self.scores, out / self._SCORES_FILE)
        meta = {
            "row_train_ids": self.row_train_ids,
            "row_steps": self.row_steps,
            "test_ids": self.test_ids,
            "algorithm": self.algorithm,
            "algorithm_meta": self.algorithm_meta,
            "layer_name": self.layer_name,
            "row_token_ids": self.row_token_ids,
            "granularity": self.granularity,
            "num_train": self.num_train,
            "num_test": self.num_test,
            "num_rows": self.num_rows,
        }
        with open(out / self._META_FILE, "w", encoding="utf-8") as f:
            json.dump(meta, f, indent=2)
        return out

    @classmethod
    def load(cls, out_dir) -> AttributionScore:
        out = Path(out_dir)
        scores = torch.load(out / cls._SCORES_FILE, weights_only=True)
        with open(out / cls._META_FILE, encoding="utf-8") as f:
            meta = json.load(f)
        algorithm_meta = meta.get("algorithm_meta", {})
        if "normalized_grad" in meta:
            algorithm_meta.setdefault("normalized_grad", meta["normalized_grad"])
        return cls(scores=scores, row_train_ids=meta["row_train_ids"], row_steps=meta["row_steps"],
                   test_ids=meta["test_ids"], algorithm=meta["algorithm"], algorithm_meta=algorithm_meta,
                   layer_name=meta["layer_name"], row_token_ids=meta.get("row_token_ids"))
