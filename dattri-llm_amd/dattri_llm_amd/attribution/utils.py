"""The inner-product scoring loop over gradient sources.

Mirrors ``dattri_llm/attribution/utils.py`` (``finalize_factors`` :180-236,
``score_sources`` :239-440) and ``rebatch_blocks``
(``dattri_llm/gradient/streaming.py:197-268``).  Sources are iterables of
``(step, Gradient, hashes)`` blocks -- the reference's ``GradientSource``
protocol -- so its ``GradientStreamer`` / ``DiskGradientSource`` plug in
unchanged.  Scores are accumulated on the device in fp32 and copied to the
host once per train block (the reference syncs once per train x test block
pair).
"""

from __future__ import annotations

import math
from typing import TYPE_CHECKING

import torch

from dattri_llm_amd.gradient import ops
from dattri_llm_amd.gradient.gradient import Factorized, Gradient
from dattri_llm_amd.utils.cache import CacheBudget, TensorCache

if TYPE_CHECKING:
    from collections.abc import Callable, Iterable, Iterator


def finalize_factors(rep: Gradient, *, budget: CacheBudget | None = None, held: int = 0) -> Gradient:
    """Preprocess every raw factorized layer once (utils.py:180-236).

    Linear layers need no rewrite here: their bias column is applied inside
    the kernels (an implicit ones column), so the raw capture *is* the final
    form and keeping ``module_kwargs`` costs nothing.  Norm layers (x_hat,
    with the bias block) and convolutions (the unfolded patches, with the ones
    column) are replaced by their final factors exactly as the reference does,
    under the same budget rule; embeddings stay raw."""
    names = [
        n for n, v in rep.data.items()
        if isinstance(v, Factorized) and v.module_kwargs is not None
        and (ops.is_norm(rep.layer_types[n]) or ops.is_conv(rep.layer_types[n])
             or ops.is_conv_transpose(rep.layer_types[n]))
    ]
    if not names:
        return rep
    charged = held

    def finalize(_name, value: Factorized, layer_type):
        nonlocal charged
        a, g = ops.preprocess_factorized(value, layer_type)
        final = Factorized(activation=a, pre_activation_grad=g, module_kwargs=None)
        growth = max(final.nbytes - value.nbytes, 0)
        if budget is not None and not budget.fits(growth, charged):
            return value
        charged += growth
        return final

    return rep.map_layers(finalize, layers=names, consume=True)


def rebatch_blocks(source: Iterable, batch_size: int) -> Iterator[tuple[list[int], Gradient, list[str]]]:
    """Re-batch dense blocks into ``batch_size``-sample batches; factorized
    blocks pass one at a time (streaming.py:197-268)."""
    if batch_size < 1:
        raise ValueError(f"batch_size must be >= 1, got {batch_size}.")
    pending: dict[str, list[torch.Tensor]] = {}
    ids: list[str] = []
    steps: list[int] = []
    count = 0
    meta = None

    def build():
        nonlocal pending, ids, steps, count
        data = {n: t[0] if len(t) == 1 else torch.cat(t, dim=0) for n, t in pending.items()}
        rep, lt, ix = meta
        batch = (steps, Gradient(rep, data, lt, ix, validate_on_init=False), ids)
        pending, ids, steps, count = {}, [], [], 0
        return batch

    for step, block, hashes in source:
        if not all(isinstance(v, torch.Tensor) for v in block.data.values()):
            if count:
                yield build()
            yield [step] * block.batch_size, block, list(hashes)
            continue
        meta = (block.representation, block.layer_types, block.indexing)
        for name, tensor in block.data.items():
            pending.setdefault(name, []).append(tensor)
        ids.extend(hashes)
        steps.extend([step] * block.batch_size)
        count += block.batch_size
        if count >= batch_size:
            yield build()
    if count:
        yield build()


def _merge_dense_test(cached: list) -> list:
    """Stack all-dense cached test reps into one block (utils.py:159-177)."""
    if len(cached) < 2:
        return cached
    stream = ((0, rep, cols) for rep, cols in cached)
    merged = list(rebatch_blocks(stream, batch_size=sum(len(c) for _, c in cached)))
    return [(rep, cols) for _s, rep, cols in merged]


def score_sources(
    train_source: Iterable,
    test_source: Iterable,
    device,
    *,
    inner_product: Callable,
    transform_train: Callable | None = None,
    transform_test: Callable | None = None,
    batch_size: int = 1,
    loop_over_test: bool = False,
    cache_budget: CacheBudget | None = None,
    granularity: str = "instance",
    inner_product_per_token: Callable | None = None,
    train_blocks_per_pass: int = 1,
    dense_group: Callable | None = None,
):
    """Score every train block against every test block (utils.py:239-440).

    The test source is iterated once to fix the column order (first-seen
    hashes) and, by default, to cache the transformed test blocks, merged
    into one block when they are all dense.  With ``loop_over_test`` nothing
    is cached: the test source (which must be ``reusable``) is re-streamed
    and re-transformed for every train block, and train blocks are scored one
    at a time.  The dense cache handed to ``inner_product`` lives for one
    train block; it is ``None`` when a cached train block meets a single
    test block.

    ``granularity="instance"`` gives one row per training sample;
    ``"token"`` one row per training token position, scored by
    ``inner_product_per_token(train_rep, test_rep) -> (B_train, T, B_test)``
    (a sample of T positions contributes T consecutive rows).

    ``train_blocks_per_pass`` > 1 (instance level, cached test side held as
    one dense block): that many train blocks are made dense together by
    ``dense_group(reps) -> Gradient`` and scored in one pass over the test
    block, which is then read once per group instead of once per train block.
    The scores are those of the block-by-block loop.  A group holds no more
    blocks than ``cache_budget`` has room for (their dense rows, re-read at
    the start of every group), and blocks that cannot be stacked with the
    same scores (:func:`groupable`: differing layers, broadcast or batch-level
    layers) are scored one at a time.

    Returns ``(scores (rows, num_test) fp32 CPU, row_train_ids, row_steps,
    test_ids, row_token_ids or None)``."""
    if loop_over_test and not getattr(test_source, "reusable", False):
        raise ValueError(
            "loop_over_test=True requires a re-iterable test source (reusable=True); got a single-shot source.",
        )
    if granularity not in {"instance", "token"}:
        raise ValueError(f"granularity must be 'instance' or 'token', got {granularity!r}.")
    per_token = granularity == "token"
    if train_blocks_per_pass < 1:
        raise ValueError(f"train_blocks_per_pass must be >= 1, got {train_blocks_per_pass}.")
    if train_blocks_per_pass > 1 and dense_group is None:
        raise ValueError("train_blocks_per_pass > 1 needs dense_group.")
    if per_token and inner_product_per_token is None:
        raise ValueError("granularity='token' needs inner_product_per_token.")
    transform_train = transform_train or (lambda g: g)
    transform_test = transform_test or (lambda g: g)
    budget = cache_budget if cache_budget is not None else CacheBudget(device)
    test_ids: list[str] = []
    index: dict[str, int] = {}
    cached = []
    for _step, test_g, hashes in test_source:
        cols = []
        for h in hashes:
            if h not in index:
                index[h] = len(test_ids)
                test_ids.append(h)
            cols.append(index[h])
        if not loop_over_test:
            cached.append((transform_test(test_g.to(device)), cols))
    test_g = None  # the last raw test block is not kept beside its transformed copy
    cached = _merge_dense_test(cached)
    num_test = len(test_ids)
    # a dense copy of the train block pays off only against several test blocks,
    # and only the instance-level kernel materializes the train side
    reuse = loop_over_test or (len(cached) > 1 and not per_token)
    grouped = (train_blocks_per_pass > 1 and not loop_over_test and not per_token and len(cached) == 1
               and all(isinstance(v, torch.Tensor) for v in cached[0][0].data.values()))

    def test_blocks():
        if not loop_over_test:
            yield from cached
            return
        for _s, tg, hashes in test_source:
            yield transform_test(tg.to(device)), [index[h] for h in hashes]

    def train_blocks():
        if not loop_over_test:
            yield from rebatch_blocks(train_source, batch_size)
            return
        for step, block, hashes in train_source:
            yield [step] * block.batch_size, block, list(hashes)

    def n_rows(train_rep) -> int:
        if not per_token:
            return train_rep.batch_size
        tokens = [t for t in train_rep.token_dim.values() if t is not None]
        return train_rep.batch_size * (max(tokens) if tokens else 1)

    rows_out = _HostRows()
    row_ids, row_steps, row_tokens = [], [], []

    def scored_blocks():
        if not grouped:
            for steps, train_g, ids in train_blocks():
                yield steps, transform_train(train_g.to(device)), ids
            return
        group: list = []
        limit = train_blocks_per_pass

        def flush(group):
            reps = [transform_train(g.to(device)) for _s, g, _i in group]
            if groupable(reps):
                yield ([s for st, _g, _i in group for s in st], dense_group(reps),
                       [h for _s, _g, ids in group for h in ids])
                return
            for (steps, _g, ids), rep in zip(group, reps, strict=True):
                yield steps, rep, ids

        for item in train_blocks():
            if not group:
                # the group's dense rows must fit the budget beside what is
                # already resident: re-read at the start of every group
                limit = group_limit(item[1], train_blocks_per_pass, budget)
            group.append(item)
            if len(group) >= limit:
                yield from flush(group)
                group = []
        if group:
            yield from flush(group)

    for steps, train_rep, ids in scored_blocks():
        row = torch.zeros(n_rows(train_rep), num_test, dtype=torch.float32, device=device)
        cache = TensorCache("memory", budget=budget) if reuse else None
        for test_rep, cols in test_blocks():
            if per_token:
                block = inner_product_per_token(train_rep, test_rep).to(torch.float32)
                block = block.reshape(-1, block.shape[-1])
            else:
                block = inner_product(train_rep, test_rep, dense_cache=cache).to(torch.float32)
            if cols and cols == list(range(cols[0], cols[0] + len(cols))):
                row[:, cols[0]:cols[0] + len(cols)] = block
            else:
                row[:, torch.tensor(cols, device=device)] = block
        if cache is not None:
            cache.clear()
        rows_out.add(row)
        if per_token:
            t = row.shape[0] // max(len(ids), 1)
            for h, st in zip(ids, steps, strict=True):
                row_ids.extend([h] * t)
                row_steps.extend([st] * t)
                row_tokens.extend(range(t))
        else:
            row_ids.extend(ids)
            row_steps.extend(steps)
        # Drop this block before the next one is built: a dense group of 8 C4
        # blocks is 28 GB, and holding it while the next one materializes
        # doubles the peak and can make the caching allocator free and map
        # tens of GB again (a 1-2 s stall).
        del train_rep
    scores = rows_out.result(num_test)
    return scores, row_ids, row_steps, test_ids, (row_tokens if per_token else None)


def _layer_rows(value) -> int:
    if isinstance(value, Factorized):
        return value.as_batch_first().activation.shape[0]
    return value.shape[0]


def groupable(reps: list[Gradient]) -> bool:
    """Whether train blocks can be stacked into one dense block with the
    scores of the block-by-block loop: the same layers with the same types in
    every block, each layer holding one row per sample (no broadcast row, no
    batch-level ``param_grad`` layer, which the per-block loop treats apart)."""
    first = reps[0]
    names = list(first.data)
    for rep in reps:
        if list(rep.data) != names:
            return False
        for name in names:
            layer_type = rep.layer_types.get(name)
            if layer_type != first.layer_types.get(name) or layer_type == ops.PARAM_GRAD_TYPES:
                return False
            if _layer_rows(rep.data[name]) != rep.batch_size:
                return False
    return True


# Rows of the score GEMM's tall tile (a 64 x 64 output tile per workgroup set).
SCORE_TILE_ROWS = 64


def group_limit(block: Gradient, blocks_per_pass: int, budget: CacheBudget) -> int:
    """How many train blocks like ``block`` to make dense together: at most
    ``blocks_per_pass``, and no more than the budget holds (at least one).

    When the budget is what caps the group, the group is cut further so that
    its rows fill whole 64-row score tiles (or stay within one): the tiles of
    one launch stream the query rows in step, and a part-filled tile runs
    ahead of the full ones and reads them again.  On the Llama-8B block (8
    rows per block, 64 query rows, one MI355X) 16 blocks per pass score at
    0.81 ms per block and 24 at 0.69, but 12 at 1.35 and 20 at 0.82."""
    per_block = block.materialized_nbytes
    if per_block <= 0:
        return blocks_per_pass
    room = budget.room() // per_block
    if room >= blocks_per_pass:
        return blocks_per_pass
    return whole_tile_group(max(1, room), block.batch_size)


def whole_tile_group(limit: int, rows: int) -> int:
    """The largest group of at most ``limit`` blocks of ``rows`` rows whose rows
    fill whole ``SCORE_TILE_ROWS``-row tiles, or fit in one; ``limit`` itself
    when one block is taller than a tile."""
    tile = SCORE_TILE_ROWS
    if rows <= 0 or rows > tile or limit * rows <= tile:
        return limit
    step = tile // math.gcd(rows, tile)  # blocks per whole number of tiles
    if limit >= step:
        return limit // step * step
    return max(1, tile // rows)


class _HostRows:
    """Score rows produced on the device, delivered to the host in a few large
    asynchronous copies: rows wait on the device until ``flush_bytes`` of them
    have gathered, then go to one pinned buffer on the device's current stream.
    The loop never waits on a copy and pays one pinned allocation per flush
    rather than one per block (whose first allocations can stall the stream)."""

    def __init__(self, flush_bytes: int = 256 << 20) -> None:
        self.flush_bytes = flush_bytes
        self.pending: list[torch.Tensor] = []
        self.pending_bytes = 0
        self.host: list[torch.Tensor] = []
        self.device = None

    def add(self, row: torch.Tensor) -> None:
        if not row.is_cuda:
            self.host.append(row)
            return
        self.device = row.device
        self.pending.append(row)
        self.pending_bytes += row.numel() * row.element_size()
        if self.pending_bytes >= self.flush_bytes:
            self._flush()

    def _flush(self) -> None:
        if not self.pending:
            return
        block = self.pending[0] if len(self.pending) == 1 else torch.cat(self.pending, dim=0)
        host = torch.empty(block.shape, dtype=block.dtype, pin_memory=True)
        host.copy_(block, non_blocking=True)
        self.host.append(host)
        self.pending, self.pending_bytes = [], 0

    def result(self, num_test: int) -> torch.Tensor:
        self._flush()
        if self.device is not None:
            torch.cuda.synchronize(self.device)
        return torch.cat(self.host, dim=0) if self.host else torch.zeros(0, num_test)
