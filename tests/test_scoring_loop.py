"""The scoring loop's host logic on the CPU (the reference's
tests/attribution/test_utils.py:229-556): score_sources over in-memory
sources with an injected inner product -- column order by first-seen hash,
row ids and steps, invariance to the train batch size, mixed dense /
factorized streams, empty sources, the loop_over_test mode and its source
requirement, the transforms, merged dense test blocks and the dense cache's
scope -- rebatch_blocks, and the token-level AttributionScore read through its
instance accessors (tests/attribution/test_token_granularity.py:135-166)."""

from __future__ import annotations

import pytest
import torch

from dattri_llm_amd.attribution.utils import rebatch_blocks, score_sources
from dattri_llm_amd.gradient.gradient import Factorized, Gradient
from dattri_llm_amd.utils.cache import TensorCache

B, T, D_IN, D_OUT = 2, 4, 3, 5


def dense_block(seed=0, b=B):
    g = torch.Generator().manual_seed(seed)
    return Gradient({"l1": "materialized"}, {"l1": torch.randn(b, D_IN * D_OUT, generator=g)}, {"l1": "nn.Linear"})


def factorized_block(seed=0, b=B):
    g = torch.Generator().manual_seed(seed)
    return Gradient({"l1": "factorized"},
                    {"l1": Factorized(torch.randn(b, T, D_IN, generator=g), torch.randn(b, T, D_OUT, generator=g))},
                    {"l1": "nn.Linear"}, {"l1": "batch_token"})


def stream(n=4, factory=dense_block):
    return [(i, factory(seed=i), [f"h{i}-{j}" for j in range(B)]) for i in range(n)]


class Source:
    """An in-memory (step, Gradient, hashes) source."""

    def __init__(self, blocks, reusable=True):
        self.blocks, self._reusable, self.passes = blocks, reusable, 0

    def __iter__(self):
        self.passes += 1
        return iter(self.blocks)

    @property
    def reusable(self):
        return self._reusable


def flat(g):
    v = g.data["l1"]
    if isinstance(v, Factorized):
        bf = v.as_batch_first()
        return torch.einsum("bti,bto->boi", bf.activation, bf.pre_activation_grad).flatten(1)
    return v


def dot(train_rep, test_rep, *, dense_cache=None):
    return flat(train_rep) @ flat(test_rep).T


def sources(n_train=3, n_test=2, reusable=True):
    train = Source(stream(n_train))
    test = Source([(0, dense_block(seed=100 + i), [f"t{i}-0", f"t{i}-1"]) for i in range(n_test)], reusable=reusable)
    return train, test


def expected(train, test):
    return torch.cat([flat(g) for _, g, _ in train.blocks]) @ torch.cat([flat(g) for _, g, _ in test.blocks]).T


def test_scores_rows_and_columns():
    train, test = sources()
    scores, ids, steps, test_ids, tokens = score_sources(train, test, "cpu", inner_product=dot)
    assert torch.allclose(scores, expected(train, test), atol=1e-6)
    assert ids == [h for _, _, hs in train.blocks for h in hs]
    assert test_ids == [h for _, _, hs in test.blocks for h in hs]
    assert steps == [s for s, _g, _ in train.blocks for _ in range(B)]
    assert tokens is None


def test_columns_land_by_first_seen_hash():
    train = Source([(0, dense_block(seed=0), ["r0", "r1"])])
    a, b = dense_block(seed=1), dense_block(seed=2)
    test = Source([(0, a, ["a0", "a1"]), (0, b, ["b0", "b1"])])
    scores, _, _, test_ids, _ = score_sources(train, test, "cpu", inner_product=dot)
    assert test_ids == ["a0", "a1", "b0", "b1"]
    tg = train.blocks[0][1]
    assert torch.allclose(scores[:, :2], flat(tg) @ flat(a).T)
    assert torch.allclose(scores[:, 2:], flat(tg) @ flat(b).T)
    # a hash seen again lands in its first column
    test = Source([(0, a, ["a0", "a1"]), (0, b, ["a1", "b1"])])
    scores, _, _, test_ids, _ = score_sources(train, test, "cpu", inner_product=dot)
    assert test_ids == ["a0", "a1", "b1"]
    assert torch.allclose(scores[:, 1], (flat(tg) @ flat(b).T)[:, 0])


@pytest.mark.parametrize("batch_size", [1, 3, 100])
def test_scores_and_rows_invariant_to_batch_size(batch_size):
    train, test = sources(n_train=4, n_test=1)
    scores, ids, steps, _, _ = score_sources(train, test, "cpu", inner_product=dot, batch_size=batch_size)
    assert ids == [h for _, _, hs in train.blocks for h in hs]
    assert steps == [s for s, g, _ in train.blocks for _ in range(g.batch_size)]
    assert torch.allclose(scores, expected(train, test), atol=1e-6)


def test_mixed_stream_stays_ordered():
    train = Source([(0, dense_block(seed=0), ["m0-a", "m0-b"]), (1, factorized_block(seed=1), ["f1-a", "f1-b"]),
                    (2, dense_block(seed=2), ["m2-a", "m2-b"])])
    test = Source([(0, dense_block(seed=99, b=3), ["t0", "t1", "t2"])])
    scores, ids, steps, _, _ = score_sources(train, test, "cpu", inner_product=dot, batch_size=100)
    assert ids == ["m0-a", "m0-b", "f1-a", "f1-b", "m2-a", "m2-b"]
    assert steps == [0, 0, 1, 1, 2, 2]
    assert scores.shape == (6, 3)
    assert torch.allclose(scores, expected(train, test), atol=1e-5)


def test_empty_train_source():
    train, test = sources(n_train=0, n_test=1)
    scores, ids, steps, test_ids, _ = score_sources(train, test, "cpu", inner_product=dot)
    assert scores.shape == (0, 2) and ids == [] and steps == [] and len(test_ids) == 2


def test_loop_over_test_matches_cached():
    train_a, test_a = sources()
    cached = score_sources(train_a, test_a, "cpu", inner_product=dot)
    train_b, test_b = sources()
    looped = score_sources(train_b, test_b, "cpu", inner_product=dot, loop_over_test=True)
    for got, want in zip(looped, cached, strict=True):
        if isinstance(got, torch.Tensor):
            assert torch.allclose(got, want, atol=1e-6)
        else:
            assert got == want
    # cached: one pass over the test source; looping: the column pass plus one per train block
    assert test_a.passes == 1
    assert test_b.passes == 1 + len(train_b.blocks)


def test_loop_over_test_requires_reusable_source():
    train, test = sources(reusable=False)
    with pytest.raises(ValueError, match="reusable"):
        score_sources(train, test, "cpu", inner_product=dot, loop_over_test=True)


def test_transforms_feed_inner_product():
    train, test = sources(n_train=1, n_test=1)
    seen = []
    train_marker, test_marker = dense_block(seed=7), dense_block(seed=8)

    def inner(train_rep, test_rep, *, dense_cache=None):
        seen.append((train_rep, test_rep))
        return torch.zeros(train_rep.batch_size, test_rep.batch_size)

    score_sources(train, test, "cpu", inner_product=inner, transform_train=lambda g: train_marker,
                  transform_test=lambda g: test_marker)
    assert seen == [(train_marker, test_marker)]


def test_dense_test_blocks_are_merged_into_one():
    seen = []

    def inner(train_rep, test_rep, *, dense_cache=None):
        seen.append((test_rep.batch_size, dense_cache))
        return dot(train_rep, test_rep)

    train, test = sources(n_train=2, n_test=3)
    scores, _, _, test_ids, _ = score_sources(train, test, "cpu", inner_product=inner)
    assert seen == [(6, None), (6, None)]  # one merged 6-column block per train block
    assert test_ids == [h for _, _, hs in test.blocks for h in hs]
    assert torch.allclose(scores, expected(train, test), atol=1e-6)


def test_dense_cache_is_scoped_to_the_train_block():
    caches = []

    def inner(train_rep, test_rep, *, dense_cache=None):
        caches.append(dense_cache)
        if dense_cache is not None:
            dense_cache.get_or_compute("l1", lambda: flat(train_rep))
        return dot(train_rep, test_rep)

    train = Source(stream(2))
    test = Source([(0, factorized_block(seed=100 + i), [f"t{i}-0", f"t{i}-1"]) for i in range(3)])
    score_sources(train, test, "cpu", inner_product=inner)
    assert all(isinstance(c, TensorCache) for c in caches)
    assert len({id(c) for c in caches}) == 2
    assert caches[0] is caches[1] is caches[2] and caches[3] is not caches[0]
    caches.clear()
    train, test = sources(n_train=2, n_test=1)
    score_sources(train, test, "cpu", inner_product=inner)
    assert caches == [None, None]


def test_token_granularity_rows():
    train = Source([(0, factorized_block(seed=0), ["r0", "r1"]), (1, factorized_block(seed=1), ["r2", "r3"])])
    test = Source([(0, dense_block(seed=5), ["q0", "q1"])])

    def per_token(train_rep, test_rep):
        bf = train_rep.data["l1"].as_batch_first()
        rows = torch.einsum("bti,bto->btoi", bf.activation, bf.pre_activation_grad).flatten(2)
        return rows @ flat(test_rep).T

    scores, ids, steps, _, tokens = score_sources(train, test, "cpu", inner_product=dot, granularity="token",
                                                  inner_product_per_token=per_token)
    assert scores.shape == (4 * T, 2)
    assert ids == [h for h in ["r0", "r1", "r2", "r3"] for _ in range(T)]
    assert steps == [0] * (2 * T) + [1] * (2 * T)
    assert tokens == list(range(T)) * 4
    # the token rows of a sample sum to its instance score
    inst, *_ = score_sources(train, test, "cpu", inner_product=dot)
    assert torch.allclose(scores.view(4, T, 2).sum(1), inst, atol=1e-5)
    with pytest.raises(ValueError, match="inner_product_per_token"):
        score_sources(train, test, "cpu", inner_product=dot, granularity="token")
    with pytest.raises(ValueError, match="granularity"):
        score_sources(train, test, "cpu", inner_product=dot, granularity="sentence")


# -- rebatch_blocks (test_utils.py:229-272) ----------------------------------------------------


def test_rebatch_at_boundary_and_remainder():
    out = list(rebatch_blocks(stream(5), batch_size=4))
    assert [len(ids) for _s, _g, ids in out] == [4, 4, 2]
    assert [g.batch_size for _s, g, _ in out] == [4, 4, 2]
    assert [s for steps, _g, _ids in out for s in steps] == [0, 0, 1, 1, 2, 2, 3, 3, 4, 4]


def test_rebatch_preserves_values_and_passes_factorized_through():
    blocks = stream(3)
    (steps, g, ids), = list(rebatch_blocks(blocks, batch_size=100))
    assert torch.equal(g.data["l1"], torch.cat([b.data["l1"] for _s, b, _h in blocks]))
    mixed = [blocks[0], (9, factorized_block(seed=9), ["f-a", "f-b"]), blocks[1]]
    out = list(rebatch_blocks(mixed, batch_size=100))
    assert [ids for _s, _g, ids in out] == [["h0-0", "h0-1"], ["f-a", "f-b"], ["h1-0", "h1-1"]]
    assert out[1][1] is mixed[1][1]
    assert list(rebatch_blocks([], batch_size=3)) == []
    with pytest.raises(ValueError):
        list(rebatch_blocks(stream(1), batch_size=0))


# -- token scores (test_token_granularity.py:135-166) ------------------------------------------


def test_token_score_accessors_agree_with_the_instance_score(tmp_path):
    """A token-level AttributionScore read through the instance accessors is
    the instance score; token_scores gives each sample's positions; the round
    trip through disk keeps the token axis."""
    from dattri_llm_amd.attribution.score import AttributionScore

    train = Source([(0, factorized_block(seed=0), ["r0", "r1"]), (0, factorized_block(seed=1), ["r2", "r3"])])
    test = Source([(0, dense_block(seed=5), ["q0", "q1"])])

    def per_token(train_rep, test_rep):
        bf = train_rep.data["l1"].as_batch_first()
        rows = torch.einsum("bti,bto->btoi", bf.activation, bf.pre_activation_grad).flatten(2)
        return rows @ flat(test_rep).T

    s_t = score_sources(train, test, "cpu", inner_product=dot, granularity="token",
                        inner_product_per_token=per_token)
    s_i = score_sources(train, test, "cpu", inner_product=dot)
    token = AttributionScore(scores=s_t[0], row_train_ids=s_t[1], row_steps=s_t[2], test_ids=s_t[3],
                             algorithm="tracin", algorithm_meta={"attribution_granularity": "token"},
                             layer_name=None, row_token_ids=s_t[4])
    inst = AttributionScore(scores=s_i[0], row_train_ids=s_i[1], row_steps=s_i[2], test_ids=s_i[3],
                            algorithm="tracin", algorithm_meta={}, layer_name=None)
    assert token.granularity == "token" and inst.granularity == "instance"
    assert token.num_rows == 4 * T and token.row_token_ids == list(range(T)) * 4
    ids_t, m_t = token.agnostic_matrix()
    ids_i, m_i = inst.agnostic_matrix()
    assert ids_t == ids_i
    torch.testing.assert_close(m_t, m_i, atol=1e-4, rtol=1e-4)
    for h in ids_t:
        positions, block = token.token_scores(h)
        assert positions == list(range(T))
        torch.testing.assert_close(block.sum(0), inst.trajectory_agnostic(h), atol=1e-4, rtol=1e-4)
        steps, rows = token.trajectory_aware(h)
        assert steps == [0]
        torch.testing.assert_close(rows[0], block.sum(0), atol=1e-4, rtol=1e-4)
    t_ids, t_m = token.step_matrix(0)
    assert t_ids == ids_i
    torch.testing.assert_close(t_m, m_i, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(token.score_at("r0", 0, "q1"), inst.score_at("r0", 0, "q1"), atol=1e-4, rtol=1e-4)
    with pytest.raises(ValueError, match="token"):
        inst.token_scores("r0")
    back = AttributionScore.load(token.save(tmp_path / "tok"))
    assert back.granularity == "token" and back.row_token_ids == token.row_token_ids
    assert torch.equal(back.scores, token.scores)


@pytest.mark.parametrize("loop_over_test", [False, True])
def test_duplicate_test_samples_share_a_column(loop_over_test):
    """Identical test samples (one content hash, inside a block and across
    blocks) collapse to one column, and no column stays zero
    (test_tracin.py:607-628)."""
    a, b = dense_block(seed=100), dense_block(seed=101)
    a.data["l1"][1] = a.data["l1"][0]          # sample 1 repeats sample 0
    b.data["l1"][0] = a.data["l1"][0]          # and so does the next block's first sample
    test = Source([(0, a, ["q0", "q0"]), (0, b, ["q0", "q1"])])
    train = Source(stream(2))
    scores, _ids, _steps, test_ids, _tok = score_sources(train, test, "cpu", inner_product=dot,
                                                         loop_over_test=loop_over_test)
    assert test_ids == ["q0", "q1"] and scores.shape == (2 * B, 2)
    tr = torch.cat([flat(g) for _, g, _ in train.blocks])
    want = tr @ torch.stack([a.data["l1"][0], b.data["l1"][1]]).T
    assert torch.allclose(scores, want, atol=1e-5)
    assert int((scores.abs().sum(0) == 0).sum()) == 0


@pytest.mark.parametrize("per_pass", [2, 3, 8])
def test_train_blocks_per_pass_groups_dense_passes(per_pass):
    """Grouped train blocks give the block-by-block scores, rows and steps; the
    hook sees groups of ``per_pass`` blocks (the last one shorter)."""
    train, test = Source(stream(5)), Source([(0, dense_block(seed=100), ["t0", "t1"])])
    seen = []

    def group(reps):
        seen.append(len(reps))
        data = torch.cat([flat(r) for r in reps])
        return Gradient({"l1": "materialized"}, {"l1": data}, {"l1": "nn.Linear"})

    want = score_sources(train, test, "cpu", inner_product=dot)
    got = score_sources(train, test, "cpu", inner_product=dot, train_blocks_per_pass=per_pass, dense_group=group)
    assert torch.allclose(got[0], want[0], atol=1e-5) and got[1:4] == want[1:4]
    assert seen == [per_pass] * (5 // per_pass) + ([5 % per_pass] if 5 % per_pass else [])
    with pytest.raises(ValueError, match="dense_group"):
        score_sources(train, test, "cpu", inner_product=dot, train_blocks_per_pass=2)


def test_train_blocks_per_pass_needs_one_dense_test_block():
    """A factorized or multi-block test side keeps the block-by-block loop."""
    train, test = Source(stream(3)), Source([(0, factorized_block(seed=100), ["t0", "t1"])])
    calls = []
    score_sources(train, test, "cpu", inner_product=dot, train_blocks_per_pass=2,
                  dense_group=lambda reps: calls.append(reps))
    assert calls == []


def _two_layer_block(seed, b=B, layers=("l1", "l2"), broadcast=()):
    g = torch.Generator().manual_seed(seed)
    data = {n: torch.randn(1 if n in broadcast else b, D_IN * D_OUT, generator=g) for n in layers}
    return Gradient(dict.fromkeys(data, "materialized"), data, dict.fromkeys(data, "nn.Linear"))


def _layer_dot(train_rep, test_rep, *, dense_cache=None):
    """Sum over the layers both sides hold; a one-row train layer is the
    whole block's (broadcast) gradient."""
    total = torch.zeros(train_rep.batch_size, test_rep.batch_size)
    for name, m1 in train_rep.data.items():
        if name in test_rep.data:
            total += (m1 @ test_rep.data[name].T).expand(train_rep.batch_size, -1)
    return total


def _stack(reps):
    data = {n: torch.cat([r.data[n] for r in reps]) for n in reps[0].data}
    return Gradient(dict.fromkeys(data, "materialized"), data, dict.fromkeys(data, "nn.Linear"))


@pytest.mark.parametrize("odd", ["missing_layer", "broadcast_layer", "other_type"])
def test_train_blocks_per_pass_keeps_unstackable_blocks_apart(odd):
    """A group whose blocks differ in their layers, or hold a broadcast
    (one-row) layer, is scored block by block: the scores stay those of the
    per-block loop and the stacking hook never sees such a group."""
    blocks = [_two_layer_block(i) for i in range(4)]
    if odd == "missing_layer":
        blocks[1] = _two_layer_block(1, layers=("l1",))
    elif odd == "broadcast_layer":
        blocks[1] = _two_layer_block(1, broadcast=("l2",))
    else:
        blocks[1].layer_types["l2"] = "nn.Conv2d"
    train = Source([(i, g, [f"h{i}-{j}" for j in range(B)]) for i, g in enumerate(blocks)])
    test = Source([(0, _two_layer_block(100), ["t0", "t1"])])
    seen = []

    def group(reps):
        seen.append(len(reps))
        return _stack(reps)

    want = score_sources(train, test, "cpu", inner_product=_layer_dot)
    got = score_sources(train, test, "cpu", inner_product=_layer_dot, train_blocks_per_pass=2, dense_group=group)
    assert torch.allclose(got[0], want[0], atol=1e-5) and got[1:4] == want[1:4]
    assert seen == [2]  # blocks 0-1 are not stacked, blocks 2-3 are


def test_train_blocks_per_pass_is_capped_by_the_budget():
    """A group holds no more blocks than the cache budget has room for (their
    dense rows), and at least one."""
    from dattri_llm_amd.utils.cache import CacheBudget

    blocks = [_two_layer_block(i) for i in range(5)]
    per_block = blocks[0].materialized_nbytes
    train = Source([(i, g, [f"h{i}-{j}" for j in range(B)]) for i, g in enumerate(blocks)])
    test = Source([(0, _two_layer_block(100), ["t0", "t1"])])
    want = score_sources(train, test, "cpu", inner_product=_layer_dot)
    for room, sizes in ((2 * per_block + 1, [2, 2, 1]), (per_block - 1, [1, 1, 1, 1, 1]), (1 << 40, [4, 1])):
        seen = []

        def group(reps):
            seen.append(len(reps))
            return _stack(reps)

        got = score_sources(train, test, "cpu", inner_product=_layer_dot, train_blocks_per_pass=4,
                            dense_group=group, cache_budget=CacheBudget(limit_bytes=room))
        assert torch.allclose(got[0], want[0], atol=1e-5) and got[1:4] == want[1:4]
        assert seen == sizes, (room, seen)


def test_budget_capped_groups_fill_whole_score_tiles():
    """A group the budget cuts short is cut to whole 64-row score tiles (or to
    one tile); a group the caller asked for is kept as asked."""
    from types import SimpleNamespace

    from dattri_llm_amd.attribution.utils import group_limit, whole_tile_group
    from dattri_llm_amd.utils.cache import CacheBudget

    assert [whole_tile_group(n, 8) for n in (1, 8, 9, 12, 17, 23, 24, 31)] == [1, 8, 8, 8, 16, 16, 24, 24]
    assert whole_tile_group(30, 3) == 21          # 64 / gcd(3, 64) = 64 blocks per whole tile: one tile
    assert whole_tile_group(5, 100) == 5          # a block taller than a tile
    assert whole_tile_group(7, 16) == 4           # 4 blocks per tile
    block = SimpleNamespace(materialized_nbytes=1000, batch_size=8)
    assert group_limit(block, 32, CacheBudget(limit_bytes=17_500)) == 16
    assert group_limit(block, 12, CacheBudget(limit_bytes=1 << 40)) == 12
    assert group_limit(block, 32, CacheBudget(limit_bytes=500)) == 1
