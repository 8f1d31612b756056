"""The store's GPU side: PinnedBlockSource delivers exactly the stored blocks
on the device (pinned staging, copy stream), scoring straight from two stores
equals scoring the same blocks held in memory, and the background writer
takes device-resident groups."""

from __future__ import annotations

import torch
import pytest

from dattri_llm_amd.gradient.gradient import Factorized, Gradient, GradientRecord
from dattri_llm_amd.gradient.store import AsyncGradientWriter, GradientStore, PinnedBlockSource, records_to_block

pytestmark = pytest.mark.gpu


def _record(step, i, seed, n=3, t=24, k=32, d=40, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    g = Gradient({"mlp": "factorized", "proj": "materialized"},
                 {"mlp": Factorized((torch.randn(n, t, k, generator=gen) / k**0.5).to(dtype),
                                    (torch.randn(n, t, d, generator=gen) / d**0.5).to(dtype),
                                    module_kwargs={"has_bias": True}),
                  "proj": (torch.randn(n, 64, generator=gen) / 8).to(dtype)},
                 {"mlp": "nn.Linear", "proj": "nn.Linear"})
    return GradientRecord(step, [f"{seed}-{i}-{j}" for j in range(n)], g)


def _fill(root, n_groups, per_group, seed0):
    store = GradientStore(root)
    for gi in range(n_groups):
        store.save_bulk([_record(gi % 2, i, seed0 + 10 * gi + i) for i in range(per_group)])
    return store


def test_pinned_source_delivers_the_stored_blocks(device, tmp_path):
    store = _fill(tmp_path / "train", 4, 2, 100)
    src = PinnedBlockSource(store, device=device, prefetch=2)
    assert len(src) == 4
    got = list(src)
    for (step, block, hashes), (file_rel, by_step) in zip(got, store.iter_steps(store.available_steps())):
        ((want_step, idxs),) = by_step.items()
        want, want_hashes = records_to_block(store.load_records(file_rel), idxs)
        assert step == want_step and hashes == want_hashes
        assert block.device.type == "cuda"
        assert torch.equal(block.data["proj"].cpu(), want.data["proj"])
        assert torch.equal(block.data["mlp"].activation.cpu(), want.data["mlp"].activation)
        assert torch.equal(block.data["mlp"].pre_activation_grad.cpu(), want.data["mlp"].pre_activation_grad)
    assert src.h2d_bytes == sum(b.nbytes for _s, b, _h in got)
    only = PinnedBlockSource(store, device=device, steps=[1], layer_name="proj")
    assert [s for s, _b, _h in only] == [1, 1] and all(set(b.data) == {"proj"} for _s, b, _h in only)
    with pytest.raises(ValueError, match="requested steps"):
        PinnedBlockSource(store, device=device, steps=[9])


def test_scores_from_stores_equal_in_memory(device, tmp_path):
    from dattri_llm_amd.attribution import TracInAttributor

    train = _fill(tmp_path / "train", 3, 2, 200)
    test = _fill(tmp_path / "test", 1, 2, 300)

    def memory(store):
        out = []
        for file_rel, by_step in store.iter_steps(store.available_steps()):
            recs = store.load_records(file_rel)
            for step, idxs in by_step.items():
                block, hashes = records_to_block(recs, idxs)
                out.append((step, block.to(device), hashes))
        return out

    attr = TracInAttributor(train_batch_size=4, device=device)
    ref = attr.attribute_sources(memory(train), memory(test))
    got = TracInAttributor(train_batch_size=4, device=device).attribute_sources(
        PinnedBlockSource(train, device=device), PinnedBlockSource(test, device=device))
    assert got.row_train_ids == ref.row_train_ids and got.test_ids == ref.test_ids
    assert torch.equal(got.scores, ref.scores)


def test_async_writer_from_device(device, tmp_path):
    store = GradientStore(tmp_path)
    recs = [_record(5, i, 400 + i) for i in range(3)]
    dev_recs = [GradientRecord(r.step, r.input_hash, r.gradient.to(device)) for r in recs]
    with AsyncGradientWriter(store) as w:
        w.submit(dev_recs[:2])
        w.submit(dev_recs[2:])
    back = GradientStore(tmp_path)
    loaded = back.load_records("batch_000000.mmap") + back.load_records("batch_000001.mmap")
    for a, b in zip(loaded, recs):
        assert torch.equal(a.gradient.data["proj"], b.gradient.data["proj"])
        assert torch.equal(a.gradient.data["mlp"].activation, b.gradient.data["mlp"].activation)


@pytest.mark.parametrize("normalized", [False, True])
def test_attribute_from_cache_equals_attribute_sources(device, tmp_path, normalized):
    """The store-then-attribute entry point on two store directories gives the
    scores, rows and columns of attribute_sources over block sources of the
    same stores."""
    from dattri_llm_amd.attribution import TracInAttributor

    print(f"attribute_from_cache vs attribute_sources, normalized={normalized}", flush=True)
    train = _fill(tmp_path / "train", 3, 2, 500)
    test = _fill(tmp_path / "test", 1, 2, 600)
    ref = TracInAttributor(train_batch_size=4, device=device).attribute_sources(
        PinnedBlockSource(train, device=device), PinnedBlockSource(test, device=device), normalized_grad=normalized)
    got = TracInAttributor(train_batch_size=4, device=device).attribute_from_cache(
        tmp_path / "train", str(tmp_path / "test"), normalized_grad=normalized)
    assert got.row_train_ids == ref.row_train_ids and got.row_steps == ref.row_steps
    assert got.test_ids == ref.test_ids and torch.equal(got.scores, ref.scores)
    assert got.algorithm == ("GradCos" if normalized else "TracIn")
    assert got.algorithm_meta["selected_training_steps"] == train.available_steps()
    one_step = TracInAttributor(train_batch_size=4, device=device).attribute_from_cache(
        train, test, selected_training_steps=[1], layer_name="proj", normalized_grad=normalized)
    ref1 = TracInAttributor(train_batch_size=4, device=device).attribute_sources(
        PinnedBlockSource(train, device=device, steps=[1], layer_name="proj"),
        PinnedBlockSource(test, device=device, layer_name="proj"), normalized_grad=normalized)
    assert one_step.row_train_ids == ref1.row_train_ids and torch.equal(one_step.scores, ref1.scores)
    assert set(one_step.row_steps) == {1} and one_step.layer_name == ["proj"]
