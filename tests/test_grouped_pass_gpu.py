"""Several train blocks scored in one pass over a dense query block
(score_sources' train_blocks_per_pass): materialize_group writes the linear
layers of every block into row slices of one k-blocked buffer, and the scores
equal the block-by-block loop's (the query side is read once per group)."""

from __future__ import annotations

import pytest
import torch
from conftest import assert_parity, roundings

pytestmark = pytest.mark.gpu


def _block(gen, b, device, t=24):
    from dattri_llm_amd.gradient import Factorized, Gradient

    r = lambda *s: torch.randn(*s, generator=gen).to(torch.bfloat16).to(device)  # noqa: E731
    data = {"up": Factorized(r(b, t, 128), r(b, t, 40)),            # k-blocked (K % 64 == 0)
            "out": Factorized(r(b, t, 40), r(b, t, 64), module_kwargs={"has_bias": True}),  # plain
            "ln": Factorized(r(b, t, 32), r(b, t, 32))}
    lts = {"up": "nn.Linear", "out": "nn.Linear", "ln": "nn.RMSNorm"}
    return Gradient(dict.fromkeys(data, "factorized"), data, lts, dict.fromkeys(data, "batch_token"))


def test_materialize_group_matches_materialize(device):
    from dattri_llm_amd import kernels
    from dattri_llm_amd.gradient import ops

    print("materialize_group: 3 blocks of 2, 3, 1 samples", flush=True)
    gen = torch.Generator().manual_seed(3)
    blocks = [_block(gen, b, device) for b in (2, 3, 1)]
    for name, lt in (("up", "nn.Linear"), ("out", "nn.Linear"), ("ln", "nn.RMSNorm")):
        if name == "out":  # a bias column: the group is concatenated row-major, with a warning
            from dattri_llm_amd.gradient.ops import materialize as mat

            mat._UNBLOCKED_GROUP_WARNED = False  # the warning is given once per process
            with pytest.warns(RuntimeWarning, match="concatenated row-major"):
                got = ops.materialize_group([bl.data[name] for bl in blocks], lt)
        else:
            got = ops.materialize_group([bl.data[name] for bl in blocks], lt)
        want = torch.cat([ops.materialize(bl.data[name], lt) for bl in blocks])
        assert kernels.is_blocked(got) == (name == "up"), name
        assert torch.equal(got.reshape(6, -1), want), name


@pytest.mark.parametrize("normalized", [False, True])
def test_grouped_passes_give_the_block_scores(device, normalized):
    from dattri_llm_amd.attribution import TracInAttributor

    print(f"train_blocks_per_pass=3 over 7 blocks, normalized={normalized}", flush=True)
    gen = torch.Generator().manual_seed(4)
    train = [(s, _block(gen, 4, device), [f"r{s}-{i}" for i in range(4)]) for s in range(7)]
    attr = TracInAttributor(train_batch_size=4, device=device)
    query = attr.route_test_rep(_block(gen, 16, device, t=16))
    assert all(isinstance(v, torch.Tensor) for v in query.data.values())
    test = [(0, query, [f"q{j}" for j in range(16)])]
    one = attr.attribute_sources(train, test, normalized_grad=normalized)
    grouped = attr.attribute_sources(train, test, normalized_grad=normalized, train_blocks_per_pass=3)
    assert grouped.row_train_ids == one.row_train_ids and grouped.row_steps == one.row_steps
    # one bf16 rounding of each score apart at most, should the kernel split its sums differently
    assert_parity(grouped.scores, one.scores, torch.bfloat16, tight=roundings(1))


def test_mixed_group_falls_back_to_row_major(device):
    """A group mixing a dense block with factorized ones cannot be written
    k-blocked: it is concatenated row-major (a plain (B, W) tensor) with the
    same values, and says so once."""
    import importlib
    import warnings

    from dattri_llm_amd import kernels
    from dattri_llm_amd.gradient import ops

    mat = importlib.import_module("dattri_llm_amd.gradient.ops.materialize")  # ops.materialize is the function

    print("materialize_group: dense + factorized blocks", flush=True)
    gen = torch.Generator().manual_seed(5)
    blocks = [_block(gen, b, device) for b in (2, 3)]
    dense_first = ops.materialize(blocks[0].data["up"], "nn.Linear")
    values = [dense_first, blocks[1].data["up"]]
    mat._UNBLOCKED_GROUP_WARNED = False
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        got = ops.materialize_group(values, "nn.Linear")
        ops.materialize_group(values, "nn.Linear")
    assert sum("k-blocked" in str(w.message) for w in caught) == 1
    assert not kernels.is_blocked(got) and got.shape == (5, 40 * 128)
    want = torch.cat([dense_first, ops.materialize(blocks[1].data["up"], "nn.Linear")])
    assert torch.equal(got, want)
