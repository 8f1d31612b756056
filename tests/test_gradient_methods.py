"""CPU tests of the Gradient block methods that only reshape payloads
(concatenate, slice, aggregate of dense layers): the contract of
dattri_llm/gradient/gradient.py:698-961, checked by construction -- a batch
join followed by slicing each part back returns the parts (with the zero-grad
padding the join adds), token joins split back along the token axis, and a
dense batch_token layer aggregates to its token sum."""

from __future__ import annotations

import pytest
import torch


def _block(b, t, seed, *, shared=False):
    from dattri_llm_amd.gradient import Factorized, Gradient

    gen = torch.Generator().manual_seed(seed)
    a = torch.randn(b, t, 6, generator=gen)
    g = torch.randn(b, t, 5, generator=gen)
    dense_tok = torch.randn(b, t, 4, generator=gen)
    dense = torch.randn(1 if shared else b, 7, generator=gen)
    ids = torch.randint(0, 50, (b, t), generator=gen)
    emb_g = torch.randn(b, t, 3, generator=gen)
    data = {
        "lin": Factorized(a, g, module_kwargs={"has_bias": False}),
        "tok": dense_tok,
        "vec": dense,
        "emb": Factorized(ids, emb_g, module_kwargs={"padding_idx": 1}),
    }
    rep = {"lin": "factorized", "tok": "materialized", "vec": "materialized", "emb": "factorized"}
    types = {"lin": "nn.Linear", "tok": "nn.Linear", "vec": "nn.Linear", "emb": "nn.Embedding"}
    index = {"lin": "batch_token", "tok": "batch_token", "vec": "batch", "emb": "batch_token"}
    return Gradient(rep, data, types, index)


def test_batch_concatenation_pads_tokens_and_slices_back():
    x, y = _block(3, 5, 0), _block(2, 8, 1)
    z = x.concatenate(y, dim="batch")
    assert z.batch_size == 5 and z.token_dim["lin"] == 8
    back = z.slice("batch", [0, 1, 2])
    lin = back.data["lin"]
    assert torch.equal(lin.activation[:, :5], x.data["lin"].activation)
    assert torch.equal(lin.pre_activation_grad[:, :5], x.data["lin"].pre_activation_grad)
    # the added positions carry zero output gradients (inert downstream)
    assert torch.count_nonzero(lin.pre_activation_grad[:, 5:]) == 0
    assert torch.count_nonzero(back.data["tok"][:, 5:]) == 0
    # integer activations (token ids) are padded with the layer's padding_idx
    assert torch.all(back.data["emb"].activation[:, 5:] == 1)
    other = z.slice("batch", torch.tensor([3, 4]))
    assert torch.equal(other.data["lin"].activation, y.data["lin"].activation)
    assert torch.equal(other.data["vec"], y.data["vec"])


def test_token_concatenation_splits_back():
    x, y = _block(3, 5, 2), _block(3, 4, 3)
    x = x.select_layers(["lin", "tok", "emb"])
    y = y.select_layers(["lin", "tok", "emb"])
    z = x.concatenate(y, dim="token")
    assert z.token_dim["lin"] == 9
    assert torch.equal(z.slice("token", list(range(5))).data["tok"], x.data["tok"])
    assert torch.equal(z.slice("token", list(range(5, 9))).data["lin"].pre_activation_grad,
                      y.data["lin"].pre_activation_grad)
    with pytest.raises(ValueError, match="batch_token"):
        _block(3, 5, 2).concatenate(_block(3, 4, 3), dim="token")
    with pytest.raises(ValueError, match="same batch size"):
        x.concatenate(_block(2, 4, 3).select_layers(["lin", "tok", "emb"]), dim="token")


def test_int_index_keeps_the_axis_and_broadcast_rows_serve_every_sample():
    x = _block(4, 5, 4, shared=True)
    one = x.slice("batch", 2)
    assert one.data["lin"].activation.shape == (1, 5, 6)
    assert torch.equal(one.data["lin"].activation[0], x.data["lin"].activation[2])
    picked = x.slice("batch", [3, 0, 1])
    assert picked.data["vec"].shape == (3, 7)
    assert torch.equal(picked.data["vec"], x.data["vec"].expand(3, 7))


def test_shared_rows_merge_by_sample_count():
    x, y = _block(4, 5, 5, shared=True), _block(2, 5, 6, shared=True)
    z = x.concatenate(y, dim="batch")
    assert z.data["vec"].shape == (1, 7)
    assert torch.allclose(z.data["vec"], (4 * x.data["vec"] + 2 * y.data["vec"]) / 6)
    with pytest.raises(ValueError, match="broadcast"):
        x.concatenate(_block(2, 5, 6), dim="batch")


def test_aggregate_sums_dense_token_layers_and_rejects_other_axes():
    x = _block(3, 5, 7).select_layers(["tok", "vec"])
    agg = x.aggregate()
    assert agg.indexing == {"tok": "batch", "vec": "batch"}
    assert torch.allclose(agg.data["tok"], x.data["tok"].sum(1))
    assert agg.data["vec"] is x.data["vec"]
    with pytest.raises(NotImplementedError):
        x.aggregate(dim="batch")


def test_incompatible_blocks_are_rejected():
    x = _block(3, 5, 8)
    y = _block(3, 5, 9).select_layers(["lin", "tok", "vec"])
    with pytest.raises(ValueError, match="Layer sets differ"):
        x.concatenate(y)
