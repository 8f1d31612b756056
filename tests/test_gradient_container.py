"""The Gradient container's host logic on the CPU (the reference's
tests/gradient/test_gradient.py): validation, properties, clone / to,
map_layers, select_layers, concatenation (batch, token, variable lengths,
broadcast rows), aggregation of dense layers, slicing, sequence-first
captures and the batch-mismatch message.  The parts that run kernels are in
tests/test_gradient_container_gpu.py."""

from __future__ import annotations

import pytest
import torch

from dattri_llm_amd.gradient import ops
from dattri_llm_amd.gradient.gradient import Factorized, Gradient, base_layer_name

B, T, D_IN, D_OUT = 2, 4, 8, 16


def mat(b=B, feat=D_OUT * D_IN):
    return torch.randn(b, feat)


def mat_bt(b=B, t=T, feat=D_OUT * D_IN):
    return torch.randn(b, t, feat)


def fac(b=B):
    return Factorized(torch.randn(b, D_IN), torch.randn(b, D_OUT))


def fac_bt(b=B, t=T):
    return Factorized(torch.randn(b, t, D_IN), torch.randn(b, t, D_OUT))


def make(layers=("l1", "l2"), rep="materialized", indexing="batch", layer_type="nn.Linear"):
    if rep == "factorized":
        data = {n: (fac_bt() if indexing == "batch_token" else fac()) for n in layers}
    else:
        data = {n: (mat_bt() if indexing == "batch_token" else mat()) for n in layers}
    return Gradient(dict.fromkeys(layers, rep), data, dict.fromkeys(layers, layer_type),
                    dict.fromkeys(layers, indexing))


# -- validate (test_gradient.py:106-206) --------------------------------------------------------


def test_valid_blocks():
    make().validate()
    make(rep="factorized").validate()
    make(indexing="batch_token").validate()


def test_validation_errors():
    with pytest.raises(ValueError, match="empty"):
        Gradient({}, {}, {}).validate()
    with pytest.raises(ValueError, match="Missing representation"):
        Gradient({"l1": "materialized"}, {"l1": mat(), "l2": mat()}, {"l1": "nn.Linear", "l2": "nn.Linear"})
    with pytest.raises(TypeError, match="Factorized"):
        Gradient({"l1": "factorized"}, {"l1": mat()}, {"l1": "nn.Linear"})
    with pytest.raises(TypeError, match="Tensor"):
        Gradient({"l1": "materialized"}, {"l1": fac()}, {"l1": "nn.Linear"})
    with pytest.raises(ValueError, match="batch size"):
        Gradient(dict.fromkeys(("l1", "l2"), "materialized"), {"l1": mat(b=2), "l2": mat(b=3)},
                 dict.fromkeys(("l1", "l2"), "nn.Linear"))
    with pytest.raises(ValueError, match="batch_token"):
        Gradient({"l1": "materialized"}, {"l1": mat()}, {"l1": "nn.Linear"}, {"l1": "batch_token"})


def _emb(b, t=T, d=D_OUT):
    return Factorized(torch.randint(0, t, (b, t)), torch.randn(b, t, d))


def test_broadcast_layers_do_not_set_the_batch():
    for order in (("wte", "wpe"), ("wpe", "wte")):
        data = {"wte": _emb(3), "wpe": _emb(1)}
        g = Gradient(dict.fromkeys(order, "factorized"), {n: data[n] for n in order},
                     dict.fromkeys(order, "nn.Embedding"), dict.fromkeys(order, "batch_token"))
        assert g.batch_size == 3
    with pytest.raises(ValueError, match="same batch size"):
        Gradient(dict.fromkeys("ab", "factorized"), {"a": _emb(2), "b": _emb(3)}, dict.fromkeys("ab", "nn.Embedding"),
                 dict.fromkeys("ab", "batch_token"))


def test_batch_mismatch_message_names_layers_and_shapes():
    a = Factorized(torch.randn(2, 5, 4), torch.randn(2, 5, 3))
    b = Factorized(torch.randn(7, 4), torch.randn(7, 3))
    with pytest.raises(ValueError, match="same batch size") as exc:
        Gradient({"attn": "factorized", "experts.2": "factorized"}, {"attn": a, "experts.2": b},
                 {"attn": "nn.Linear", "experts.2": "nn.Linear"})
    msg = str(exc.value)
    assert "attn has 2 samples (captured shape (2, 5, 4))" in msg
    assert "experts.2 has 7 (captured shape (7, 4))" in msg


# -- properties, clone, to (test_gradient.py:209-303) -------------------------------------------


def test_properties():
    g = make(layers=("l1", "l2", "l3"))
    assert g.layer_names == {"l1", "l2", "l3"}
    assert make().batch_size == B and make(rep="factorized").batch_size == B
    assert make(indexing="batch_token").token_dim == {"l1": T, "l2": T}
    assert make().token_dim == {"l1": None, "l2": None}
    mixed = Gradient(dict.fromkeys(("l1", "l2"), "materialized"), {"l1": mat_bt(), "l2": mat()},
                     dict.fromkeys(("l1", "l2"), "nn.Linear"), {"l1": "batch_token", "l2": "batch"})
    assert mixed.token_dim == {"l1": T, "l2": None}
    assert make().device == torch.device("cpu") and make().dtype == torch.float32


def test_clone_is_independent():
    g = make()
    c = g.clone()
    for n in g.layer_names:
        g.data[n].fill_(0)
        assert not torch.allclose(g.data[n], c.data[n])
    assert c.representation == g.representation and c.representation is not g.representation
    g = make(rep="factorized")
    c = g.clone()
    for n in g.layer_names:
        g.data[n].activation.fill_(0)
        assert not torch.allclose(g.data[n].activation, c.data[n].activation)


def test_to_dtype():
    assert all(v.dtype == torch.float64 for v in make().to(dtype=torch.float64).data.values())
    for v in make(rep="factorized").to(dtype=torch.float64).data.values():
        assert v.activation.dtype == v.pre_activation_grad.dtype == torch.float64
    g = make()
    assert g.to(dtype=torch.float16).representation == g.representation
    f = fac().to(dtype=torch.float64)
    assert f.activation.dtype == f.pre_activation_grad.dtype == torch.float64


# -- map_layers, select_layers (test_gradient.py:311-486) ---------------------------------------


def test_map_layers_consume_and_default():
    g = make(rep="factorized")
    names = sorted(g.layer_names)
    keep, convert = names[0], names[1:]

    def dense(_n, v, _t):
        return torch.einsum("bi,bo->boi", v.activation, v.pre_activation_grad).flatten(1)

    expected = {n: dense(n, g.data[n], "nn.Linear") for n in convert}
    out = g.map_layers(dense, layers=convert, consume=True)
    assert set(g.data) == {keep} and isinstance(g.data[keep], Factorized)
    assert set(out.data) == set(names) and isinstance(out.data[keep], Factorized)
    for n in convert:
        assert out.representation[n] == "materialized" and torch.equal(out.data[n], expected[n])
    g = make(rep="factorized")
    before = dict(g.data)
    g.map_layers(dense)
    assert g.data == before


def test_select_layers():
    g = make(layers=("l1", "l2", "l3"))
    s = g.select_layers(["l1", "l3"])
    assert s.layer_names == {"l1", "l3"} and set(s.representation) == {"l1", "l3"}
    typed = Gradient(g.representation, g.data, dict.fromkeys(g.data, "Linear"), g.indexing)
    assert typed.select_layers(["l1"]).layer_types == {"l1": "Linear"}
    with pytest.raises(KeyError, match="Unknown layers"):
        g.select_layers(["l99"])
    g = make(layers=("l1", "l1@2", "l1@3", "l2"))
    assert g.select_layers(["l1"]).layer_names == {"l1"}
    assert g.select_layers(["l1"], include_derived=True).layer_names == {"l1", "l1@2", "l1@3"}
    assert g.select_layers(["l2"], include_derived=True).layer_names == {"l2"}
    assert base_layer_name("l1@2") == "l1" and base_layer_name("mlp.up") == "mlp.up"


# -- concatenate (test_gradient.py:489-662, :840-911) -------------------------------------------


def test_concatenate_batch_and_token():
    c = make().concatenate(make(), dim="batch")
    assert c.batch_size == 2 * B and all(v.shape[0] == 2 * B for v in c.data.values())
    c = make(indexing="batch_token").concatenate(make(indexing="batch_token"), dim="token")
    assert c.token_dim == {"l1": 2 * T, "l2": 2 * T}
    with pytest.raises(ValueError, match="batch_token"):
        make().concatenate(make(), dim="token")
    other = Gradient(dict.fromkeys(("l1", "l2"), "materialized"), {"l1": mat_bt(b=3), "l2": mat_bt(b=3)},
                     dict.fromkeys(("l1", "l2"), "nn.Linear"), dict.fromkeys(("l1", "l2"), "batch_token"))
    with pytest.raises(ValueError, match="batch size"):
        make(indexing="batch_token").concatenate(other, dim="token")
    mixed = Gradient(dict.fromkeys(("l1", "l2"), "materialized"), {"l1": mat_bt(), "l2": mat()},
                     dict.fromkeys(("l1", "l2"), "nn.Linear"), {"l1": "batch_token", "l2": "batch"})
    with pytest.raises(ValueError, match="batch_token"):
        mixed.concatenate(mixed, dim="token")
    with pytest.raises(ValueError, match="representation"):
        make(rep="materialized").concatenate(make(rep="factorized"))


def test_variable_length_batch_concatenate_pads_inert_rows():
    def grad(f):
        return Gradient({"l1": "factorized"}, {"l1": f}, {"l1": "nn.Linear"}, {"l1": "batch_token"})

    g1, g2 = grad(fac_bt(t=T)), grad(fac_bt(t=T + 3))
    c = g1.concatenate(g2, dim="batch")
    assert c.batch_size == 2 * B and c.token_dim == {"l1": T + 3}
    f = c.data["l1"]
    assert torch.equal(f.activation[:B, :T], g1.data["l1"].activation)
    assert (f.pre_activation_grad[:B, T:] == 0).all()  # padded rows carry no gradient
    c = grad(fac_bt(t=T + 5)).concatenate(grad(fac_bt(t=T)), dim="batch")
    assert c.token_dim == {"l1": T + 5}
    dense = [Gradient({"l1": "materialized"}, {"l1": mat_bt(t=t)}, {"l1": "nn.Linear"}, {"l1": "batch_token"})
             for t in (T, T + 2)]
    v = dense[0].concatenate(dense[1], dim="batch").data["l1"]
    assert v.shape == (2 * B, T + 2, D_OUT * D_IN) and (v[:B, T:] == 0).all()
    with pytest.raises(RuntimeError):
        make(layers=("l1",), rep="factorized").concatenate(
            Gradient({"l1": "factorized"}, {"l1": Factorized(torch.randn(B, D_IN + 1), torch.randn(B, D_OUT))},
                     {"l1": "nn.Linear"}, {"l1": "batch"}), dim="batch")
    with pytest.raises(ValueError, match="representation"):
        Gradient({"l1": "materialized"}, {"l1": mat()}, {"l1": "nn.Linear"}).concatenate(
            Gradient({"l1": "factorized"}, {"l1": fac()}, {"l1": "nn.Linear"}))


def test_variable_length_embedding_pads_with_padding_idx():
    vocab, emb, pad = 11, 5, 7
    mk = {"has_bias": False, "num_embeddings": vocab, "padding_idx": pad}

    def grad(t):
        return Gradient({"e": "factorized"}, {"e": Factorized(torch.randint(0, vocab, (B, t)),
                                                              torch.randn(B, t, emb), module_kwargs=mk)},
                        {"e": "nn.Embedding"}, {"e": "batch_token"})

    f = grad(T).concatenate(grad(T + 4), dim="batch").data["e"]
    assert (f.activation[:B, T:] == pad).all() and (f.pre_activation_grad[:B, T:] == 0).all()


def _broadcast(b, t=3, d=5, seed=0):
    g = torch.Generator().manual_seed(seed)
    fc = Factorized(torch.randn(b, t, d, generator=g), torch.randn(b, t, d, generator=g))
    pos = Factorized(torch.arange(t).unsqueeze(0), torch.randn(1, t, d, generator=g),
                     module_kwargs={"has_bias": False, "num_embeddings": t, "padding_idx": None})
    return Gradient({"fc": "factorized", "pos": "factorized"}, {"fc": fc, "pos": pos},
                    {"fc": "nn.Linear", "pos": "nn.Embedding"}, {"fc": "batch_token", "pos": "batch_token"})


def test_broadcast_rows_under_batch_concatenation():
    g1, g2 = _broadcast(4, seed=0), _broadcast(2, seed=1)
    out = g1.concatenate(g2, dim="batch")
    out.validate()
    assert out.batch_size == 6 and out.data["fc"].activation.shape[0] == 6
    assert out.representation["pos"] == "factorized"
    want = (4 * g1.data["pos"].pre_activation_grad + 2 * g2.data["pos"].pre_activation_grad) / 6
    assert torch.allclose(out.data["pos"].pre_activation_grad, want)
    assert torch.equal(out.data["pos"].activation, g1.data["pos"].activation)
    r1, r2 = torch.randn(1, 7), torch.randn(1, 7)

    def dense(b, row):
        return Gradient({"fc": "materialized", "pos": "materialized"}, {"fc": torch.randn(b, 7), "pos": row},
                        {"fc": "nn.Linear", "pos": "nn.Embedding"})

    out = dense(3, r1).concatenate(dense(5, r2), dim="batch")
    assert torch.allclose(out.data["pos"], (3 * r1 + 5 * r2) / 8) and out.data["fc"].shape[0] == 8
    g2 = _broadcast(2, seed=1)
    g2.data["pos"] = Factorized(torch.arange(3).repeat(2, 1), torch.randn(2, 3, 5))
    with pytest.raises(ValueError, match="broadcast"):
        g1.concatenate(g2, dim="batch")
    out = _broadcast(1, seed=0).concatenate(_broadcast(1, seed=1), dim="batch")
    assert out.batch_size == 2 and out.data["pos"].activation.shape[0] == 2


# -- aggregate, slice (test_gradient.py:670-837) ------------------------------------------------


def test_aggregate_dense_layers():
    g = make(indexing="batch_token")
    a = g.aggregate(dim="token")
    assert all(v == "batch" for v in a.indexing.values())
    for n in g.layer_names:
        assert a.data[n].shape == (B, D_OUT * D_IN) and torch.allclose(a.data[n], g.data[n].sum(dim=1))
    mixed = Gradient(dict.fromkeys(("l1", "l2"), "materialized"), {"l1": mat_bt(), "l2": mat()},
                     dict.fromkeys(("l1", "l2"), "nn.Linear"), {"l1": "batch_token", "l2": "batch"})
    a = mixed.aggregate(dim="token")
    assert a.data["l1"].shape == a.data["l2"].shape == (B, D_OUT * D_IN)
    g = make()
    assert all(torch.equal(g.aggregate(dim="token").data[n], g.data[n]) for n in g.layer_names)
    with pytest.raises(NotImplementedError):
        make(indexing="batch_token").aggregate(dim="batch")
    with pytest.raises(TypeError):
        make(indexing="batch_token").aggregate(dim="token", mode="mean")


def test_slice():
    g = make()
    assert g.slice(dim="batch", index=0).batch_size == 1
    assert g.slice(dim="batch", index=slice(0, 1)).batch_size == 1
    assert g.slice(dim="batch", index=0).representation == g.representation
    assert make(indexing="batch_token").slice(dim="token", index=0).token_dim == {"l1": 1, "l2": 1}
    mixed = Gradient(dict.fromkeys(("l1", "l2"), "materialized"), {"l1": mat_bt(), "l2": mat()},
                     dict.fromkeys(("l1", "l2"), "nn.Linear"), {"l1": "batch_token", "l2": "batch"})
    with pytest.raises(ValueError, match="batch_token"):
        mixed.slice(dim="token", index=0)
    for v in make(rep="factorized").slice(dim="batch", index=0).data.values():
        assert isinstance(v, Factorized) and v.activation.shape[0] == 1


def test_batch_slice_copies_broadcast_rows_and_keeps_param_grads():
    n, t, d = 4, 3, 5
    fc = Factorized(torch.randn(n, t, d), torch.randn(n, t, d))
    pos = Factorized(torch.arange(t).unsqueeze(0), torch.randn(1, t, d))
    g = Gradient({"fc": "factorized", "pos": "factorized"}, {"fc": fc, "pos": pos},
                 {"fc": "nn.Linear", "pos": "nn.Embedding"}, {"fc": "batch_token", "pos": "batch_token"})
    for i in range(n):
        s = g.slice(dim="batch", index=i)
        assert torch.equal(s.data["fc"].activation[0], fc.activation[i])
        assert torch.equal(s.data["pos"].pre_activation_grad[0], pos.pre_activation_grad[0])
    s = g.slice(dim="batch", index=[1, 3])
    assert s.data["fc"].activation.shape[0] == s.data["pos"].activation.shape[0] == 2
    assert torch.equal(s.data["pos"].activation[0], s.data["pos"].activation[1])
    pg = torch.randn(7, 3)
    g = Gradient({"sample": "materialized", "weight": "materialized"}, {"sample": torch.randn(B, 5), "weight": pg},
                 {"sample": "nn.Linear", "weight": ops.PARAM_GRAD_TYPES}, {"sample": "batch", "weight": "batch"})
    s = g.slice(dim="batch", index=0)
    assert s.data["sample"].shape[0] == 1 and torch.equal(s.data["weight"], pg)


# -- sequence-first captures (test_gradient.py:1084-1210) ---------------------------------------


def _seq_first_pair():
    torch.manual_seed(0)
    a, g = torch.randn(B, T, D_IN), torch.randn(B, T, D_OUT)
    bf = Gradient({"l": "factorized"}, {"l": Factorized(a, g)}, {"l": "nn.Linear"}, {"l": "batch_token"})
    sf = Gradient({"l": "factorized"}, {"l": Factorized(a.transpose(0, 1), g.transpose(0, 1), batch_first=False)},
                  {"l": "nn.Linear"}, {"l": "batch_token"})
    return bf, sf


def test_sequence_first_host_logic():
    assert Factorized(torch.randn(B, D_IN), torch.randn(B, D_OUT)).batch_first is True
    f = Factorized(torch.randn(B, T, D_IN), torch.randn(B, T, D_OUT))
    assert f.as_batch_first() is f
    f = Factorized(torch.randn(T, B, D_IN), torch.randn(T, B, D_OUT), batch_first=False)
    bf = f.as_batch_first()
    assert bf.batch_first and bf.activation.shape == (B, T, D_IN) and bf.pre_activation_grad.shape == (B, T, D_OUT)
    _bf, sf = _seq_first_pair()
    sf.validate()
    assert sf.batch_size == B and sf.token_dim["l"] == T
    a, g = torch.randn(B, T, D_IN), torch.randn(B, T, D_OUT)
    both = Gradient({"bf": "factorized", "sf": "factorized"},
                    {"bf": Factorized(a, g), "sf": Factorized(a.transpose(0, 1), g.transpose(0, 1), batch_first=False)},
                    {"bf": "nn.Linear", "sf": "nn.Linear"}, {"bf": "batch_token", "sf": "batch_token"})
    both.validate()
    assert both.batch_size == B
    assert sf.clone().data["l"].batch_first is False
    assert sf.to(dtype=torch.float64).data["l"].batch_first is False
    sl = sf.slice("batch", 0)
    assert sl.data["l"].batch_first is False and sl.batch_size == 1 and sl.data["l"].activation.shape == (T, 1, D_IN)
    bf, sf = _seq_first_pair()
    assert sf.concatenate(sf, dim="batch").batch_size == 2 * B
    with pytest.raises(ValueError, match="batch_first"):
        bf.concatenate(sf, dim="batch")
