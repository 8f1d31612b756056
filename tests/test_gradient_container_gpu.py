"""The Gradient container's kernel-backed methods on the MI355X (the
reference's tests/gradient/test_gradient.py): materialize, project (LoGRA /
dense, per-layer configs), similarity (dot and cosine, every mode and reduce,
broadcast rows, batch-level layers left out), token-padded concatenation
scoring like its parts, sequence-first captures, and factorized aggregation."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

B, T, D_IN, D_OUT = 2, 4, 8, 16


def _fac(device, b=B, t=None, gen=None):
    shape_a = (b, D_IN) if t is None else (b, t, D_IN)
    shape_g = (b, D_OUT) if t is None else (b, t, D_OUT)
    from dattri_llm_amd.gradient.gradient import Factorized

    return Factorized(torch.randn(*shape_a, generator=gen).to(device), torch.randn(*shape_g, generator=gen).to(device))


def _make(device, layers=("l1", "l2"), rep="factorized", indexing="batch", b=B, seed=0):
    from dattri_llm_amd.gradient.gradient import Gradient

    gen = torch.Generator().manual_seed(seed)
    t = T if indexing == "batch_token" else None
    if rep == "factorized":
        data = {n: _fac(device, b, t, gen) for n in layers}
    else:
        shape = (b, D_OUT * D_IN) if t is None else (b, t, D_OUT * D_IN)
        data = {n: torch.randn(*shape, generator=gen).to(device) for n in layers}
    return Gradient(dict.fromkeys(layers, rep), data, dict.fromkeys(layers, "nn.Linear"),
                    dict.fromkeys(layers, indexing))


def test_materialize(device):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    g = _make(device)
    m = g.materialize()
    for n in m.layer_names:
        assert isinstance(m.data[n], torch.Tensor) and m.representation[n] == "materialized"
        assert m.data[n].shape == (B, D_OUT * D_IN)
    dense = _make(device, rep="materialized")
    assert dense.materialize() is dense
    l2 = torch.randn(B, D_OUT * D_IN, device=device)
    mixed = Gradient({"l1": "factorized", "l2": "materialized"}, {"l1": _fac(device), "l2": l2},
                     {"l1": "nn.Linear", "l2": "nn.Linear"})
    mm = mixed.materialize()
    assert mm.representation == {"l1": "materialized", "l2": "materialized"} and mm.data["l2"] is l2
    assert ops.materialize(Factorized(torch.ones(B, D_IN, device=device), torch.ones(B, D_OUT, device=device)),
                           "nn.Linear").shape == (B, D_OUT * D_IN)
    assert ops.materialize(_fac(device, t=T), "nn.Linear").shape == (B, D_OUT * D_IN)


def test_project(device):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Gradient

    proj = ops.DattriProjector()
    g = _make(device)
    p = g.project(proj, {"__default__": {"style": "logra", "proj_dim": 32, "proj_seed": 0}})
    for n in p.layer_names:
        f = p.data[n]
        assert p.representation[n] == "factorized" and p.layer_types[n] == "nn.Linear"
        assert f.activation.shape[-1] == f.pre_activation_grad.shape[-1] == 32 and f.module_kwargs is None
    p = g.project(proj, {"__default__": {"style": "dense", "proj_dim": 24, "proj_seed": 0}})
    for n in p.layer_names:
        assert p.representation[n] == "materialized" and p.data[n].shape == (B, 24) and p.indexing[n] == "batch"
    data = {"l1": _fac(device), "l2": _fac(device)}
    two = Gradient(dict.fromkeys(data, "factorized"), data, dict.fromkeys(data, "nn.Linear"))
    p = two.project(proj, {"l1": {"style": "logra", "proj_dim": 16}, "l2": {"style": "dense", "proj_dim": 16}})
    assert p.representation == {"l1": "factorized", "l2": "materialized"}
    p = g.project(proj, {})
    assert all(p.data[n] is g.data[n] and p.representation[n] == g.representation[n] for n in g.layer_names)
    p = two.project(proj, {"l1": {"style": "dense", "proj_dim": 8}})
    assert p.representation["l1"] == "materialized" and p.data["l1"].shape == (B, 8) and p.data["l2"] is data["l2"]


def test_similarity_modes_metrics_and_reduce(device):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Gradient

    g = _make(device, indexing="batch_token")
    cross = g.similarity(g, mode="factorized")
    for n, mtx in cross.items():
        assert mtx.shape == (B, B)
        assert torch.allclose(mtx.diagonal(), ops.dot(g.data[n], g.data[n], "nn.Linear"), atol=1e-4, rtol=1e-4)
    mat = g.similarity(g, mode="materialized")
    assert set(cross) == set(mat)
    for n in cross:
        assert torch.allclose(cross[n], mat[n], atol=1e-4, rtol=1e-4)
    other = _make(device, b=5, seed=1)
    assert all(m.shape == (B, 5) for m in _make(device).similarity(other).values())
    assert set(_make(device).similarity(_make(device, layers=("l1",), seed=2))) == {"l1"}
    cos = g.similarity(g, metric="cosine")
    for mtx in cos.values():
        assert torch.allclose(mtx.diagonal(), torch.ones(B, device=device), atol=1e-4, rtol=1e-4)
    h = _make(device, indexing="batch_token", seed=3)
    fc = g.similarity(h, metric="cosine", mode="factorized")
    mc = g.similarity(h, metric="cosine", mode="materialized")
    for n in fc:
        assert (fc[n].abs() <= 1 + 1e-4).all() and torch.allclose(fc[n], mc[n], atol=1e-4, rtol=1e-4)
    per_layer = g.similarity(g, reduce="none")
    overall = g.similarity(g, reduce="all")
    assert isinstance(overall, torch.Tensor) and overall.shape == (B, B)
    assert torch.allclose(overall, torch.stack(list(per_layer.values())).sum(0), atol=1e-4, rtol=1e-4)
    with pytest.raises(ValueError, match="No shared layers"):
        _make(device, layers=("l1",)).similarity(_make(device, layers=("l2",)), reduce="all")
    with pytest.raises(ValueError, match="metric"):
        g.similarity(g, metric="l2")
    with pytest.raises(ValueError, match="reduce"):
        g.similarity(g, reduce="layer")
    with pytest.raises(ValueError, match="mode"):
        g.similarity(g, mode="ghost")
    # batch-level (param_grad) layers are left out of whole-block products
    a, gg = torch.randn(3, 5, 4, device=device), torch.randn(3, 5, 2, device=device)
    from dattri_llm_amd.gradient.gradient import Factorized

    with_norm = Gradient({"lin": "factorized", "norm.weight": "materialized"},
                         {"lin": Factorized(a, gg), "norm.weight": torch.randn(16, device=device)},
                         {"lin": "nn.Linear", "norm.weight": ops.PARAM_GRAD_TYPES})
    only = Gradient({"lin": "factorized"}, {"lin": Factorized(a, gg)}, {"lin": "nn.Linear"})
    torch.testing.assert_close(with_norm.similarity(with_norm, reduce="all"), only.similarity(only, reduce="all"))
    assert "norm.weight" not in ops.layerwise_cross_dot(with_norm, with_norm, reduce="none")


def test_similarity_does_not_materialize_in_factorized_mode(device, monkeypatch):
    from dattri_llm_amd.gradient import ops

    g = _make(device, indexing="batch_token")
    calls = []
    real = ops.materialize
    monkeypatch.setattr(ops, "materialize", lambda *a, **k: calls.append(1) or real(*a, **k))
    g.similarity(g, mode="factorized")
    assert calls == []


def _broadcast(device, b, t=3, d=5, seed=0):
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    g = torch.Generator().manual_seed(seed)
    fc = Factorized(torch.randn(b, t, d, generator=g).to(device), torch.randn(b, t, d, generator=g).to(device))
    pos = Factorized(torch.arange(t).unsqueeze(0).to(device), torch.randn(1, t, d, generator=g).to(device),
                     module_kwargs={"has_bias": False, "num_embeddings": t, "padding_idx": None})
    return Gradient({"fc": "factorized", "pos": "factorized"}, {"fc": fc, "pos": pos},
                    {"fc": "nn.Linear", "pos": "nn.Embedding"}, {"fc": "batch_token", "pos": "batch_token"})


def test_broadcast_rows_in_similarity_and_concatenation(device):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized

    g1, g2 = _broadcast(device, 4, seed=0), _broadcast(device, 2, seed=1)
    total = g1.similarity(g2, metric="dot", reduce="all")
    per = g1.similarity(g2, metric="dot", reduce="none")
    assert total.shape == (4, 2) and per["pos"].shape == (1, 1)
    assert torch.allclose(total, per["fc"] + per["pos"].expand(4, 2), atol=1e-5)
    cos = g1.similarity(g2, metric="cosine", reduce="all")
    assert cos.shape == (4, 2) and bool(torch.isfinite(cos).all()) and float(cos.abs().max()) <= 1 + 1e-5
    # broadcast rows with different ids are averaged as dense gradients
    pos2 = g2.data["pos"]
    g2.data["pos"] = Factorized(torch.flip(pos2.activation, dims=[1]), pos2.pre_activation_grad,
                                module_kwargs=pos2.module_kwargs)
    out = g1.concatenate(g2, dim="batch")
    out.validate()
    assert out.representation["pos"] == "materialized"
    m1 = ops.materialize(g1.data["pos"], "nn.Embedding")
    m2 = ops.materialize(g2.data["pos"], "nn.Embedding")
    assert torch.allclose(out.data["pos"], (4 * m1 + 2 * m2) / 6, atol=1e-6)


def test_padded_concatenation_scores_like_its_parts(device):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    def grad(f):
        return Gradient({"l1": "factorized"}, {"l1": f}, {"l1": "nn.Linear"}, {"l1": "batch_token"})

    for t1, t2 in ((T, T + 3), (T + 5, T)):
        g1, g2 = grad(_fac(device, t=t1)), grad(_fac(device, t=t2))
        m = ops.materialize(g1.concatenate(g2, dim="batch").data["l1"], "nn.Linear")
        assert torch.allclose(m[:B], ops.materialize(g1.data["l1"], "nn.Linear"), atol=1e-6)
        assert torch.allclose(m[B:], ops.materialize(g2.data["l1"], "nn.Linear"), atol=1e-6)
    sf = [grad(Factorized(torch.randn(t, B, D_IN, device=device), torch.randn(t, B, D_OUT, device=device),
                          batch_first=False)) for t in (T, T + 2)]
    m = ops.materialize(sf[0].concatenate(sf[1], dim="batch").data["l1"], "nn.Linear")
    assert torch.allclose(m[:B], ops.materialize(sf[0].data["l1"], "nn.Linear"), atol=1e-6)
    vocab, emb, pad = 11, 5, 7
    mk = {"has_bias": False, "num_embeddings": vocab, "padding_idx": pad}

    def emb_grad(t):
        return Gradient({"e": "factorized"}, {"e": Factorized(torch.randint(0, vocab, (B, t), device=device),
                                                              torch.randn(B, t, emb, device=device), module_kwargs=mk)},
                        {"e": "nn.Embedding"}, {"e": "batch_token"})

    e1, e2 = emb_grad(T), emb_grad(T + 4)
    m = ops.materialize(e1.concatenate(e2, dim="batch").data["e"], "nn.Embedding")
    assert torch.allclose(m[:B], ops.materialize(e1.data["e"], "nn.Embedding"), atol=1e-6)
    assert torch.allclose(m[B:], ops.materialize(e2.data["e"], "nn.Embedding"), atol=1e-6)


def test_sequence_first_matches_batch_first(device):
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    torch.manual_seed(0)
    a, g = torch.randn(B, T, D_IN, device=device), torch.randn(B, T, D_OUT, device=device)
    bf = Gradient({"l": "factorized"}, {"l": Factorized(a, g)}, {"l": "nn.Linear"}, {"l": "batch_token"})
    sf = Gradient({"l": "factorized"}, {"l": Factorized(a.transpose(0, 1), g.transpose(0, 1), batch_first=False)},
                  {"l": "nn.Linear"}, {"l": "batch_token"})
    assert torch.allclose(bf.materialize().data["l"], sf.materialize().data["l"], atol=1e-5)
    assert torch.allclose(bf.similarity(bf)["l"], sf.similarity(sf)["l"], atol=1e-4)
    assert torch.allclose(bf.aggregate().data["l"], sf.aggregate().data["l"], atol=1e-5)
    assert torch.allclose(bf.concatenate(bf, dim="batch").materialize().data["l"],
                          sf.concatenate(sf, dim="batch").materialize().data["l"], atol=1e-5)


def test_factorized_aggregate_promotes_to_materialized(device):
    g = _make(device, indexing="batch_token")
    a = g.aggregate(dim="token")
    for n in a.layer_names:
        assert a.representation[n] == "materialized" and isinstance(a.data[n], torch.Tensor)
