"""CPU tests of the product's host logic: routing rules, data model, score
container, caches and the no-fallback contract.  No kernel runs here."""

from __future__ import annotations

import json
import os

import pytest
import torch

from conftest import REPO


@pytest.fixture
def ops():
    from dattri_llm_amd.gradient import ops

    return ops


def _known():
    with open(os.path.join(REPO, "tests", "golden", "routing_known_answers.json")) as f:
        return json.load(f)


def test_product_cost_rules_match_known_answers(ops):
    k = _known()
    for c in k["maybe_materialize_projected"]:
        assert ops.maybe_materialize_projected(c["seq_len"], c["k_a"], c["k_g"], c["kappa"]) is c["expected"]
    for c in k["should_materialize"]:
        assert ops.should_materialize(c["style"], c["seq_len"], c["k_a"], c["k_g"]) is c["expected"]
    for c in k["maybe_use_materialized_gram"]:
        assert ops.maybe_use_materialized_gram(c["B1"], c["B2"], c["S"], c["K"], c["D"]) is c["expected"]
    with pytest.raises(ValueError, match="capture_style"):
        ops.should_materialize("bogus", 4, 8, 8)


def test_routing_is_looked_up_through_module_globals(ops, monkeypatch):
    """The reference's pin_route patches maybe_use_materialized_gram in the ops
    namespaces and expects cross_gram to see it."""
    import importlib

    dot = importlib.import_module("dattri_llm_amd.gradient.ops.dot")  # the module, not ops.dot()

    calls = []
    monkeypatch.setattr(dot, "maybe_use_materialized_gram", lambda *a, **k: calls.append(a) or True)
    assert dot._route(1, 2, 3, 4, 5) == "materialized"
    assert calls == [(1, 2, 3, 4, 5)]


def test_calibrated_policy(ops):
    from dattri_llm_amd.gradient.ops import cost

    model = cost.calibrated_model()
    assert model.ghost_tflops > 0 and model.stream_gbs > 0
    prev = ops.set_routing_policy("calibrated")
    try:
        # the Llama-3-8B block shapes: every linear materializes
        for k, d in [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]:
            assert ops.maybe_use_materialized_gram(8, 64, 2048, k, d)
        # a single short query against a small batch stays ghost
        assert not ops.maybe_use_materialized_gram(2, 1, 16, 4096, 4096)
        # more tokens can only push toward materializing
        flips = [ops.maybe_use_materialized_gram(8, 8, s, 4096, 4096) for s in (8, 64, 512, 4096)]
        assert flips == sorted(flips)
    finally:
        ops.set_routing_policy(prev)
    with pytest.raises(ValueError):
        ops.set_routing_policy("nope")


def test_kernels_refuse_cpu_tensors(ops):
    from dattri_llm_amd._native import NativeLibraryError

    a = torch.randn(2, 3, 8)
    with pytest.raises(NativeLibraryError, match="ROCm GPU"):
        ops.cross_gram(a, a, a, a, "nn.Linear", mode="factorized")
    with pytest.raises(NativeLibraryError):
        ops.materialize_factors(a, a, "nn.Linear")
    with pytest.raises(NativeLibraryError):
        ops.kfac_factors(a, a, "nn.Linear")
    eye = torch.eye(8)
    with pytest.raises(NativeLibraryError):
        ops.kfac_cross_factors(a, a, a, a, "nn.Linear", eye, eye)


def test_unsupported_layers_raise(ops):
    a = torch.randn(2, 3, 8)
    with pytest.raises(NotImplementedError, match="normalization"):
        ops.kfac_factors(a, a, "nn.LayerNorm")
    with pytest.raises(NotImplementedError):
        ops.kfac_cross_factors(a, a, a, a, "nn.Embedding", torch.eye(8), torch.eye(8))
    with pytest.raises(NotImplementedError):
        ops.preprocess_factors(a, a, "nn.PixelShuffle", {"has_bias": False})
    with pytest.raises(NotImplementedError):
        ops.project_factors(a, a, "nn.PixelShuffle", None, None, proj_dim=4)
    with pytest.raises(ValueError, match="factorized projection is undefined"):
        ops.project_factors(a, a, "nn.LayerNorm", None, None, proj_dim=4)


def test_dtype_policy(ops):
    bf, f32 = torch.zeros(1, dtype=torch.bfloat16), torch.zeros(1)
    assert ops.dtypes.resolve(bf) == torch.bfloat16
    assert ops.dtypes.resolve(bf, f32) == torch.float32
    with ops.compute_dtype("fp32"):
        assert ops.dtypes.resolve(bf) == torch.float32
    assert ops.get_compute_dtype() == "auto"
    with pytest.raises(ValueError):
        ops.set_compute_dtype("int8")


def test_effective_dims(ops):
    from dattri_llm_amd.gradient import Factorized

    f = Factorized(torch.zeros(4, 7, 5), torch.zeros(4, 7, 3), module_kwargs={"has_bias": True})
    assert ops.effective_dims(f, "nn.Linear") == (4, 7, 5, 3)
    f2 = Factorized(torch.zeros(7, 4, 5), torch.zeros(7, 4, 3), batch_first=False)
    assert ops.effective_dims(f2, "nn.Linear") == (4, 7, 5, 3)


def test_gradient_validation_and_batch(ops):
    from dattri_llm_amd.gradient import Factorized, Gradient

    g = Gradient(
        representation={"a": "factorized", "b": "materialized", "pos": "materialized"},
        data={"a": Factorized(torch.zeros(4, 3, 5), torch.zeros(4, 3, 2)), "b": torch.zeros(4, 10),
              "pos": torch.zeros(1, 6)},
        layer_types={"a": "nn.Linear", "b": "nn.Linear", "pos": "nn.Linear"},
        indexing={"a": "batch_token"},
    )
    assert g.batch_size == 4
    assert g.token_dim == {"a": 3, "b": None, "pos": None}
    assert g.materialized_nbytes == 4 * 5 * 2 * 4 + 4 * 10 * 4 + 6 * 4
    with pytest.raises(ValueError, match="same batch size"):
        Gradient({"a": "materialized", "b": "materialized"}, {"a": torch.zeros(3, 2), "b": torch.zeros(4, 2)},
                 {"a": "nn.Linear", "b": "nn.Linear"})
    with pytest.raises(ValueError, match="mismatch"):
        Gradient({"a": "factorized"}, {"a": Factorized(torch.zeros(4, 3, 5), torch.zeros(4, 2, 2))},
                 {"a": "nn.Linear"})
    kept = g.map_layers(lambda n, v, t: None if n == "b" else v)
    assert kept.layer_names == {"a", "pos"}


def test_attribution_score_round_trip(tmp_path):
    from dattri_llm_amd.attribution import AttributionScore

    s = AttributionScore(scores=torch.arange(12.0).view(4, 3), row_train_ids=["x", "y", "x", "z"],
                         row_steps=[0, 0, 1, 1], test_ids=["p", "q", "r"], algorithm="TracIn",
                         algorithm_meta={"normalized_grad": False}, layer_name=None)
    ids, m = s.agnostic_matrix()
    assert ids == ["x", "y", "z"]
    assert torch.equal(m[0], s.scores[0] + s.scores[2])
    assert s.score_at("x", 1, "q") == s.scores[2, 1]
    assert torch.equal(s.query(["z"], ["r", "p"]), torch.tensor([[11.0, 9.0]]))
    assert torch.equal(s.query(trajectory="aware"), s.scores[[0, 2, 1, 3]])
    out = s.save(tmp_path / "sc")
    meta = json.loads((out / "metadata.json").read_text())
    assert meta["num_rows"] == 4 and meta["granularity"] == "instance"
    back = AttributionScore.load(out)
    assert torch.equal(back.scores, s.scores) and back.train_index == s.train_index
    with pytest.raises(ValueError):
        AttributionScore(scores=torch.zeros(2, 2), row_train_ids=["a"], row_steps=[0, 1], test_ids=["p", "q"],
                         algorithm="TracIn", algorithm_meta={}, layer_name=None)


def test_tensor_cache_budget():
    from dattri_llm_amd.utils import CacheBudget, TensorCache

    cache = TensorCache("memory", budget=CacheBudget(limit_bytes=100))
    assert cache.put("a", torch.zeros(10))  # 40 bytes
    assert cache.put("b", torch.zeros(10))
    assert cache.put("c", torch.zeros(10))  # evicts "a"
    assert "a" not in cache and "c" in cache
    assert not cache.put("big", torch.zeros(100))
    calls = []
    assert cache.get_or_compute("b", lambda: calls.append(1)) is not None and not calls


def test_rebatch_blocks_concatenates_dense():
    from dattri_llm_amd.attribution import rebatch_blocks
    from dattri_llm_amd.gradient import Gradient

    def block(v):
        return Gradient({"l": "materialized"}, {"l": torch.full((2, 3), float(v))}, {"l": "nn.Linear"})

    out = list(rebatch_blocks([(0, block(1), ["a", "b"]), (1, block(2), ["c", "d"]), (2, block(3), ["e", "f"])], 4))
    assert [len(ids) for _s, _g, ids in out] == [4, 2]
    steps, big, ids = out[0]
    assert steps == [0, 0, 1, 1] and ids == ["a", "b", "c", "d"]
    assert big.data["l"].shape == (4, 3)


def _query_block(n_test, seed=0, *, s=4, k=8, d=8):
    from dattri_llm_amd.gradient import Factorized, Gradient

    gen = torch.Generator().manual_seed(seed)
    data = {f"l{i}": Factorized(torch.randn(n_test, s, k, generator=gen), torch.randn(n_test, s, d, generator=gen))
            for i in range(2)}
    return Gradient(dict.fromkeys(data, "factorized"), data, dict.fromkeys(data, "nn.Linear"),
                    dict.fromkeys(data, "batch_token"))


def test_query_routing_plan_known_answers():
    """The reference's routing cases (tests/attribution/test_tracin.py:203-235),
    decided from shapes alone: one query stays factorized, sixteen go dense,
    a zero budget keeps them factorized, and a budget that fits one layer
    admits the one with the larger flop saving."""
    from dattri_llm_amd.attribution.routing import plan_query
    from dattri_llm_amd.gradient import Factorized
    from dattri_llm_amd.utils.cache import CacheBudget

    roomy = CacheBudget(limit_bytes=1 << 40)
    assert plan_query(_query_block(1), 8, roomy).dense == []
    assert sorted(plan_query(_query_block(16), 8, roomy).dense) == ["l0", "l1"]
    assert plan_query(_query_block(16, k=16, d=16), 8, CacheBudget(limit_bytes=0)).dense == []
    block = _query_block(16, k=16, d=16)
    block.data["l1"] = Factorized(torch.randn(16, 4, 12), torch.randn(16, 4, 12))
    layer = block.select_layers(["l1"])
    growth = layer.materialized_nbytes - layer.nbytes
    plan = plan_query(block, 8, CacheBudget(limit_bytes=growth))
    assert plan.dense == ["l1"] and plan.held == growth
    assert [r.name for r in plan.routes] == ["l1", "l0"]  # admission order: larger saving first
    assert plan.routes[0].saving > plan.routes[1].saving


def test_query_routing_plan_follows_the_patched_rule(monkeypatch):
    """plan_query looks the cost rule up in the ops namespace, where the
    reference's pin_route patches it."""
    from dattri_llm_amd.attribution.routing import plan_query
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.utils.cache import CacheBudget

    monkeypatch.setattr(ops, "maybe_use_materialized_gram", lambda *a, **k: True)
    assert sorted(plan_query(_query_block(1), 8, CacheBudget(limit_bytes=1 << 40)).dense) == ["l0", "l1"]
    monkeypatch.setattr(ops, "maybe_use_materialized_gram", lambda *a, **k: False)
    assert plan_query(_query_block(16), 8, CacheBudget(limit_bytes=1 << 40)).dense == []


def test_mask_indices_are_a_seeded_sorted_subset():
    """The "mask" style's coordinates: proj_dim distinct, sorted indices into
    the flat width, the same for the same (seed, width, size) on every call
    and device, different for another seed; out-of-range sizes raise."""
    from dattri_llm_amd.gradient import ops

    proj = ops.DattriProjector()
    idx = proj.mask_indices(1000, proj_dim=37, proj_seed=3, device="cpu")
    assert idx.shape == (37,) and torch.equal(idx, idx.sort().values) and idx.unique().numel() == 37
    assert int(idx.min()) >= 0 and int(idx.max()) < 1000
    again = ops.DattriProjector().mask_indices(1000, proj_dim=37, proj_seed=3, device="cpu")
    assert torch.equal(idx, again)
    assert not torch.equal(idx, proj.mask_indices(1000, proj_dim=37, proj_seed=4, device="cpu"))
    with pytest.raises(ValueError, match="0 < proj_dim <= d"):
        proj.mask_indices(10, proj_dim=11, proj_seed=0, device="cpu")
    cfg = {"fc": {"style": "mask", "proj_dim": 37, "proj_seed": 3}, "other": {"style": "logra", "proj_dim": 8}}
    assert torch.equal(ops.mask_coordinates(cfg, "fc", 1000, proj), idx)
    assert ops.mask_coordinates(cfg, "absent", 1000, proj) is None and ops.mask_coordinates(None, "fc", 10, proj) is None
    with pytest.raises(ValueError, match="coordinate-wise"):
        ops.mask_coordinates(cfg, "other", 1000, proj)
    dense = torch.randn(4, 1000)
    assert torch.equal(ops.mask_materialized(dense, proj, proj_dim=37, proj_seed=3), dense[:, idx])
    with pytest.raises(ValueError, match="style 'mask'"):
        ops.mask_materialized(dense, proj, proj_dim=37, proj_seed=3, ensemble=2)


# ---------------------------------------------------------------------------
# embedding preprocessing (host side, no kernels)
# ---------------------------------------------------------------------------


def test_embedding_preprocess_matches_oracle():
    import numpy as np

    import oracle
    from dattri_llm_amd.gradient.ops import embedding as emb
    from dattri_llm_amd.gradient.ops import preprocess_factors
    from dattri_llm_amd.gradient.ops.preprocess import final_embedding

    gen = torch.Generator().manual_seed(3)
    ids = torch.randint(1, 20, (4, 7), generator=gen)
    ids[:, -2:] = 0
    g = torch.randn(4, 7, 5, generator=gen)
    mk = {"has_bias": False, "num_embeddings": 20, "padding_idx": 0}
    a_p, g_p = preprocess_factors(ids, g, "nn.Embedding", mk)
    assert torch.equal(a_p, ids) and torch.equal(g_p[:, -2:], torch.zeros(4, 2, 5))
    assert torch.equal(g_p[:, :-2], g[:, :-2])
    # the kernels' operands: ids -1 at the pads, g untouched
    k_ids, k_g = final_embedding(ids, g, "nn.Embedding", mk)
    assert torch.equal(k_ids[:, -2:], torch.full((4, 2), -1)) and k_g is g
    for mode in ("sum", "mean"):
        for pad in (None, 0):
            bag = torch.randn(4, 5, generator=gen)
            mkb = {"has_bias": False, "num_embeddings": 20, "mode": mode, "padding_idx": pad}
            _, rows = preprocess_factors(ids, bag, "nn.EmbeddingBag", mkb)
            _, ref = oracle.embedding_bag_expand(ids.numpy(), bag.double().numpy(), mode, pad)
            np.testing.assert_allclose(rows.double().numpy(), ref, rtol=1e-6, atol=1e-7)
            k_ids, k_rows = final_embedding(ids, bag, "nn.EmbeddingBag", mkb)
            assert k_rows.stride(1) == 0  # the bag row is spread as a view, not copied
            live = (k_ids >= 0).unsqueeze(-1).numpy()
            np.testing.assert_allclose(np.where(live, k_rows.double().numpy(), 0.0), ref, rtol=1e-6, atol=1e-7)
    with pytest.raises(NotImplementedError, match="max"):
        final_embedding(ids, bag, "nn.EmbeddingBag", dict(mkb, mode="max"))
    emb.check_ids(ids, vocab=20)
    with pytest.raises(ValueError, match="out of range"):
        emb.check_ids(ids, vocab=10)
    with pytest.raises(ValueError, match="negative"):
        emb.check_ids(ids - 5)


# ---------------------------------------------------------------------------
# convolution unfolding (host side, no kernels)
# ---------------------------------------------------------------------------


def test_conv_preprocess_matches_oracle():
    import numpy as np

    import oracle
    from dattri_llm_amd.gradient.ops import conv, preprocess_factors
    from test_oracle import CONV_CASES, conv_inputs

    names = {(False, 1): "nn.Conv1d", (False, 2): "nn.Conv2d", (False, 3): "nn.Conv3d",
             (True, 1): "nn.ConvTranspose1d", (True, 2): "nn.ConvTranspose2d"}
    for case in CONV_CASES:
        transpose, rank, _ci, _co, k, s, p, d, groups, bias, _sp = case
        x, gout = conv_inputs(case)
        mk = {"has_bias": bias, "kernel_size": k, "stride": s, "padding": p, "dilation": d, "groups": groups}
        lt = names[(transpose, rank)]
        a, g = preprocess_factors(torch.from_numpy(x), torch.from_numpy(gout), lt, mk)
        ra, rg = oracle.conv_preprocess(x, gout, transpose, k, s, p, d, groups, bias)
        np.testing.assert_array_equal(a.numpy(), ra)
        np.testing.assert_allclose(g.numpy(), rg, rtol=1e-12, atol=1e-12)  # the bias sums' order differs
        # the kernels' operands: views, the conv bias left implicit
        f = conv.final(torch.from_numpy(x), torch.from_numpy(gout), lt, mk, True)
        assert f.transpose == transpose and f.groups == groups and f.bias == (bias and not transpose)
        if f.bias:
            np.testing.assert_array_equal(f.a.numpy(), ra[..., :-1])
    # 'same' and 'valid' padding strings
    x = torch.randn(2, 3, 9)
    assert conv.unfold_patches(x, 3, 1, "same", 1).shape == (2, 9, 9)
    assert conv.unfold_patches(x, 4, 1, "same", 2).shape == (2, 9, 12)
    assert torch.equal(conv.unfold_patches(x, 3, 1, "valid", 1), conv.unfold_patches(x, 3, 1, 0, 1))


def test_ops_namespace_holds_every_reference_name(ops):
    """Every name of the reference's ops namespace (its ``__all__``) imports
    from ours; the optimizer maps of the out-of-scope attributors raise."""
    names = ["OPTIMIZER_STATE_KEYS", "adam_preconditioner", "adamw_influence_coupling", "adamw_influence_push",
             "adamw_influence_transition", "precondition", "cross_gram", "mask_factors", "project_materialized"]
    for n in names:
        assert hasattr(ops, n) and n in ops.__all__, n
    assert ops.OPTIMIZER_STATE_KEYS["AdamW"] == ("exp_avg", "exp_avg_sq", "max_exp_avg_sq")
    with pytest.raises(NotImplementedError, match="outside"):
        ops.precondition(torch.zeros(2, 3), {}, optimizer_type="Adam", step=1)


def test_locate_rows_identity_and_regroup_on_host():
    """The block's own rows in order take the identity layout without a kernel
    (routing.py:303-304); RowLayout.regroup scatters routed rows back to
    (B, T, ...) with zeros elsewhere (routing.py:71-86)."""
    from dattri_llm_amd.gradient.routing import RowLayout, locate_rows

    x = torch.randn(6, 4)
    lay = locate_rows(x, x.clone(), 2, 3)
    assert lay == RowLayout(2, 3, 6)
    assert torch.equal(lay.regroup(x), x.reshape(2, 3, 4))
    with pytest.raises(ValueError):
        lay.regroup(x[:5])
    with pytest.raises(ValueError):
        locate_rows(x, x[:5], 2, 3)
    sparse = RowLayout(2, 3, 2, torch.tensor([1, 0]), torch.tensor([2, 0]))
    dense = sparse.regroup(torch.tensor([[1.0], [2.0]]))
    want = torch.zeros(2, 3, 1)
    want[1, 2, 0], want[0, 0, 0] = 1.0, 2.0
    assert torch.equal(dense, want)


def test_ghost_probe_cache_follows_tensor_identity_and_version():
    """The live-row probe cache of the factorized route: an entry is found
    through any view of the same tensor, is stale once the tensor is written
    in place, and leaves with the tensor."""
    import gc
    import importlib

    dot = importlib.import_module("dattri_llm_amd.gradient.ops.dot")
    g = torch.randn(3, 4, 5)
    root, sig = dot._probe_key(g[:, :, :])
    assert root is g
    dot._probe_put(root, sig, ["seg", "rows", 7])
    assert dot._probe_get(*dot._probe_key(g[:, :, :])) == ["seg", "rows", 7]
    assert dot._probe_get(*dot._probe_key(g[:2])) is None  # another view: another shape
    g.mul_(2.0)
    assert dot._probe_get(*dot._probe_key(g[:, :, :])) is None
    n = len(dot._PROBES)
    del g, root
    gc.collect()
    assert len(dot._PROBES) == n - 1


def test_ghost_tile_share_and_packed_pricing():
    """The share of the dense ghost engine's 256 x 128-token tiles that holds
    real token pairs decides the packed route; the calibrated cost model
    prices the factorized route at the cheaper of the two kernels."""
    from dattri_llm_amd.gradient.ops import cost

    assert cost.ghost_tile_share(512, 512) == 1.0
    assert cost.ghost_tile_share(256, 128) == 1.0
    assert cost.ghost_tile_share(64, 64) == pytest.approx(0.25 * 0.5)
    assert cost.ghost_tile_share(1, 1) == pytest.approx(1 / (256 * 128))
    assert cost.ghost_tile_share(200, 200) == pytest.approx((200 / 256) ** 2)
    assert cost.ghost_tile_share(2048, 512) == 1.0
    # packed below the relative rate, dense at or above it
    for s1, s2, packed in ((64, 64, True), (128, 128, True), (200, 200, True), (256, 256, False), (512, 512, False),
                           (1000, 1000, False)):
        assert (cost.ghost_tile_share(s1, s2) < cost.PACKED_RELATIVE_RATE) == packed, (s1, s2)
    m = cost.CostModel(ghost_tflops=1000.0, materialize_tflops=1200.0, stream_gbs=6000.0)
    k = d = 4096
    flops = 2.0 * 256 * 64 * 64 * 64 * (k + d)
    assert m.time_factorized(256, 64, 64, 64, k, d) == pytest.approx(
        flops / cost.PACKED_RELATIVE_RATE / 1e15 + m.launch_us * 1e-6)
    dense512 = 2.0 * 8 * 8 * 512 * 512 * (k + d)
    assert m.time_factorized(8, 8, 512, 512, k, d) == pytest.approx(dense512 / 1e15 + m.launch_us * 1e-6)
