"""The reference's op-contract tests (tests/gradient/test_ops.py:340-524,
:778-1080) on the MI355X path, at its shapes (B=4, T=6, D_IN=8, D_OUT=12) and
tolerances: K-FAC / Fisher shapes (linear and convolution layers), the
norm / embedding refusals and the gradient-free rows (dropped for sequence
layers, kept for convolutions), streaming accumulators equal one-shot K-FAC / Fisher factors,
token collapse of norm gradients, the multi-layer accumulators and the
Fisher size cap, the Factorized wrappers (and sequence-first captures), the
damped inverses, per-token cross-grams summing to the full one, the outer
product against its einsum, and ProjectionMatrix.matches."""

from __future__ import annotations

import types

import pytest
import torch

pytestmark = pytest.mark.gpu

B, T, D_IN, D_OUT, VOCAB, E = 4, 6, 8, 12, 32, 10


@pytest.fixture
def gen():
    return torch.Generator().manual_seed(0)


def _on(device, *ts):
    return tuple(t.to(device) for t in ts)


def _linear_2d(gen, device):
    return _on(device, torch.randn(B, D_IN, generator=gen), torch.randn(B, D_OUT, generator=gen))


def _linear_3d(gen, device):
    return _on(device, torch.randn(B, T, D_IN, generator=gen), torch.randn(B, T, D_OUT, generator=gen))


def _norm_3d(gen, device):
    return _on(device, torch.randn(B, T, D_IN, generator=gen), torch.randn(B, T, D_IN, generator=gen))


def _embedding(gen, device):
    return _on(device, torch.randint(0, VOCAB, (B, T), generator=gen), torch.randn(B, T, E, generator=gen))


def _block(layers):
    """name -> (layer_type, a, g), as the reference's _fake_gradient."""
    from dattri_llm_amd.gradient.gradient import Factorized

    return types.SimpleNamespace(data={n: Factorized(a, g) for n, (_lt, a, g) in layers.items()},
                                 layer_types={n: lt for n, (lt, _a, _g) in layers.items()})


def _seq_first(f):
    from dattri_llm_amd.gradient.gradient import Factorized

    return Factorized(f.activation.transpose(0, 1).contiguous(), f.pre_activation_grad.transpose(0, 1).contiguous(),
                      module_kwargs=f.module_kwargs, batch_first=False)


# -- streaming accumulators (test_ops.py:428-482) ---------------------------------------------


def test_kfac_streaming_equals_batch(device, gen):
    from dattri_llm_amd.gradient import ops

    (a1, g1), (a2, g2) = _linear_2d(gen, device), _linear_2d(gen, device)
    A_b, G_b = ops.kfac_factors(torch.cat([a1, a2]), torch.cat([g1, g2]), "nn.Linear")
    acc = ops.LayerKroneckerAccumulator()
    acc.update(a1, g1, "nn.Linear")
    acc.update(a2, g2, "nn.Linear")
    A_s, G_s = acc.result()
    assert torch.allclose(A_b, A_s, atol=1e-5) and torch.allclose(G_b, G_s, atol=1e-5)


def test_fim_streaming_and_update_from_grad(device, gen):
    from dattri_llm_amd.gradient import ops

    (a1, g1), (a2, g2) = _linear_2d(gen, device), _linear_2d(gen, device)
    F_b = ops.fim_factors(torch.cat([a1, a2]), torch.cat([g1, g2]), "nn.Linear")
    acc = ops.LayerFisherAccumulator()
    acc.update(a1, g1, "nn.Linear")
    acc.update(a2, g2, "nn.Linear")
    assert torch.allclose(F_b, acc.result(), atol=1e-5)
    ref = ops.LayerFisherAccumulator()
    ref.update(a1, g1, "nn.Linear")
    direct = ops.LayerFisherAccumulator()
    direct.update_from_grad(ops.materialize_factors(a1, g1, "nn.Linear"))
    assert torch.allclose(ref.result(), direct.result(), atol=1e-6)


def test_reset_clears_state(device, gen):
    from dattri_llm_amd.gradient import ops

    acc = ops.LayerKroneckerAccumulator()
    acc.update(*_linear_2d(gen, device), "nn.Linear")
    acc.reset()
    with pytest.raises(RuntimeError):
        acc.result()


# -- token collapse (test_ops.py:485-518) ------------------------------------------------------


def test_norm_collapse_and_per_token(device, gen):
    from dattri_llm_amd.gradient import ops

    a, g = _norm_3d(gen, device)
    per_token = ops.materialize_factors(a, g, "nn.LayerNorm", per_token=True)
    wg = ops.materialize_factors(a, g, "nn.LayerNorm")
    assert wg.shape == (B, D_IN)
    assert torch.allclose(wg, per_token.reshape(B, T, D_IN).sum(1), atol=1e-5)
    m1 = ops.materialize_factors(*_on(device, torch.randn(B, 3, D_IN), torch.randn(B, 3, D_IN)), "nn.LayerNorm")
    m2 = ops.materialize_factors(*_on(device, torch.randn(B, 7, D_IN), torch.randn(B, 7, D_IN)), "nn.LayerNorm")
    assert m1.shape == m2.shape == (B, D_IN)


@pytest.mark.parametrize("lt", ["nn.Linear", "nn.Embedding"])
def test_per_token_noop_for_token_contracting_types(device, gen, lt):
    from dattri_llm_amd.gradient import ops

    if lt == "nn.Linear":
        a, g = _linear_3d(gen, device)
        kw = {}
    else:
        a, g = _embedding(gen, device)
        kw = {"module_kwargs": {"has_bias": False, "num_embeddings": VOCAB, "padding_idx": None}}
    assert torch.allclose(ops.materialize_factors(a, g, lt, per_token=True, **kw),
                          ops.materialize_factors(a, g, lt, **kw), atol=1e-6)


# -- multi-layer accumulators (test_ops.py:778-825) --------------------------------------------


def test_multi_layer_accumulators(device, gen):
    from dattri_llm_amd.gradient import ops

    (a1, g1), (a2, g2) = _linear_2d(gen, device), _linear_2d(gen, device)
    multi = ops.KroneckerAccumulator()
    multi.update(_block({"fc": ("nn.Linear", a1, g1), "out": ("nn.Linear", a2, g2)}), ["fc", "out"])
    res = multi.result()
    for name, (a, g) in {"fc": (a1, g1), "out": (a2, g2)}.items():
        ref = ops.LayerKroneckerAccumulator()
        ref.update(a, g, "nn.Linear")
        A_ref, G_ref = ref.result()
        assert torch.allclose(res[name][0], A_ref, atol=1e-6) and torch.allclose(res[name][1], G_ref, atol=1e-6)

    a, g = _norm_3d(gen, device)
    block = _block({"ln": ("nn.LayerNorm", a, g)})
    fisher = ops.FisherAccumulator()
    fisher.update(block, ["ln"])
    ref = ops.LayerFisherAccumulator()
    ref.update(a, g, "nn.LayerNorm")
    assert torch.allclose(fisher.result()["ln"], ref.result(), atol=1e-6)
    capped = ops.FisherAccumulator(max_params=D_IN - 1)
    capped.update(block, ["ln"])
    assert "ln" not in capped.result() and capped.skipped == {"ln": D_IN}
    kept = ops.FisherAccumulator(max_params=D_IN)
    kept.update(block, ["ln"])
    assert "ln" in kept.result() and kept.skipped == {}


# -- Factorized wrappers (test_ops.py:841-955) -------------------------------------------------


def test_factorized_wrappers_match_raw(device, gen):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized

    a, g = _linear_3d(gen, device)
    f = Factorized(a, g)
    assert torch.allclose(ops.materialize(f, "nn.Linear"), ops.materialize_factors(a, g, "nn.Linear"))
    assert torch.allclose(ops.grad_norm_sq(f, "nn.Linear"), ops.grad_norm_sq_factors(a, g, "nn.Linear"))
    A1, G1 = ops.kfac(f, "nn.Linear")
    A2, G2 = ops.kfac_factors(a, g, "nn.Linear")
    assert torch.allclose(A1, A2) and torch.allclose(G1, G2)
    na, ng = _norm_3d(gen, device)
    assert torch.allclose(ops.materialize(Factorized(na, ng), "nn.LayerNorm"),
                          ops.materialize_factors(na, ng, "nn.LayerNorm"))
    a2, g2 = _linear_3d(gen, device)
    assert torch.allclose(ops.cross_dot(f, Factorized(a2, g2), "nn.Linear"),
                          ops.cross_dot_factors(a, g, a2, g2, "nn.Linear"))


@pytest.mark.parametrize("lt", ["nn.Linear", "nn.LayerNorm"])
def test_materialize_seq_first_equals_batch_first(device, gen, lt):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized

    bf = Factorized(*(_linear_3d if lt == "nn.Linear" else _norm_3d)(gen, device))
    assert torch.allclose(ops.materialize(bf, lt), ops.materialize(_seq_first(bf), lt), atol=1e-5)


def test_kfac_and_ekfac_seq_first_and_dense_block(device, gen):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized

    bf1, bf2 = Factorized(*_linear_3d(gen, device)), Factorized(*_linear_3d(gen, device))
    A, G = ops.kfac_factors(bf1.activation, bf1.pre_activation_grad, "nn.Linear")
    A_inv, G_inv = ops.sym_inverse(A, 1e-3), ops.sym_inverse(G, 1e-3)
    assert torch.allclose(ops.kfac_cross(bf1, bf2, "nn.Linear", A_inv, G_inv),
                          ops.kfac_cross(_seq_first(bf1), _seq_first(bf2), "nn.Linear", A_inv, G_inv), atol=1e-4)
    _sA, U_A, _sG, U_G = ops.kfac_eigh(A, G)
    assert torch.allclose(ops.ekfac_materialize(bf1, "nn.Linear", U_A, U_G),
                          ops.ekfac_materialize(_seq_first(bf1), "nn.Linear", U_A, U_G), atol=1e-4)
    dense = ops.materialize(bf1, "nn.Linear")
    M = ops.ekfac_materialize(dense, "nn.Linear", U_A, U_G)
    assert torch.allclose(M, ops.ekfac_materialize(bf1, "nn.Linear", U_A, U_G), atol=1e-4)
    back = ops.ekfac_precondition(M, U_A, U_G, torch.ones(M.shape[1], device=device), "nn.Linear")
    assert torch.allclose(back, dense.float(), atol=1e-4)


# -- damped inverses (test_ops.py:957-1000) ----------------------------------------------------


def test_dense_inverse(device):
    from dattri_llm_amd.gradient import ops

    torch.manual_seed(0)
    g = torch.randn(64, 32, device=device)
    m = g.T @ g
    inv = ops.dense_inverse(m, 1e-2)
    assert torch.allclose((m + 1e-2 * torch.eye(32, device=device)) @ inv, torch.eye(32, device=device), atol=1e-4)
    assert torch.allclose(inv, inv.T, atol=1e-5)
    g = torch.randn(128, 40, device=device)
    m = g.T @ g
    for damping in (1e-1, 1e-2):
        assert torch.allclose(ops.sym_inverse(m, damping), ops.dense_inverse(m, damping), rtol=1e-3, atol=1e-4)
    v = torch.randn(16, 1, device=device)
    singular = v @ v.T  # not positive definite at zero damping: the eigh fallback
    assert torch.allclose(ops.dense_inverse(singular, 0.0), ops.sym_inverse(singular, 0.0), atol=1e-4)


# -- per-token cross-gram and the outer product (test_ops.py:1003-1042) ------------------------


@pytest.mark.parametrize("lt", ["nn.Linear", "nn.LayerNorm", "nn.Embedding"])
def test_cross_gram_per_token_sums_to_full(device, gen, lt):
    from dattri_llm_amd.gradient import ops

    factory = {"nn.Linear": _linear_3d, "nn.LayerNorm": _norm_3d, "nn.Embedding": _embedding}[lt]
    a1, g1 = factory(gen, device)
    a2, g2 = factory(gen, device)
    full = ops.cross_gram(a1, g1, a2, g2, lt)
    per_token = ops.cross_gram_per_token(a1, g1, a2, g2, lt)
    assert per_token.shape == (a1.shape[0], a1.shape[1], a2.shape[0])
    assert torch.allclose(per_token.sum(1), full, atol=1e-4, rtol=1e-4)


def test_outer_product_matches_einsum(device, gen):
    from dattri_llm_amd.gradient import ops

    a, g = _on(device, torch.randn(3, 7, 5, generator=gen), torch.randn(3, 7, 4, generator=gen))
    got = ops.materialize_factors(a, g, "nn.Linear")
    assert got.shape == (3, 4 * 5)
    assert torch.allclose(got, torch.einsum("bto,bti->boi", g, a).flatten(1), atol=1e-6)
    got = ops.materialize_factors(a, g, "nn.ConvTranspose2d")
    assert got.shape == (3, 5 * 4)
    assert torch.allclose(got, torch.einsum("blc,blp->bcp", a, g).flatten(1), atol=1e-6)


# -- ProjectionMatrix (test_ops.py:1045-1075) --------------------------------------------------


@pytest.mark.parametrize("include_bias", [False, True])
def test_projection_matrix_matches_apply(device, include_bias):
    from dattri_llm_amd.gradient.ops.projection import DattriProjector

    proj = DattriProjector()
    x = torch.randn(2, 5, 12, device=device)
    kw = {"proj_dim": 8, "proj_seed": 3, "proj_max_batch_size": 32}
    want = proj.apply(x, include_bias=include_bias, **kw)
    resolved = proj.resolve(12, include_bias=include_bias, device=x.device, dtype=x.dtype, **kw)
    assert resolved.matches(x)
    assert torch.equal(resolved(x), want)
    assert resolved(x).shape == (2, 5, 8)
    assert not resolved.matches(torch.randn(2, 5, 13, device=device))
    assert not resolved.matches(torch.randn(2, 5, 12, dtype=torch.float64, device=device))


# -- K-FAC shapes and gradient-free rows (test_ops.py:340-425) ----------------------------------


@pytest.mark.parametrize("lt,shape", [("nn.Linear", "2d"), ("nn.Linear", "3d"), ("nn.Conv1d", "3d"),
                                      ("nn.ConvTranspose1d", "3d")])
def test_kfac_and_fim_shapes(device, gen, lt, shape):
    from dattri_llm_amd.gradient import ops

    a, g = (_linear_2d if shape == "2d" else _linear_3d)(gen, device)
    A, G = ops.kfac_factors(a, g, lt)
    assert A.shape == (D_IN, D_IN) and G.shape == (D_OUT, D_OUT)
    F = ops.fim_factors(a, g, lt)
    assert F.dim() == 2 and F.shape[0] == F.shape[1] == D_IN * D_OUT


@pytest.mark.parametrize("lt", ["nn.LayerNorm", "nn.Embedding"])
def test_kfac_not_implemented(device, gen, lt):
    from dattri_llm_amd.gradient import ops

    a, g = _norm_3d(gen, device) if "Norm" in lt else _embedding(gen, device)
    with pytest.raises(NotImplementedError):
        ops.kfac_factors(a, g, lt)


def _padded(device):
    gen = torch.Generator().manual_seed(0)
    a = torch.randn(B, 5, D_IN, generator=gen)
    g = torch.randn(B, 5, D_OUT, generator=gen)
    g[:, 3:] = 0.0
    return _on(device, a, g)


def test_kfac_gradient_free_rows(device):
    """Sequence layers drop rows with an all-zero gradient from the factors and
    the count; a convolution keeps them (its zeros are architectural)."""
    from dattri_llm_amd.gradient import ops

    a, g = _padded(device)
    A_pad, G_pad = ops.kfac_factors(a, g, "nn.Linear")
    A_ref, G_ref = ops.kfac_factors(a[:, :3].contiguous(), g[:, :3].contiguous(), "nn.Linear")
    assert torch.allclose(A_pad, A_ref, atol=1e-6) and torch.allclose(G_pad, G_ref, atol=1e-6)
    acc = ops.LayerKroneckerAccumulator()
    acc.update(a, g, "nn.Linear")
    A_s, G_s = acc.result()
    assert torch.allclose(A_s, A_pad, atol=1e-6) and torch.allclose(G_s, G_pad, atol=1e-6)
    a_long = torch.cat([a, torch.randn(B, 4, D_IN, device=device)], dim=1)
    g_long = torch.cat([g, torch.zeros(B, 4, D_OUT, device=device)], dim=1)
    A2, G2 = ops.kfac_factors(a_long, g_long, "nn.Linear")
    assert torch.allclose(A_pad, A2, atol=1e-6) and torch.allclose(G_pad, G2, atol=1e-6)
    # a convolution's rows all count
    A_c, _G_c = ops.kfac_factors(a, g, "nn.Conv1d")
    a64 = a.double().reshape(-1, D_IN)
    assert torch.allclose(A_c.double(), a64.T @ a64 / a64.shape[0], atol=1e-5)
    zeros = torch.zeros(B, 3, D_OUT, device=device)
    with pytest.raises(ValueError, match="zero"):
        ops.kfac_factors(a[:, :3].contiguous(), zeros, "nn.Linear")
    acc = ops.LayerKroneckerAccumulator()
    acc.update(a[:, :3].contiguous(), zeros, "nn.Linear")
    with pytest.raises(RuntimeError, match="gradient-carrying"):
        acc.result()
