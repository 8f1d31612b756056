"""Pinning the numpy oracle (CPU).  Each check is independent of the oracle's
own formula: brute-force loops, torch autograd per-sample gradients, torch
library routines, algebraic identities, and the reference's known-answer
tables (tests/golden/routing_known_answers.json)."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import REPO, rel_err

GOLDEN = os.path.join(REPO, "tests", "golden")


def _rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# ghost cross-gram
# ---------------------------------------------------------------------------


def _brute_ghost(a1, g1, a2, g2):
    b1, s1, _ = a1.shape
    b2, s2, _ = a2.shape
    out = np.zeros((b1, b2))
    for i in range(b1):
        for j in range(b2):
            acc = 0.0
            for t in range(s1):
                for s in range(s2):
                    acc += float(a1[i, t] @ a2[j, s]) * float(g1[i, t] @ g2[j, s])
            out[i, j] = acc
    return out


def test_ghost_matches_brute_force_loops():
    r = _rng(0)
    a1, g1 = r.standard_normal((3, 4, 5)), r.standard_normal((3, 4, 6))
    a2, g2 = r.standard_normal((2, 3, 5)), r.standard_normal((2, 3, 6))
    np.testing.assert_allclose(oracle.cross_gram_factorized(a1, g1, a2, g2), _brute_ghost(a1, g1, a2, g2),
                               rtol=1e-12, atol=1e-12)


def test_ghost_bias_is_a_ones_column():
    r = _rng(1)
    a1, g1 = r.standard_normal((2, 5, 4)), r.standard_normal((2, 5, 3))
    a2, g2 = r.standard_normal((3, 2, 4)), r.standard_normal((3, 2, 3))
    ones = lambda a: np.concatenate([a, np.ones(a.shape[:-1] + (1,))], -1)  # noqa: E731
    np.testing.assert_allclose(oracle.cross_gram_factorized(a1, g1, a2, g2, bias=True),
                               _brute_ghost(ones(a1), g1, ones(a2), g2), rtol=1e-12)


def _brute_per_token(a1, g1, a2, g2, bias=0.0):
    b1, s1, _ = a1.shape
    b2, s2, _ = a2.shape
    out = np.zeros((b1, s1, b2))
    for i in range(b1):
        for t in range(s1):
            for j in range(b2):
                out[i, t, j] = sum((float(a1[i, t] @ a2[j, s]) + bias) * float(g1[i, t] @ g2[j, s])
                                   for s in range(s2))
    return out


@pytest.mark.parametrize("bias", [False, True])
def test_per_token_matches_brute_force_loops(bias):
    r = _rng(11)
    a1, g1 = r.standard_normal((2, 5, 4)), r.standard_normal((2, 5, 3))
    a2, g2 = r.standard_normal((3, 2, 4)), r.standard_normal((3, 2, 3))
    got = oracle.cross_gram_per_token(a1, g1, a2, g2, bias=bias)
    np.testing.assert_allclose(got, _brute_per_token(a1, g1, a2, g2, 1.0 if bias else 0.0), rtol=1e-12, atol=1e-12)


def test_per_token_sums_to_the_cross_gram():
    """dot.py:181-183: summing over side 1's tokens recovers the (B1, B2) score."""
    r = _rng(12)
    a1, g1 = r.standard_normal((3, 7, 6)), r.standard_normal((3, 7, 5))
    a2, g2 = r.standard_normal((2, 4, 6)), r.standard_normal((2, 4, 5))
    for bias in (False, True):
        np.testing.assert_allclose(oracle.cross_gram_per_token(a1, g1, a2, g2, bias=bias).sum(axis=1),
                                   _brute_ghost(*(np.concatenate([x, np.ones(x.shape[:-1] + (1,))], -1)
                                                  if bias and n in (0, 2) else x
                                                  for n, x in enumerate((a1, g1, a2, g2)))),
                                   rtol=1e-10)
    x1, y1, x2, y2 = r.standard_normal((2, 5, 8)), r.standard_normal((2, 5, 8)), \
        r.standard_normal((3, 4, 8)), r.standard_normal((3, 4, 8))
    np.testing.assert_allclose(oracle.cross_gram_per_token(x1, y1, x2, y2, "nn.RMSNorm").sum(axis=1),
                               (x1 * y1).sum(1) @ (x2 * y2).sum(1).T, rtol=1e-10)


def test_per_token_dense_equals_factorized_form():
    r = _rng(13)
    a1, g1 = r.standard_normal((2, 6, 5)), r.standard_normal((2, 6, 4))
    a2, g2 = r.standard_normal((3, 3, 5)), r.standard_normal((3, 3, 4))
    for bias in (False, True):
        m2 = oracle.materialize_linear(a2, g2, bias=bias)  # (B2, D*(K+bias)), index o*K' + i
        np.testing.assert_allclose(oracle.cross_gram_per_token_dense(a1, g1, m2, bias=bias),
                                   _brute_per_token(a1, g1, a2, g2, 1.0 if bias else 0.0), rtol=1e-10)
    x1, y1 = r.standard_normal((2, 5, 8)), r.standard_normal((2, 5, 8))
    grad2 = r.standard_normal((3, 8))
    want = np.array([[[sum(x1[i, t, d] * y1[i, t, d] * grad2[j, d] for d in range(8)) for j in range(3)]
                      for t in range(5)] for i in range(2)])
    np.testing.assert_allclose(oracle.cross_gram_per_token_dense(x1, y1, grad2, "nn.RMSNorm"), want, rtol=1e-10)


def test_ghost_equals_materialized_route():
    r = _rng(2)
    a1, g1 = r.standard_normal((4, 7, 6)), r.standard_normal((4, 7, 5))
    a2, g2 = r.standard_normal((3, 9, 6)), r.standard_normal((3, 9, 5))
    for bias in (False, True):
        np.testing.assert_allclose(oracle.cross_gram_factorized(a1, g1, a2, g2, bias),
                                   oracle.cross_gram_materialized(a1, g1, a2, g2, bias), rtol=1e-10)


def _linear_per_sample(a, c):
    """Per-sample [W.grad, b.grad] of a linear layer under loss_i = sum_t c_it . y_it."""
    a_t = torch.tensor(a)
    c_t = torch.tensor(c)
    lin = torch.nn.Linear(a.shape[-1], c.shape[-1]).double()
    rows = []
    for i in range(a.shape[0]):
        lin.zero_grad()
        (lin(a_t[i]) * c_t[i]).sum().backward()
        rows.append(torch.cat([lin.weight.grad, lin.bias.grad[:, None]], 1).flatten().numpy().copy())
    return np.stack(rows)


def test_cross_gram_and_materialize_against_autograd():
    """<dW_i, dW_j> with the bias and the (B, out*(in+1)) layout pinned by autograd."""
    r = _rng(3)
    a1, c1 = r.standard_normal((3, 6, 5)), r.standard_normal((3, 6, 4))
    a2, c2 = r.standard_normal((2, 4, 5)), r.standard_normal((2, 4, 4))
    w1, w2 = _linear_per_sample(a1, c1), _linear_per_sample(a2, c2)
    np.testing.assert_allclose(oracle.materialize_linear(a1, c1, bias=True), w1, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(oracle.cross_gram_factorized(a1, c1, a2, c2, bias=True), w1 @ w2.T, rtol=1e-10)


# ---------------------------------------------------------------------------
# norms
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("eps", [1e-6, None])
def test_rms_x_hat_matches_torch(eps):
    x = torch.randn(3, 7, 16, dtype=torch.float64) * 2
    ref = torch.nn.functional.rms_norm(x, (16,), eps=eps)
    eps_v = torch.finfo(torch.float64).eps if eps is None else eps
    np.testing.assert_allclose(oracle.rms_x_hat(x.numpy(), eps_v), ref.numpy(), rtol=1e-12)


def test_machine_eps_constants():
    assert oracle.BF16_EPS == torch.finfo(torch.bfloat16).eps
    assert oracle.F32_EPS == torch.finfo(torch.float32).eps
    assert oracle.F16_EPS == torch.finfo(torch.float16).eps


def test_layer_norm_x_hat_matches_torch():
    x = torch.randn(2, 5, 12, dtype=torch.float64) + 3
    ref = torch.nn.functional.layer_norm(x, (12,), eps=1e-5)
    np.testing.assert_allclose(oracle.layer_norm_x_hat(x.numpy(), 1e-5), ref.numpy(), rtol=1e-10)


@pytest.mark.parametrize("layer_type", ["nn.RMSNorm", "nn.LayerNorm"])
def test_norm_weight_grad_against_autograd(layer_type):
    torch.manual_seed(4)
    d = 10
    x = torch.randn(3, 6, d, dtype=torch.float64)
    c = torch.randn(3, 6, d, dtype=torch.float64)
    mod = (torch.nn.RMSNorm(d, eps=1e-5) if layer_type == "nn.RMSNorm" else torch.nn.LayerNorm(d, eps=1e-5)).double()
    with torch.no_grad():
        mod.weight.copy_(torch.randn(d))
    has_bias = getattr(mod, "bias", None) is not None
    rows = []
    for i in range(3):
        mod.zero_grad()
        (mod(x[i]) * c[i]).sum().backward()
        parts = [mod.weight.grad.clone()] + ([mod.bias.grad.clone()] if has_bias else [])
        rows.append(torch.cat(parts).numpy())
    # the captured output gradient of a norm's *affine* input is c * weight
    g = (c * mod.weight.detach()).numpy()
    got = oracle.norm_weight_grad(x.numpy(), g / mod.weight.detach().numpy(), layer_type, 1e-5, has_bias)
    np.testing.assert_allclose(got, np.stack(rows), rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("layer_type,has_bias", [("nn.LayerNorm", True), ("nn.LayerNorm", False),
                                                   ("nn.RMSNorm", False), ("nn.Linear", True), ("nn.Linear", False)])
def test_preprocess_against_autograd(layer_type, has_bias):
    """preprocess_factors' final factors give the per-sample parameter gradient
    autograd computes: norms by the token sum of a * g ([dgamma, dbeta] with a
    bias), linear layers by sum_t g_t a_t^T (the ones column is the bias)."""
    torch.manual_seed(11)
    b, t, d_in, d_out = 3, 5, 8, 6
    d = d_in
    x = torch.randn(b, t, d, dtype=torch.float64) + 0.5
    if layer_type == "nn.Linear":
        mod = torch.nn.Linear(d_in, d_out, bias=has_bias).double()
        c = torch.randn(b, t, d_out, dtype=torch.float64)
    elif layer_type == "nn.LayerNorm":
        mod = torch.nn.LayerNorm(d, eps=1e-5, elementwise_affine=True, bias=has_bias).double()
        c = torch.randn(b, t, d, dtype=torch.float64)
    else:
        mod = torch.nn.RMSNorm(d, eps=1e-5).double()
        c = torch.randn(b, t, d, dtype=torch.float64)
    want = []
    for i in range(b):
        mod.zero_grad()
        (mod(x[i]) * c[i]).sum().backward()
        if layer_type == "nn.Linear":
            parts = [mod.weight.grad.clone()] + ([mod.bias.grad[:, None].clone()] if has_bias else [])
            want.append(torch.cat(parts, 1).flatten().numpy())
        else:
            parts = [mod.weight.grad.clone()] + ([mod.bias.grad.clone()] if has_bias else [])
            want.append(torch.cat(parts).numpy())
    a, g = oracle.preprocess(x.numpy(), c.numpy(), layer_type, {"eps": 1e-5, "has_bias": has_bias})
    if layer_type == "nn.Linear":
        got = np.einsum("bto,bti->boi", g, a).reshape(b, -1)
    else:
        got = (a * g).sum(1)
    np.testing.assert_allclose(got, np.stack(want), rtol=1e-10, atol=1e-12)
    # without module kwargs the factors are already final and pass through
    a0, g0 = oracle.preprocess(x.numpy(), c.numpy(), layer_type, None)
    assert a0 is not None and np.array_equal(a0, x.numpy()) and np.array_equal(g0, c.numpy())


# ---------------------------------------------------------------------------
# projection
# ---------------------------------------------------------------------------


def test_project_bias_row_is_a_ones_column():
    r = _rng(5)
    x = r.standard_normal((2, 3, 6))
    p = r.standard_normal((7, 4))
    with_ones = np.concatenate([x, np.ones((2, 3, 1))], -1)
    np.testing.assert_allclose(oracle.project(x, p[:-1], p[-1]), with_ones @ p, rtol=1e-12)


def test_project_outer_is_kronecker_of_materialized():
    """materialize(project) == P_out^T dW P_in (vec-Kronecker identity)."""
    r = _rng(6)
    a, g = r.standard_normal((3, 8, 6)), r.standard_normal((3, 8, 5))
    p_in, p_out = r.standard_normal((7, 4)), r.standard_normal((5, 3))
    got = oracle.project_outer(a, g, p_in, p_out, bias=True).reshape(3, 3, 4)
    dw = oracle.materialize_linear(a, g, bias=True).reshape(3, 5, 7)
    want = np.einsum("go,bgi,ik->bok", p_out, dw, p_in)
    np.testing.assert_allclose(got, want, rtol=1e-10)


# ---------------------------------------------------------------------------
# score GEMM and cost rules
# ---------------------------------------------------------------------------


def test_score_gemm_matches_loops():
    r = _rng(7)
    m1 = [r.standard_normal((3, 5)), r.standard_normal((3, 2))]
    m2 = [r.standard_normal((4, 5)), r.standard_normal((4, 2))]
    want = np.array([[sum(float(m1[L][i] @ m2[L][j]) for L in range(2)) for j in range(4)] for i in range(3)])
    np.testing.assert_allclose(oracle.score_gemm(m1, m2), want, rtol=1e-12)


def _known():
    with open(os.path.join(GOLDEN, "routing_known_answers.json")) as f:
        return json.load(f)


def test_cost_rules_known_answers():
    k = _known()
    for c in k["maybe_materialize_projected"]:
        assert oracle.maybe_materialize_projected(c["seq_len"], c["k_a"], c["k_g"], c["kappa"]) is c["expected"]
    for c in k["should_materialize"]:
        assert oracle.should_materialize(c["style"], c["seq_len"], c["k_a"], c["k_g"]) is c["expected"]
    for c in k["maybe_use_materialized_gram"]:
        assert oracle.maybe_use_materialized_gram(c["B1"], c["B2"], c["S"], c["K"], c["D"]) is c["expected"]
    with pytest.raises(ValueError, match="capture_style"):
        oracle.should_materialize("bogus", 4, 8, 8)


def test_norm_rule_crossover_known_answers():
    """Per-sample norms: materialize iff S >= H = D*K / (D + K), the crossover
    where the ghost's S^2 (D + K) flops meet the dW's S*D*K.  Known answers
    on both sides of H, at H exactly (materialize), and at the Llama-8B block's
    train (S = 2048) and query (S = 512) widths."""
    cases = [
        ((32, 64, 64), True),       # H = 32
        ((31, 64, 64), False),
        ((2048, 4096, 4096), True),  # H = 2048: attention q/o at the train length
        ((2047, 4096, 4096), False),
        ((2048, 4096, 1024), True),  # k/v: H = 819.2
        ((819, 4096, 1024), False),
        ((820, 4096, 1024), True),
        ((2048, 4096, 14336), False),  # gate/up: H = 3185.8
        ((2048, 14336, 4096), False),  # down
        ((3186, 4096, 14336), True),
        ((3185, 4096, 14336), False),
        ((512, 4096, 4096), False),  # every query-length layer stays factorized
        ((1, 1, 1), True),  # H = 1/2
        ((0, 8, 8), False),
    ]
    for (s, k, d), want in cases:
        assert oracle.maybe_use_materialized_norm(s, k, d) is want, (s, k, d)
        assert oracle.maybe_use_materialized_norm(s, d, k) is want  # symmetric in K and D


def test_every_oracle_function_is_pinned():
    """Each public oracle name is exercised by a pinning test in this file or
    in tests/test_topk_select.py (constants by test_machine_eps_constants)."""
    here = os.path.dirname(os.path.abspath(__file__))
    text = "".join(open(os.path.join(here, f)).read() for f in ("test_oracle.py", "test_topk_select.py"))
    import oracle.ops

    missing = [n for n in oracle.ops.__all__ if f"oracle.{n}" not in text]
    assert not missing, missing


def test_cost_rule_is_the_flop_comparison():
    """A route the rule calls cheaper really has fewer counted flops."""
    for b1, b2, s, k, d in [(8, 64, 2048, 4096, 14336), (256, 64, 512, 4096, 4096), (8, 1, 4, 8, 8)]:
        f = b1 * b2 * s * s * (k + d)
        m = (b1 + b2) * s * d * k + b1 * b2 * d * k
        assert oracle.maybe_use_materialized_gram(b1, b2, s, k, d) == (f >= m)


# ---------------------------------------------------------------------------
# MoE
# ---------------------------------------------------------------------------


def test_router_matches_torch_topk():
    logits = torch.randn(300, 8, generator=torch.Generator().manual_seed(8))
    w, idx = oracle.moe_router_topk(logits.numpy(), 2)
    probs = torch.softmax(logits.float(), dim=-1)
    tv, ti = torch.topk(probs, 2, dim=-1)
    assert np.array_equal(idx, ti.numpy())
    np.testing.assert_allclose(w, (tv / tv.sum(-1, keepdim=True)).numpy(), rtol=1e-6)


def test_segments_match_torch_where_order():
    idx = torch.randint(0, 8, (50, 2), generator=torch.Generator().manual_seed(9))
    mask = torch.nn.functional.one_hot(idx, num_classes=8).permute(2, 1, 0)
    segs = oracle.moe_segments(idx.numpy(), 8)
    for e in range(8):
        pos, tok = torch.where(mask[e])
        assert np.array_equal(segs[e][0], pos.numpy()) and np.array_equal(segs[e][1], tok.numpy())


def test_regroup_scatters_rows_to_their_positions():
    """RowLayout.regroup: routed row p lands at (token // T, token % T), every
    other position stays zero."""
    r = _rng(12)
    rows = r.standard_normal((4, 3))
    tok = np.array([5, 0, 11, 7])
    got = oracle.moe_regroup_dense(rows, tok, 3, 4)
    want = np.zeros((3, 4, 3))
    for p in range(4):
        want[tok[p] // 4, tok[p] % 4] = rows[p]
    assert np.array_equal(got, want)
    assert np.count_nonzero(got.any(-1)) == 4


def test_segment_ghost_equals_dense_with_zeros_by_brute_force():
    r = _rng(10)
    batch, tokens = 3, 5
    tok1 = np.array([0, 3, 7, 8, 14])
    tok2 = np.array([1, 2, 9])
    a1, g1 = r.standard_normal((5, 4)), r.standard_normal((5, 3))
    a2, g2 = r.standard_normal((3, 4)), r.standard_normal((3, 3))
    got = oracle.moe_segment_ghost(a1, g1, tok1, a2, g2, tok2, batch, batch, tokens, tokens)
    want = np.zeros((batch, batch))
    for p in range(5):
        for q in range(3):
            want[tok1[p] // tokens, tok2[q] // tokens] += float(a1[p] @ a2[q]) * float(g1[p] @ g2[q])
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("bias", [False, True])
def test_compact_segment_ghost_equals_dense_with_zeros(bias):
    r = _rng(13)
    b1, b2, t1, t2 = 4, 3, 9, 7
    cases = [(np.array([0, 5, 8, 13, 30, 35]), np.array([2, 3, 9, 20])),  # ragged samples
             (np.array([], dtype=np.int64), np.array([1, 4])),             # empty side
             (np.array([10, 11, 12]), np.array([0, 6]))]                   # one sample per side
    for tok1, tok2 in cases:
        a1, g1 = r.standard_normal((len(tok1), 5)), r.standard_normal((len(tok1), 6))
        a2, g2 = r.standard_normal((len(tok2), 5)), r.standard_normal((len(tok2), 6))
        want = oracle.moe_segment_ghost(a1, g1, tok1, a2, g2, tok2, b1, b2, t1, t2, bias=bias)
        got = oracle.moe_segment_ghost_compact(a1, g1, tok1, a2, g2, tok2, b1, b2, t1, t2, bias=bias)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
        brute = np.zeros((b1, b2))
        for p in range(len(tok1)):
            for q in range(len(tok2)):
                ka = float(a1[p] @ a2[q]) + (1.0 if bias else 0.0)
                brute[tok1[p] // t1, tok2[q] // t2] += ka * float(g1[p] @ g2[q])
        np.testing.assert_allclose(got, brute, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# C1 end to end: oracle from captured factors == autograd ground truth fixture
# ---------------------------------------------------------------------------


def test_c1_oracle_matches_autograd_fixture():
    from c1_model import c1_inputs, capture_factors

    with open(os.path.join(GOLDEN, "c1_scores.json")) as f:
        fixture = json.load(f)
    model, train, query = c1_inputs(0)
    assert int(train.sum()) == fixture["train_ids_checksum"]
    assert int(query.sum()) == fixture["query_ids_checksum"]
    f_tr = capture_factors(model, train)
    f_q = capture_factors(model, query)
    total = None
    for name in f_tr:
        a1, g1 = (t.double().numpy() for t in f_tr[name])
        a2, g2 = (t.double().numpy() for t in f_q[name])
        part = oracle.cross_gram(a1, g1, a2, g2, "nn.Linear", mode="factorized", bias=True)
        total = part if total is None else total + part
    assert rel_err(total, np.array(fixture["scores"])) <= 1e-5


# ---------------------------------------------------------------------------
# K-FAC / EK-FAC
# ---------------------------------------------------------------------------


def _spd(rng, n):
    m = rng.standard_normal((n, n))
    return m @ m.T / n + 0.5 * np.eye(n)


def _dw(a, g):
    """Per-sample dW = sum_t g_t a_t^T by explicit loops: (B, D, K)."""
    b, t, k = a.shape
    d = g.shape[-1]
    out = np.zeros((b, d, k))
    for i in range(b):
        for s in range(t):
            out[i] += np.outer(g[i, s], a[i, s])
    return out


def test_kfac_factors_brute_force_with_gradient_free_rows():
    rng = _rng(41)
    a = rng.standard_normal((3, 5, 4))
    g = rng.standard_normal((3, 5, 3))
    g[0, 1] = 0.0
    g[2, 4] = 0.0
    big_a, big_g = oracle.kfac_factors(a, g)
    rows = [(i, s) for i in range(3) for s in range(5) if (i, s) not in ((0, 1), (2, 4))]
    ref_a = sum(np.outer(a[i, s], a[i, s]) for i, s in rows) / len(rows)
    ref_g = sum(np.outer(g[i, s], g[i, s]) for i, s in rows) / len(rows)
    assert rel_err(big_a, ref_a) < 1e-12 and rel_err(big_g, ref_g) < 1e-12
    with pytest.raises(ValueError):
        oracle.kfac_factors(a, np.zeros_like(g))


def test_fim_and_sym_inverse_identities():
    rng = _rng(42)
    grad = rng.standard_normal((6, 5))
    ref = sum(np.outer(r, r) for r in grad) / 6
    assert rel_err(oracle.fim_factors(grad), ref) < 1e-12
    m = _spd(rng, 7)
    inv = oracle.sym_inverse(m, 0.3)
    assert np.abs((m + 0.3 * np.eye(7)) @ inv - np.eye(7)).max() < 1e-10


def test_kfac_cross_equals_explicit_kronecker_form():
    rng = _rng(43)
    b1, b2, t, k, d = 3, 2, 4, 5, 3
    a1, g1 = rng.standard_normal((b1, t, k)), rng.standard_normal((b1, t, d))
    a2, g2 = rng.standard_normal((b2, t, k)), rng.standard_normal((b2, t, d))
    a_inv, g_inv = np.linalg.inv(_spd(rng, k)), np.linalg.inv(_spd(rng, d))
    got = oracle.kfac_cross_factors(a1, g1, a2, g2, a_inv, g_inv)
    # vec(dW) row-major (index o*K + k): the preconditioner is kron(G^-1, A^-1)
    f_inv = np.kron(g_inv, a_inv)
    v1, v2 = _dw(a1, g1).reshape(b1, -1), _dw(a2, g2).reshape(b2, -1)
    ref = v1 @ f_inv @ v2.T
    assert rel_err(got, ref) < 1e-12
    # identity inverses reduce to the plain cross-gram; whitening side 2 instead gives the same
    assert rel_err(oracle.kfac_cross_factors(a1, g1, a2, g2, np.eye(k), np.eye(d)),
                   oracle.cross_gram_factorized(a1, g1, a2, g2)) < 1e-12
    assert rel_err(oracle.kfac_cross_factors(a2, g2, a1, g1, a_inv, g_inv).T, ref) < 1e-12


def test_kfac_precondition_materialized_is_the_kronecker_product():
    rng = _rng(44)
    k, d = 4, 3
    a_inv, g_inv = np.linalg.inv(_spd(rng, k)), np.linalg.inv(_spd(rng, d))
    block = rng.standard_normal((5, d * k))
    got = oracle.kfac_precondition_materialized(block, a_inv, g_inv)
    assert rel_err(got, block @ np.kron(g_inv, a_inv).T) < 1e-12


def test_ekfac_rotation_and_precondition():
    rng = _rng(45)
    b, t, k, d = 3, 4, 5, 3
    a, g = rng.standard_normal((b, t, k)), rng.standard_normal((b, t, d))
    _, u_a = np.linalg.eigh(_spd(rng, k))
    _, u_g = np.linalg.eigh(_spd(rng, d))
    rot = oracle.ekfac_materialize_factors(a, g, u_a, u_g)
    dw = _dw(a, g)
    ref = np.stack([u_g.T @ m @ u_a for m in dw]).reshape(b, -1)
    assert rel_err(rot, ref) < 1e-12
    assert rel_err(oracle.ekfac_rotate_materialized(dw.reshape(b, -1), u_a, u_g), ref) < 1e-12
    # lam = 1 undoes the rotation (orthogonal bases)
    assert rel_err(oracle.ekfac_precondition(rot, u_a, u_g, np.ones(d * k)), dw.reshape(b, -1)) < 1e-12
    # the EK-FAC score against a raw side: vec(dW1)^T (U (x) U) diag(1/lam) (U (x) U)^T vec(dW2)
    lam = rng.uniform(0.5, 2.0, d * k)
    u = np.kron(u_g, u_a)
    dw2 = _dw(rng.standard_normal((2, t, k)), rng.standard_normal((2, t, d))).reshape(2, -1)
    score = dw.reshape(b, -1) @ oracle.ekfac_precondition(
        oracle.ekfac_rotate_materialized(dw2, u_a, u_g), u_a, u_g, lam).T
    assert rel_err(score, dw.reshape(b, -1) @ u @ np.diag(1 / lam) @ u.T @ dw2.T) < 1e-12


# ---------------------------------------------------------------------------
# embedding layers
# ---------------------------------------------------------------------------


def _autograd_embedding_grads(ids, g, vocab, padding_idx=None, bag_mode=None):
    """Per-sample weight.grad of nn.Embedding / nn.EmbeddingBag (float64, CPU)
    for output gradients g, flattened to (B, vocab*E)."""
    e = g.shape[-1]
    torch.manual_seed(0)
    if bag_mode is None:
        layer = torch.nn.Embedding(vocab, e, padding_idx=padding_idx).double()
    else:
        layer = torch.nn.EmbeddingBag(vocab, e, mode=bag_mode, padding_idx=padding_idx).double()
    ids_t, g_t = torch.from_numpy(ids), torch.from_numpy(g)
    out = []
    for i in range(ids.shape[0]):
        layer.weight.grad = None
        (layer(ids_t[i:i + 1]) * g_t[i:i + 1]).sum().backward()
        out.append(layer.weight.grad.flatten().numpy().copy())
    return np.stack(out)


def test_embedding_materialize_against_autograd():
    r = _rng(40)
    vocab, b, t, e = 13, 3, 9, 5
    ids = r.integers(0, vocab, (b, t))
    ids[0, :4] = 7  # repeated ids accumulate into one row
    g = r.standard_normal((b, t, e))
    np.testing.assert_allclose(oracle.embedding_materialize(ids, g, vocab),
                               _autograd_embedding_grads(ids, g, vocab), rtol=1e-12, atol=1e-12)
    # padding_idx: the reference zeroes g at the pad positions (preprocess.py:403-408)
    pad = 2
    ids[:, -2:] = pad
    g_pad = np.where((ids == pad)[..., None], 0.0, g)
    np.testing.assert_allclose(oracle.embedding_materialize(ids, g_pad, vocab),
                               _autograd_embedding_grads(ids, g, vocab, padding_idx=pad), rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError):
        oracle.embedding_materialize(ids, g, 5)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_embedding_materialize_rounds_like_torch_scatter_add(dtype):
    """torch's CPU scatter_add_ (the reference's call, expanded index) sums in
    fp32 in ascending token order and rounds once to the dtype; the oracle
    agrees bit for bit (many repeats of few ids make the order and the
    accumulation dtype matter)."""
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    r = _rng(41)
    vocab, b, t, e = 6, 4, 200, 16
    ids = r.integers(0, vocab, (b, t))
    g = torch.from_numpy(r.standard_normal((b, t, e)) * 3).to(tdt)
    ref = torch.zeros(b, vocab, e, dtype=tdt)
    ref.scatter_add_(1, torch.from_numpy(ids).unsqueeze(-1).expand(b, t, e), g)
    got = oracle.embedding_materialize(ids, g.float().numpy(), vocab, dtype=dtype)
    assert np.array_equal(got.reshape(b, vocab, e), ref.float().numpy())
    # the accumulation dtype is visible: rounding after every add differs
    if dtype != "f32":
        per_add = torch.zeros(b, vocab, e, dtype=tdt)
        for s in range(t):
            per_add[torch.arange(b), torch.from_numpy(ids[:, s])] += g[:, s]
        assert not torch.equal(per_add, ref)


@pytest.mark.parametrize("mode", ["sum", "mean"])
@pytest.mark.parametrize("pad", [None, 0])
def test_embedding_bag_expand_against_autograd(mode, pad):
    r = _rng(42)
    vocab, n, t, e = 11, 4, 6, 3
    ids = r.integers(1, vocab, (n, t))
    if pad is not None:
        ids[:, -2:] = pad
        ids[1, -3] = pad  # a bag with another non-pad count
        ids[3, :] = pad  # an all-pad bag: zero gradient
    g = r.standard_normal((n, e))
    a, rows = oracle.embedding_bag_expand(ids, g, mode, pad)
    np.testing.assert_allclose(oracle.embedding_materialize(a, rows, vocab),
                               _autograd_embedding_grads(ids, g, vocab, padding_idx=pad, bag_mode=mode),
                               rtol=1e-12, atol=1e-12)


def _brute_embedding_gram(tok1, g1, tok2, g2):
    out = np.zeros((tok1.shape[0], tok1.shape[1], tok2.shape[0]))
    for i in range(tok1.shape[0]):
        for t in range(tok1.shape[1]):
            for j in range(tok2.shape[0]):
                out[i, t, j] = sum(float(g1[i, t] @ g2[j, s]) for s in range(tok2.shape[1])
                                   if tok1[i, t] == tok2[j, s])
    return out


def test_embedding_cross_gram_against_loops_and_autograd():
    r = _rng(43)
    vocab, e = 7, 4
    tok1, tok2 = r.integers(0, vocab, (3, 5)), r.integers(0, vocab, (2, 8))
    g1, g2 = r.standard_normal((3, 5, e)), r.standard_normal((2, 8, e))
    brute = _brute_embedding_gram(tok1, g1, tok2, g2)
    np.testing.assert_allclose(oracle.embedding_cross_gram(tok1, g1, tok2, g2), brute.sum(1), rtol=1e-12)
    m1 = _autograd_embedding_grads(tok1, g1, vocab)
    m2 = _autograd_embedding_grads(tok2, g2, vocab)
    np.testing.assert_allclose(oracle.embedding_cross_gram(tok1, g1, tok2, g2), m1 @ m2.T, rtol=1e-12, atol=1e-12)


def test_embedding_per_token_against_loops_and_dense_form():
    r = _rng(44)
    vocab, e = 6, 3
    tok1, tok2 = r.integers(0, vocab, (2, 7)), r.integers(0, vocab, (3, 4))
    g1, g2 = r.standard_normal((2, 7, e)), r.standard_normal((3, 4, e))
    per_tok = oracle.embedding_cross_gram_per_token(tok1, g1, tok2, g2)
    np.testing.assert_allclose(per_tok, _brute_embedding_gram(tok1, g1, tok2, g2), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(per_tok.sum(1), oracle.embedding_cross_gram(tok1, g1, tok2, g2), rtol=1e-12)
    m2 = oracle.embedding_materialize(tok2, g2, vocab)
    np.testing.assert_allclose(oracle.embedding_per_token_dense(tok1, g1, m2, vocab), per_tok,
                               rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# convolutions and grouped factors
# ---------------------------------------------------------------------------

# (transpose, rank, c_in, c_out, kernel, stride, padding, dilation, groups, bias, spatial)
CONV_CASES = [
    (False, 1, 3, 4, (3,), (2,), (1,), (1,), 1, True, (9,)),
    (False, 2, 4, 6, (3, 2), (1, 2), (1, 0), (2, 1), 2, True, (7, 6)),
    (False, 2, 4, 4, (3, 3), (1, 1), (1, 1), (1, 1), 4, False, (5, 5)),   # depthwise
    (False, 3, 2, 4, (2, 2, 2), (1, 2, 1), (1, 0, 1), (1, 1, 1), 2, True, (4, 4, 3)),
    (True, 1, 4, 3, (3,), (2,), (1,), (1,), 1, True, (5,)),
    (True, 2, 4, 6, (3, 3), (2, 1), (1, 1), (1, 2), 2, True, (3, 4)),
    (True, 2, 3, 2, (2, 2), (1, 1), (0, 0), (1, 1), 1, False, (3, 3)),
]


def conv_autograd_grads(case, x, gout):
    """Per-sample [weight.grad | bias.grad] of the layer in the reference's
    materialized layout, float64."""
    transpose, rank, c_in, c_out, k, s, p, d, groups, bias, _sp = case
    nn = torch.nn
    cls = {(False, 1): nn.Conv1d, (False, 2): nn.Conv2d, (False, 3): nn.Conv3d,
           (True, 1): nn.ConvTranspose1d, (True, 2): nn.ConvTranspose2d, (True, 3): nn.ConvTranspose3d}
    torch.manual_seed(0)
    layer = cls[(transpose, rank)](c_in, c_out, k, stride=s, padding=p, dilation=d, groups=groups,
                                   bias=bias).double()
    rows = []
    for i in range(x.shape[0]):
        layer.zero_grad()
        (layer(torch.from_numpy(x[i:i + 1])) * torch.from_numpy(gout[i:i + 1])).sum().backward()
        w = layer.weight.grad.numpy()
        if not transpose:
            m = w.reshape(c_out, -1)
            if bias:
                m = np.concatenate([m, layer.bias.grad.numpy()[:, None]], axis=1)
            rows.append(m.reshape(-1))
            continue
        cg_in, cg_out = c_in // groups, c_out // groups
        blocks = []
        for e in range(groups):
            wb = w[e * cg_in:(e + 1) * cg_in].reshape(cg_in, -1)
            if bias:
                full = np.zeros((cg_in + 1, wb.shape[1] + cg_out))
                full[:cg_in, :wb.shape[1]] = wb
                full[cg_in, wb.shape[1]:] = layer.bias.grad.numpy()[e * cg_out:(e + 1) * cg_out]
                wb = full
            blocks.append(wb.reshape(-1))
        rows.append(np.concatenate(blocks))
    return np.stack(rows)


def conv_inputs(case, n=3, seed=50):
    transpose, rank, c_in, c_out, k, s, p, d, groups, bias, sp = case
    r = _rng(seed)
    x = r.standard_normal((n, c_in) + sp)
    nn = torch.nn
    cls = {1: (nn.Conv1d, nn.ConvTranspose1d), 2: (nn.Conv2d, nn.ConvTranspose2d),
           3: (nn.Conv3d, nn.ConvTranspose3d)}[rank][int(transpose)]
    out_shape = cls(c_in, c_out, k, stride=s, padding=p, dilation=d, groups=groups).double()(
        torch.from_numpy(x)).shape
    gout = r.standard_normal(tuple(out_shape))
    return x, gout


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_preprocess_and_materialize_against_autograd(case):
    transpose, _rank, _ci, _co, k, s, p, d, groups, bias, _sp = case
    x, gout = conv_inputs(case)
    a, g = oracle.conv_preprocess(x, gout, transpose, k, s, p, d, groups, bias)
    assert a.ndim == (4 if groups > 1 else 3)
    np.testing.assert_allclose(oracle.conv_materialize(a, g, transpose), conv_autograd_grads(case, x, gout),
                               rtol=1e-10, atol=1e-10)
    # the unfolding itself for a 1-D conv, by hand: location l reads padded
    # positions l*s + j*d for taps j, channel-major
    if not transpose and len(k) == 1:
        xp = np.pad(x, [(0, 0), (0, 0), (p[0], p[0])])
        unf = oracle.conv_unfold(x, k, s, p, d)
        for loc in range(unf.shape[1]):
            want = [xp[:, c, loc * s[0] + j * d[0]] for c in range(x.shape[1]) for j in range(k[0])]
            np.testing.assert_array_equal(unf[:, loc], np.stack(want, axis=1))


def test_grouped_cross_gram_and_per_token():
    r = _rng(51)
    a1, g1 = r.standard_normal((3, 5, 2, 4)), r.standard_normal((3, 5, 2, 3))
    a2, g2 = r.standard_normal((2, 4, 2, 4)), r.standard_normal((2, 4, 2, 3))
    m1, m2 = oracle.conv_materialize(a1, g1), oracle.conv_materialize(a2, g2)
    np.testing.assert_allclose(oracle.grouped_cross_gram(a1, g1, a2, g2), m1 @ m2.T, rtol=1e-12)
    pt = oracle.grouped_cross_gram_per_token(a1, g1, a2, g2)
    np.testing.assert_allclose(pt.sum(1), m1 @ m2.T, rtol=1e-12)
    brute = np.zeros_like(pt)
    for i in range(3):
        for t in range(5):
            for j in range(2):
                brute[i, t, j] = sum(float(a1[i, t, e] @ a2[j, s, e]) * float(g1[i, t, e] @ g2[j, s, e])
                                     for e in range(2) for s in range(4))
    np.testing.assert_allclose(pt, brute, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# channel norms
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("kind", ["group", "instance"])
def test_channel_norm_oracle_against_torch(kind):
    r = _rng(90)
    n, c, h, w = 3, 6, 4, 5
    groups = 3 if kind == "group" else c
    x, gout = r.standard_normal((n, c, h, w)) * 2 + 1, r.standard_normal((n, c, h, w))
    eps = 1e-5
    want = torch.nn.functional.group_norm(torch.from_numpy(x), groups, eps=eps).numpy()
    np.testing.assert_allclose(oracle.group_norm_x_hat(x, groups, eps), want, rtol=1e-10, atol=1e-10)
    if kind == "group":
        layer = torch.nn.GroupNorm(groups, c, eps=eps).double()
    else:
        layer = torch.nn.InstanceNorm2d(c, eps=eps, affine=True).double()
    rows = []
    for i in range(n):
        layer.zero_grad()
        (layer(torch.from_numpy(x[i:i + 1])) * torch.from_numpy(gout[i:i + 1])).sum().backward()
        rows.append(np.concatenate([layer.weight.grad.numpy(), layer.bias.grad.numpy()]))
    a, g = oracle.channel_norm_preprocess(x, gout, groups, eps, has_bias=True)
    assert a.shape == (n, h * w, 2 * c)
    np.testing.assert_allclose((a * g).sum(axis=1), np.stack(rows), rtol=1e-10, atol=1e-10)


# ---------------------------------------------------------------------------
# routed-row location
# ---------------------------------------------------------------------------


def test_match_rows_known_cases():
    r = _rng(95)
    src = r.standard_normal((24, 5)).astype(np.float32)
    src[7] = src[3]  # a repeated token (a repeated sample or shared prefix)
    src[19] = src[3]
    # an expert's rows as fused_experts gathers them: torch.where over a mask, ascending
    mask = np.zeros(24, dtype=bool)
    mask[[1, 3, 7, 8, 19, 22]] = True
    idx = torch.where(torch.from_numpy(mask))[0].numpy()
    assert np.array_equal(oracle.match_rows(src[idx], src), idx)
    # the same value three times in x: ascending tokens in order of appearance
    assert np.array_equal(oracle.match_rows(src[[3, 5, 3, 3]], src), [3, 5, 7, 19])
    # identity
    assert np.array_equal(oracle.match_rows(src, src), np.arange(24))
    # a row that is not a block row, and more copies than the block holds
    assert oracle.match_rows(r.standard_normal((1, 5)).astype(np.float32), src) is None
    assert oracle.match_rows(src[[3, 3, 3, 3]], src) is None
    # a NaN row has matching bits but is not equal to itself (torch.equal)
    nan_src = src.copy()
    nan_src[2, 1] = np.nan
    assert oracle.match_rows(nan_src[[2]], nan_src) is None
    assert not torch.equal(torch.from_numpy(nan_src[[2]]), torch.from_numpy(nan_src[[2]]))
