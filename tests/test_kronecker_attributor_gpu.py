"""K-FAC / EK-FAC attributors on the MI355X against the oracle
(the reference's attribution/algorithm/kronecker.py workflow; its suites are
tests/attribution/test_kronecker.py and test_token_granularity.py:168-216).

Every expected score is built in float64 from oracle functions pinned in
test_oracle.py: kfac_factors, sym_inverse, kfac_cross_factors,
ekfac_materialize_factors, ekfac_precondition, fim_factors and
materialize_linear.  Three further checks need no oracle at all:
- K-FAC under a large damping is the TracIn dot over lambda^2;
- EK-FAC with the Kronecker eigenvalues as its spectrum and no damping
  preconditions exactly as K-FAC;
- token rows sum to the instance scores.

fp32 inputs.  The tight bound is 1e-4 rather than 1e-5 because the fit
inverts fp32 eigendecompositions, whose error grows with the damped
covariances' condition number (about 10 here)."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from conftest import assert_parity

import oracle

pytestmark = pytest.mark.gpu

T, K_UP, D_UP, K_DN, D_DN, D_LN = 5, 12, 10, 10, 8, 8
TIGHT = 1e-4


class Source:
    """A re-iterable ``(step, Gradient, hashes)`` source."""

    reusable = True

    def __init__(self, blocks):
        self.blocks = blocks

    def __iter__(self):
        return iter(self.blocks)


def _np(t):
    return t.double().cpu().numpy()


def _factors(gen, b):
    r = lambda *s: torch.randn(*s, generator=gen)  # noqa: E731
    return {"up": (r(b, T, K_UP), r(b, T, D_UP)), "down": (r(b, T, K_DN), r(b, T, D_DN)),
            "ln": (r(b, T, D_LN), r(b, T, D_LN))}


def _block(f, device, dense=()):
    from dattri_llm_amd.gradient import Factorized, Gradient, ops

    kw = {"up": {"has_bias": True}, "down": {"has_bias": False}, "ln": None}
    lts = {"up": "nn.Linear", "down": "nn.Linear", "ln": "nn.RMSNorm"}
    data = {n: Factorized(a.to(device), g.to(device), module_kwargs=kw[n]) for n, (a, g) in f.items()}
    for n in dense:
        data[n] = ops.materialize(data[n], lts[n])
    rep = {n: ("materialized" if isinstance(v, torch.Tensor) else "factorized") for n, v in data.items()}
    idx = {n: ("batch" if isinstance(v, torch.Tensor) else "batch_token") for n, v in data.items()}
    return Gradient(rep, data, lts, idx)


def _setup(device, dense=()):
    gen = torch.Generator().manual_seed(11)
    train_f = [_factors(gen, 6), _factors(gen, 6)]
    test_f = _factors(gen, 4)
    train = Source([(0, _block(f, device, dense), [f"r{i}-{j}" for j in range(6)]) for i, f in enumerate(train_f)])
    test = Source([(0, _block(test_f, device, dense), [f"q{j}" for j in range(4)])])
    cat = {n: tuple(np.concatenate([_np(f[n][k]) for f in train_f]) for k in (0, 1)) for n in train_f[0]}
    q = {n: (_np(test_f[n][0]), _np(test_f[n][1])) for n in test_f}
    return train, test, cat, q


def _pre(n, a, g):
    """The oracle's preprocessed factors: the ones column for the biased layer."""
    return oracle.preprocess(a, g, "nn.Linear", {"has_bias": n == "up"})


def _kfac_want(cat, q, damping, relative=False):
    total = 0.0
    for n in ("up", "down"):
        a, g = _pre(n, *cat[n])
        qa, qg = _pre(n, *q[n])
        big_a, big_g = oracle.kfac_factors(a, g)
        lam_a = damping * np.trace(big_a) / len(big_a) if relative else damping
        lam_g = damping * np.trace(big_g) / len(big_g) if relative else damping
        a_inv, g_inv = oracle.sym_inverse(big_a, lam_a), oracle.sym_inverse(big_g, lam_g)
        total = total + oracle.kfac_cross_factors(qa, qg, a, g, a_inv, g_inv).T
    return total


def _norm_dense(a, g):
    return (a * g).sum(axis=1)


@pytest.mark.parametrize("relative", [False, True])
def test_kfac_scores(device, relative):
    from dattri_llm_amd.attribution import KFACAttributor

    print(f"kfac attributor relative={relative}", flush=True)
    train, test, cat, q = _setup(device)
    score = KFACAttributor(train_batch_size=6, device=device).attribute_sources(
        train, test, damping=0.1, relative_damping=relative)
    assert score.algorithm == "KFAC" and score.scores.shape == (12, 4)
    assert score.algorithm_meta["damping"] == 0.1 and score.algorithm_meta["direct_fim_layers"] == []
    assert_parity(score.scores, _kfac_want(cat, q, 0.1, relative), torch.float32, tight=TIGHT)


def test_kfac_direct_fisher_for_norm_layers(device):
    from dattri_llm_amd.attribution import KFACAttributor

    print("kfac attributor, direct Fisher for the norm layer", flush=True)
    train, test, cat, q = _setup(device)
    score = KFACAttributor(train_batch_size=6, device=device).attribute_sources(
        train, test, damping=0.1, non_kfac_strategy="direct")
    m_tr, m_q = _norm_dense(*cat["ln"]), _norm_dense(*q["ln"])
    fisher = oracle.fim_factors(m_tr)
    f_inv = np.linalg.inv(fisher + 0.1 * np.eye(len(fisher)))
    want = _kfac_want(cat, q, 0.1) + m_tr @ f_inv @ m_q.T
    assert score.algorithm_meta["direct_fim_layers"] == ["ln"]
    assert_parity(score.scores, want, torch.float32, tight=TIGHT)


def test_materialized_linear_takes_the_direct_fisher(device):
    from dattri_llm_amd.attribution import KFACAttributor

    print("kfac attributor, materialized linear layer", flush=True)
    train, test, cat, q = _setup(device, dense=("down",))
    with pytest.warns(UserWarning, match="not preconditioned by KFAC"):
        score = KFACAttributor(train_batch_size=6, device=device).attribute_sources(train, test, damping=0.1)
    a, g = cat["up"]
    qa, qg = q["up"]
    big_a, big_g = oracle.kfac_factors(*_pre("up", a, g))
    want = oracle.kfac_cross_factors(*_pre("up", qa, qg), *_pre("up", a, g), oracle.sym_inverse(big_a, 0.1),
                                     oracle.sym_inverse(big_g, 0.1)).T
    m_tr, m_q = oracle.materialize_linear(*cat["down"]), oracle.materialize_linear(*q["down"])
    fisher = oracle.fim_factors(m_tr)
    want = want + m_tr @ np.linalg.inv(fisher + 0.1 * np.eye(len(fisher))) @ m_q.T
    assert score.algorithm_meta["direct_fim_layers"] == ["down"]
    assert_parity(score.scores, want, torch.float32, tight=TIGHT)


def test_ekfac_scores(device):
    from dattri_llm_amd.attribution import EKFACAttributor

    print("ekfac attributor", flush=True)
    train, test, cat, q = _setup(device)
    score = EKFACAttributor(train_batch_size=6, device=device, mode="approx").attribute_sources(
        train, test, damping=0.1)
    assert score.algorithm == "EKFAC" and score.algorithm_meta["mode"] == "approx"
    want = 0.0
    for n in ("up", "down"):
        a, g = _pre(n, *cat[n])
        qa, qg = _pre(n, *q[n])
        big_a, big_g = oracle.kfac_factors(a, g)
        u_a, u_g = np.linalg.eigh(big_a)[1], np.linalg.eigh(big_g)[1]
        lam = (oracle.ekfac_materialize_factors(a, g, u_a, u_g) ** 2).mean(axis=0)
        pre_q = oracle.ekfac_precondition(oracle.ekfac_materialize_factors(qa, qg, u_a, u_g), u_a, u_g, lam + 0.1)
        want = want + oracle.materialize_linear(a, g) @ pre_q.T
    assert_parity(score.scores, want, torch.float32, tight=TIGHT)


def test_kfac_large_damping_is_tracin_over_lambda_squared(device):
    from dattri_llm_amd.attribution import KFACAttributor, TracInAttributor

    print("kfac attributor, damping 1e4", flush=True)
    train, test, _cat, _q = _setup(device)
    lam = 1e4
    kfac = KFACAttributor(train_batch_size=6, device=device).attribute_sources(train, test, damping=lam)
    lin = Source([(s, b.select_layers(["up", "down"]), h) for s, b, h in train.blocks])
    lin_q = Source([(s, b.select_layers(["up", "down"]), h) for s, b, h in test.blocks])
    dot = TracInAttributor(train_batch_size=6, device=device).attribute_sources(lin, lin_q)
    # (A + lam)^-1 = I/lam (1 - A/lam + ...): the first-order term is ~ |A|/lam ~ 1e-3 of the score
    got, want = _np(kfac.scores) * lam * lam, _np(dot.scores)
    assert np.linalg.norm(got - want) <= 5e-3 * np.linalg.norm(want)


def test_ekfac_with_kronecker_spectrum_is_kfac(device):
    from dattri_llm_amd.attribution import EKFACAttributor, KFACAttributor
    from dattri_llm_amd.gradient import ops

    print("ekfac with the Kronecker eigenvalues == kfac", flush=True)
    train, test, _cat, _q = _setup(device)
    kf = KFACAttributor(device=device)
    raw = kf.fit(train)[0]
    ek = EKFACAttributor(device=device)
    ek_raw = {}
    for n, (big_a, big_g) in raw.items():
        s_a, u_a, s_g, u_g = ops.kfac_eigh(big_a, big_g)
        ek_raw[n] = (u_a, u_g, torch.outer(s_g, s_a).flatten())
    kf_pre, _ = kf.damp_fit((raw, {}), 0.0)
    ek_pre, _ = ek.damp_fit((ek_raw, {}), 0.0)
    query = test.blocks[0][1]
    for n in raw:
        k_side = kf.precondition_test_layer(query.data[n], "nn.Linear", kf_pre[n])
        e_side = ek.precondition_test_layer(query.data[n], "nn.Linear", ek_pre[n])
        k_dense = ops.materialize(k_side, "nn.Linear")
        assert_parity(e_side, k_dense, torch.float32, tight=TIGHT, label=n)


def test_fit_reuse_and_token_rows(device):
    from dattri_llm_amd.attribution import KFACAttributor

    print("kfac attributor, reused fit and token granularity", flush=True)
    train, test, cat, q = _setup(device)
    attr = KFACAttributor(train_batch_size=6, device=device)
    raw = attr.fit(train)
    for damping in (0.1, 1.0):
        reused = attr.attribute_sources(train, test, damping=damping, raw_fit=raw)
        assert_parity(reused.scores, _kfac_want(cat, q, damping), torch.float32, tight=TIGHT, label=str(damping))
    tok = attr.attribute_sources(train, test, damping=0.1, raw_fit=raw, attribution_granularity="token")
    assert tok.granularity == "token" and tok.scores.shape == (12 * T, 4)
    _ids, summed = tok.agnostic_matrix()
    assert_parity(summed, _kfac_want(cat, q, 0.1), torch.float32, tight=TIGHT, label="token rows")
    looped = attr.attribute_sources(train, test, damping=0.1, raw_fit=raw, loop_over_test=True)
    assert_parity(looped.scores, _kfac_want(cat, q, 0.1), torch.float32, tight=TIGHT, label="loop_over_test")


def test_dense_query_matches_factorized_query(device):
    """A query stored materialized takes the two-sided dense product and scores
    as the factorized query does (test_kronecker.py:395-419)."""
    from dattri_llm_amd.attribution import EKFACAttributor, KFACAttributor

    print("kfac/ekfac attributors, dense query side", flush=True)
    train, test, _cat, _q = _setup(device)
    _tr, dense_test, _c, _qq = _setup(device, dense=("up", "down"))
    for cls in (KFACAttributor, EKFACAttributor):
        attr = cls(train_batch_size=6, device=device)
        raw = attr.fit(train)
        fact = attr.attribute_sources(train, test, damping=0.1, raw_fit=raw)
        dense = attr.attribute_sources(train, dense_test, damping=0.1, raw_fit=raw)
        assert_parity(dense.scores, fact.scores, torch.float32, tight=TIGHT, label=cls.__name__)


def test_fisher_cap_skips_a_layer_with_a_warning(device):
    from dattri_llm_amd.attribution import KFACAttributor

    print("kfac attributor, direct Fisher cap", flush=True)
    train, test, cat, q = _setup(device)
    with pytest.warns(UserWarning, match="direct_fim_max_params=4"):
        score = KFACAttributor(train_batch_size=6, device=device).attribute_sources(
            train, test, damping=0.1, non_kfac_strategy="direct", direct_fim_max_params=4)
    assert score.algorithm_meta["direct_fim_layers"] == []
    assert_parity(score.scores, _kfac_want(cat, q, 0.1), torch.float32, tight=TIGHT)


def test_norm_only_scores_the_direct_fisher(device):
    from dattri_llm_amd.attribution import EKFACAttributor, KFACAttributor

    print("kfac/ekfac attributors, norm layer only", flush=True)
    train, test, cat, q = _setup(device)
    only = lambda src: Source([(s, b.select_layers(["ln"]), h) for s, b, h in src.blocks])  # noqa: E731
    m_tr, m_q = _norm_dense(*cat["ln"]), _norm_dense(*q["ln"])
    fisher = oracle.fim_factors(m_tr)
    want = m_tr @ np.linalg.inv(fisher + 0.1 * np.eye(len(fisher))) @ m_q.T
    for cls in (KFACAttributor, EKFACAttributor):
        score = cls(train_batch_size=6, device=device).attribute_sources(
            only(train), only(test), damping=0.1, non_kfac_strategy="direct")
        assert_parity(score.scores, want, torch.float32, tight=TIGHT, label=cls.__name__)


def test_ekfac_heavy_damping_is_the_gradient_dot(device):
    """(lambda_raw + lam)^-1 = 1/lam (1 - lambda_raw/lam + ...)
    (test_kronecker.py:252-286)."""
    from dattri_llm_amd.attribution import EKFACAttributor, TracInAttributor

    print("ekfac attributor, damping 1e4", flush=True)
    train, test, _cat, _q = _setup(device)
    lam = 1e4
    ek = EKFACAttributor(train_batch_size=6, device=device).attribute_sources(train, test, damping=lam)
    lin = lambda src: Source([(s, b.select_layers(["up", "down"]), h) for s, b, h in src.blocks])  # noqa: E731
    dot = TracInAttributor(train_batch_size=6, device=device).attribute_sources(lin(train), lin(test))
    got, want = _np(ek.scores) * lam, _np(dot.scores)
    assert np.linalg.norm(got - want) <= 5e-3 * np.linalg.norm(want)


def _conv_expected(case, train_in, query_in, kind, damping):
    """K-FAC / EK-FAC scores of one convolution layer from the oracle's
    preprocessed factors, group by group.  Both are symmetric in the two
    factors' roles, so one rule covers convolutions and transposed ones."""
    transpose, _rank, _ci, _co, k, s, p, d, groups, bias, _sp = case
    pre = [oracle.conv_preprocess(x, g, transpose, k, s, p, d, groups, bias) for x, g in train_in]
    a, f = np.concatenate([x for x, _ in pre]), np.concatenate([g for _, g in pre])
    qa, qf = oracle.conv_preprocess(*query_in, transpose, k, s, p, d, groups, bias)
    assert not (f == 0).all(-1).any()  # no gradient-free rows: the oracle's drop rule is moot
    parts = ([(a[:, :, i], f[:, :, i], qa[:, :, i], qf[:, :, i]) for i in range(groups)] if a.ndim == 4
             else [(a, f, qa, qf)])
    total = 0.0
    for pa, pf, pqa, pqf in parts:
        big_a, big_g = oracle.kfac_factors(pa, pf)
        if kind == "kfac":
            total = total + oracle.kfac_cross_factors(pqa, pqf, pa, pf, oracle.sym_inverse(big_a, damping),
                                                      oracle.sym_inverse(big_g, damping)).T
        else:
            u_a, u_g = np.linalg.eigh(big_a)[1], np.linalg.eigh(big_g)[1]
            lam = (oracle.ekfac_materialize_factors(pa, pf, u_a, u_g) ** 2).mean(axis=0)
            pre_q = oracle.ekfac_precondition(oracle.ekfac_materialize_factors(pqa, pqf, u_a, u_g), u_a, u_g,
                                              lam + damping)
            total = total + oracle.materialize_linear(pa, pf) @ pre_q.T
    return total


@pytest.mark.parametrize("kind", ["kfac", "ekfac"])
@pytest.mark.parametrize("case", range(7))
def test_convolution_layers(device, case, kind):
    """Convolutions, transposed convolutions, grouped and depthwise ones
    (the K-FAC family's conv support, kronecker.py:638-659 via ops)."""
    from test_oracle import CONV_CASES, conv_inputs

    from dattri_llm_amd.attribution import EKFACAttributor, KFACAttributor
    from dattri_llm_amd.gradient import Factorized, Gradient

    conv = CONV_CASES[case]
    transpose, rank, _ci, _co, k, s, p, d, groups, bias, _sp = conv
    print(f"{kind} attributor, conv case {conv}", flush=True)
    lt = {(False, 1): "nn.Conv1d", (False, 2): "nn.Conv2d", (False, 3): "nn.Conv3d",
          (True, 1): "nn.ConvTranspose1d", (True, 2): "nn.ConvTranspose2d"}[(transpose, rank)]
    mk = {"has_bias": bias, "kernel_size": k, "stride": s, "padding": p, "dilation": d, "groups": groups}
    train_in = [conv_inputs(conv, n=3, seed=60), conv_inputs(conv, n=3, seed=62)]
    query_in = conv_inputs(conv, n=2, seed=61)

    def block(x, g):
        data = {"conv": Factorized(torch.from_numpy(x).float().to(device), torch.from_numpy(g).float().to(device),
                                   module_kwargs=mk)}
        return Gradient({"conv": "factorized"}, data, {"conv": lt}, {"conv": "batch_token"})

    # the oracle sees the fp32-rounded inputs the kernels read
    rounded = lambda xg: tuple(v.astype(np.float32).astype(np.float64) for v in xg)  # noqa: E731
    train = Source([(0, block(*xg), [f"r{i}-{j}" for j in range(3)]) for i, xg in enumerate(train_in)])
    test = Source([(0, block(*query_in), ["q0", "q1"])])
    cls = KFACAttributor if kind == "kfac" else EKFACAttributor
    score = cls(train_batch_size=3, device=device).attribute_sources(train, test, damping=0.1)
    want = _conv_expected(conv, [rounded(xg) for xg in train_in], rounded(query_in), kind, 0.1)
    assert score.scores.shape == (6, 2)
    assert_parity(score.scores, want, torch.float32, tight=TIGHT)
