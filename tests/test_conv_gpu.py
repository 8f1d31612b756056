"""GPU parity of the convolution family (Conv1d/2d/3d, ConvTranspose1d/2d,
grouped, with bias) through the ops layer, against the oracle's unfolding
(pinned against autograd in tests/test_oracle.py).

The unfolding is layout work on the device; every product runs on the linear
kernels (ghost, grouped ghost, dW, score GEMM, per-token).  Bars:
conftest.assert_parity; results rounded to bf16 on the way (bf16 operands, a
transposed convolution's bias sums, a bf16 dense side) widen the tight bound
by one half-ulp each.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_parity, roundings
from test_oracle import CONV_CASES, conv_inputs

pytestmark = pytest.mark.gpu

_NAMES = {(False, 1): "nn.Conv1d", (False, 2): "nn.Conv2d", (False, 3): "nn.Conv3d",
          (True, 1): "nn.ConvTranspose1d", (True, 2): "nn.ConvTranspose2d"}


def _setup(case, dtype):
    transpose, rank, _ci, _co, k, s, p, d, groups, bias, _sp = case
    lt = _NAMES[(transpose, rank)]
    mk = {"has_bias": bias, "kernel_size": k, "stride": s, "padding": p, "dilation": d, "groups": groups}
    x1, g1 = conv_inputs(case, n=3, seed=60)
    x2, g2 = conv_inputs(case, n=2, seed=61)
    raw = [torch.from_numpy(v).to(dtype) for v in (x1, g1, x2, g2)]
    ref_in = [r.double().numpy() for r in raw]  # the oracle sees the rounded inputs
    a1, f1 = oracle.conv_preprocess(ref_in[0], ref_in[1], transpose, k, s, p, d, groups, bias)
    a2, f2 = oracle.conv_preprocess(ref_in[2], ref_in[3], transpose, k, s, p, d, groups, bias)
    return lt, mk, raw, (a1, f1, a2, f2), transpose


def _tight(dtype, n):
    return roundings(n) if dtype == torch.bfloat16 else None


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_ops_match_oracle(device, dtype, case):
    from dattri_llm_amd.gradient import ops

    lt, mk, raw, (a1, f1, a2, f2), transpose = _setup(case, dtype)
    print(f"conv case={case} dtype={dtype}", flush=True)
    x1, g1, x2, g2 = (t.to(device) for t in raw)
    m1_ref, m2_ref = oracle.conv_materialize(a1, f1, transpose), oracle.conv_materialize(a2, f2, transpose)
    grouped = a1.ndim == 4

    m1 = ops.materialize_factors(x1, g1, lt, module_kwargs=mk)
    assert m1.shape == m1_ref.shape and m1.dtype == dtype
    assert_parity(m1, m1_ref, dtype, tight=_tight(dtype, 2), label="materialize")

    gram_ref = m1_ref @ m2_ref.T
    for mode in ("factorized", "materialized", "auto"):
        got = ops.cross_dot_factors(x1, g1, x2, g2, lt, mk, mk, mode=mode)
        assert_parity(got, gram_ref, dtype, tight=_tight(dtype, 2), label=f"cross {mode}")
    for mode in ("factorized", "materialized"):
        sq = ops.grad_norm_sq_factors(x1, g1, lt, module_kwargs=mk, mode=mode)
        assert_parity(sq, (m1_ref * m1_ref).sum(-1), dtype, tight=_tight(dtype, 2), label=f"norm {mode}")
    dots = ops.dot_factors(x1[:2], g1[:2], x2, g2, lt, mk, mk)
    assert_parity(dots, (m1_ref[:2] * m2_ref).sum(-1), dtype, tight=_tight(dtype, 2), label="dot")

    # cross_gram on the preprocessed factors (3-D, or 4-D with the group axis)
    pre = [torch.from_numpy(v).to(dtype).to(device) for v in (a1, f1, a2, f2)]
    assert_parity(ops.cross_gram(*pre, lt), gram_ref, dtype, tight=_tight(dtype, 2), label="cross_gram")

    # per-token: side 1's locations against side 2 (factorized, then dense)
    if grouped:
        pt_ref = oracle.grouped_cross_gram_per_token(a1, f1, a2, f2)
    else:
        pt_ref = oracle.cross_gram_per_token(a1, f1, a2, f2)
    from dattri_llm_amd.gradient.gradient import Factorized

    fa = Factorized(activation=x1, pre_activation_grad=g1, module_kwargs=mk)
    fb = Factorized(activation=x2, pre_activation_grad=g2, module_kwargs=mk)
    pt = ops.cross_dot_per_token(fa, fb, lt)
    assert pt.shape == pt_ref.shape
    assert_parity(pt, pt_ref, dtype, tight=_tight(dtype, 2), label="per_token")
    assert_parity(ops.cross_gram_per_token(*pre, lt), pt_ref, dtype, tight=_tight(dtype, 2), label="per_token pre")
    m2 = ops.materialize_factors(x2, g2, lt, module_kwargs=mk)
    assert_parity(ops.cross_dot_per_token(fa, m2, lt), pt_ref, dtype, tight=_tight(dtype, 3),
                  label="per_token dense")
    assert_parity(ops.cross_gram_per_token_dense(pre[0], pre[1], m2, lt), pt_ref, dtype, tight=_tight(dtype, 3),
                  label="per_token_dense pre")


def test_conv_layerwise_block(device):
    """A block mixing a grouped Conv2d, a ConvTranspose1d and a linear layer
    through layerwise_cross_dot (the scoring entry point)."""
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    cases = {"conv": CONV_CASES[1], "convt": CONV_CASES[4]}
    reps, ref = [], 0.0
    for side, n, seed in ((0, 3, 70), (1, 2, 71)):
        data, types, rep_ = {}, {}, {}
        for name, case in cases.items():
            transpose, rank, _ci, _co, k, s, p, d, groups, bias, _sp = case
            lt = _NAMES[(transpose, rank)]
            mk = {"has_bias": bias, "kernel_size": k, "stride": s, "padding": p, "dilation": d, "groups": groups}
            x, g = conv_inputs(case, n=n, seed=seed)
            data[name] = Factorized(torch.from_numpy(x).float().to(device), torch.from_numpy(g).float().to(device),
                                    module_kwargs=mk)
            types[name] = lt
            a, f = oracle.conv_preprocess(x, g, transpose, k, s, p, d, groups, bias)
            rep_[name] = oracle.conv_materialize(a, f, transpose)
        gen = np.random.default_rng(seed)
        la, lg = gen.standard_normal((n, 5, 16)), gen.standard_normal((n, 5, 8))
        data["lin"] = Factorized(torch.from_numpy(la).float().to(device), torch.from_numpy(lg).float().to(device))
        types["lin"] = "nn.Linear"
        rep_["lin"] = oracle.materialize_linear(la, lg)
        reps.append((Gradient({k: "factorized" for k in data}, data, types), rep_))
    (tr, tr_ref), (te, te_ref) = reps
    ref = sum(tr_ref[k] @ te_ref[k].T for k in tr_ref)
    assert_parity(ops.layerwise_cross_dot(tr, te), ref, torch.float32, label="layerwise")
