"""GPU parity of the channel norms (GroupNorm, InstanceNorm) against the oracle
(norm.py:44-62, :120-141; pinned against autograd in tests/test_oracle.py):
the fused statistics + weight-gradient kernel, the x_hat kernel behind
preprocess_factors, and the ops that route through them."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import HALF_ULP, SPEC_BAR, TIGHT_FP32, assert_parity, roundings, stable_seed

pytestmark = pytest.mark.gpu

CASES = [
    # (layer_type, n, c, spatial, groups, bias)
    ("nn.GroupNorm", 3, 8, (5, 7), 4, True),
    ("nn.GroupNorm", 2, 6, (33,), 2, False),
    ("nn.InstanceNorm2d", 3, 4, (6, 6), 4, True),
    ("nn.InstanceNorm1d", 2, 5, (301,), 5, False),
    ("nn.GroupNorm", 2, 64, (24, 24), 32, True),   # wide groups: 1152 values per block
]


def _mk(layer_type, c, groups, bias):
    mk = {"has_bias": bias, "eps": 1e-5}
    if layer_type == "nn.GroupNorm":
        mk.update(num_groups=groups, num_channels=c)
    else:
        mk.update(num_features=c)
    return mk


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", CASES)
def test_channel_norm_ops(device, dtype, case):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized

    lt, n, c, sp, groups, bias = case
    mk = _mk(lt, c, groups, bias)
    gen = torch.Generator().manual_seed(stable_seed(case))
    raw = [(torch.randn(b, c, *sp, generator=gen) * 1.5 + 0.5).to(dtype) for b in (n, n - 1)]
    grads = [torch.randn(b, c, *sp, generator=gen).to(dtype) for b in (n, n - 1)]
    print(f"channel norm case={case} dtype={dtype}", flush=True)
    refs = [oracle.channel_norm_preprocess(x.double().numpy(), g.double().numpy(), groups, 1e-5, bias)
            for x, g in zip(raw, grads)]
    dense = [(a * g).sum(axis=1) for a, g in refs]
    x1, g1, x2, g2 = raw[0].to(device), grads[0].to(device), raw[1].to(device), grads[1].to(device)
    tight = roundings(1) if dtype == torch.bfloat16 else None

    m1 = ops.materialize_factors(x1, g1, lt, module_kwargs=mk)
    assert m1.shape == dense[0].shape and m1.dtype == dtype
    assert_parity(m1, dense[0], dtype, tight=tight, label="materialize")
    a_p, g_p = ops.preprocess_factors(x1, g1, lt, mk)
    assert a_p.shape == refs[0][0].shape
    assert_parity(a_p, refs[0][0], dtype, tight=tight, label="x_hat")
    assert torch.equal(g_p.cpu(), torch.from_numpy(refs[0][1]).to(dtype))
    gram = ops.cross_dot_factors(x1, g1, x2, g2, lt, mk, mk)
    assert_parity(gram, dense[0] @ dense[1].T, dtype, tight=tight, label="cross")
    assert_parity(ops.grad_norm_sq_factors(x1, g1, lt, mk), (dense[0] ** 2).sum(-1), dtype, tight=tight,
                  label="norm")
    # A per-sample dot of two C-wide rows may cancel: its error is measured
    # against |row1| |row2| (the Cauchy-Schwarz scale of the sum), not |dot|.
    dot = ops.dot_factors(x1[:n - 1], g1[:n - 1], x2, g2, lt, mk, mk)
    assert dot.dtype == dtype
    ref_dot = (dense[0][:n - 1] * dense[1]).sum(-1)
    scale = np.linalg.norm(dense[0][:n - 1], axis=-1) * np.linalg.norm(dense[1], axis=-1)
    dot_err = float(np.max(np.abs(dot.double().cpu().numpy() - ref_dot) / scale))
    name = str(dtype).replace("torch.", "")
    assert dot_err <= SPEC_BAR[name], f"dot error {dot_err:.3e} above the spec bar"
    assert dot_err <= TIGHT_FP32 + HALF_ULP.get(name, 0.0), f"dot error {dot_err:.3e} above the tight bound"
    # per-token: positions of side 1 against side 2 (factorized, then dense)
    rows_ref = refs[0][0] * refs[0][1]
    pt_ref = np.einsum("bsd,cd->bsc", rows_ref, dense[1])
    f1 = Factorized(x1, g1, module_kwargs=mk)
    f2 = Factorized(x2, g2, module_kwargs=mk)
    tight_pt = roundings(3) if dtype == torch.bfloat16 else None  # x_hat, the row product, the output
    assert_parity(ops.cross_dot_per_token(f1, f2, lt), pt_ref, dtype, tight=tight_pt, label="per_token")
    m2 = ops.materialize_factors(x2, g2, lt, module_kwargs=mk)
    assert_parity(ops.cross_dot_per_token(f1, m2, lt), pt_ref, dtype, tight=tight_pt, label="per_token dense")
    per_tok = ops.materialize_factors(x1, g1, lt, module_kwargs=mk, per_token=True)
    assert_parity(per_tok, rows_ref.reshape(n, -1), dtype, tight=roundings(2) if dtype == torch.bfloat16 else None,
                  label="per_token rows")
