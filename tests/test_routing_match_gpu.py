"""GPU parity of the routed-row location (``da_match_rows``, the drop-in for
RoutedTokenTracker._match, routing.py:300-333) against the oracle, at small
sizes and at the Mixtral-shaped block (16 x 256 tokens, d = 4096, top-2 of 8
experts, rows gathered as fused_experts.py:219-228 does)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_match_rows_small_cases(device, dtype):
    from dattri_llm_amd import kernels

    gen = torch.Generator().manual_seed(5)
    src = torch.randn(40, 24, generator=gen).to(dtype)
    src[7] = src[3]
    src[19] = src[3]
    src[30] = -0.0 * src[30]  # signed zeros stay distinct values of the fingerprint
    cases = [
        [1, 3, 7, 8, 19, 22],       # ascending gather
        [3, 5, 3, 3],               # one value three times
        list(range(40)),            # identity
        [39, 0, 20, 3, 10, 3],      # unordered, repeated
    ]
    for rows in cases:
        x = src[rows]
        want = oracle.match_rows(x.float().numpy(), src.float().numpy())
        got = kernels.match_rows(src.to(device), x.to(device))
        assert got is not None and np.array_equal(got.cpu().numpy(), want), rows
    assert kernels.match_rows(src.to(device), src[[3, 3, 3, 3]].to(device)) is None
    other = torch.randn(2, 24, generator=gen).to(dtype)
    assert kernels.match_rows(src.to(device), other.to(device)) is None
    nan_src = src.clone()
    nan_src[2, 1] = float("nan")
    assert kernels.match_rows(nan_src.to(device), nan_src[[2]].to(device)) is None
    # width not a multiple of a 16-byte chunk: zero-padded copies, same answer
    odd = torch.randn(12, 5, generator=gen).to(dtype)
    got = kernels.match_rows(odd.to(device), odd[[4, 2, 11]].to(device))
    assert np.array_equal(got.cpu().numpy(), [4, 2, 11])


def test_match_rows_mixtral_block(device):
    from dattri_llm_amd.gradient.ops import moe
    from dattri_llm_amd.gradient.routing import locate_rows

    b, t, d, n_exp, k = 16, 256, 4096, 8, 2
    gen = torch.Generator().manual_seed(6)
    hidden = torch.randn(b, t, d, generator=gen).to(torch.bfloat16)
    hidden[5] = hidden[4]          # a repeated sample: every row of it appears twice
    hidden[9, 100:] = hidden[8, 100:]  # a shared suffix
    flat = hidden.reshape(b * t, d)
    logits = torch.randn(b * t, n_exp, generator=gen)
    _w, idx = moe.router_topk(logits.to(device), k)
    mask = torch.nn.functional.one_hot(idx.cpu(), n_exp).permute(2, 1, 0)  # (E, k, B*T)
    flat_d = flat.to(device)
    print("match_rows Mixtral block", flush=True)
    for e in range(n_exp):
        _slot, tok = torch.where(mask[e])
        x = flat[tok]
        want = oracle.match_rows(x.float().numpy(), flat.float().numpy())
        layout = locate_rows(x.to(device), flat_d, b, t)
        assert layout is not None and want is not None
        got = (layout.sample * t + layout.position).cpu().numpy()
        assert np.array_equal(got, want), e
        # the regroup scatters the rows back to (B, T, d), zeros elsewhere
        rows = torch.randn(x.shape[0], 8, generator=gen)
        dense = layout.regroup(rows.to(device)).cpu().numpy()
        ref = oracle.moe_regroup_dense(rows.numpy(), want, b, t)
        assert np.array_equal(dense, ref)
    ident = locate_rows(flat_d, flat_d, b, t)
    assert ident is not None and ident.sample is None


def test_locate_rows_signed_zero(device):
    """The block's own rows match by float equality (routing.py:303-304);
    gathered rows match by their bits (routing.py:335-340), so a zero of the
    other sign finds no token."""
    from dattri_llm_amd.gradient.routing import locate_rows

    gen = torch.Generator().manual_seed(8)
    src = torch.randn(4 * 8, 16, generator=gen).to(torch.bfloat16)
    src[5, 3] = 0.0
    x = src.clone()
    x[5, 3] = -0.0
    ident = locate_rows(x.to(device), src.to(device), 4, 8)
    assert ident is not None and ident.sample is None
    assert locate_rows(x[[5, 2]].to(device), src.to(device), 4, 8) is None
    part = locate_rows(src[[5, 2]].to(device), src.to(device), 4, 8)
    assert part is not None and part.sample.tolist() == [0, 0] and part.position.tolist() == [5, 2]
