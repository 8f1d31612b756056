"""GPU parity of the fused ghost cross-gram (K1) against the oracle.

Bar: normwise relative error (max|got-ref| / max|ref|) <= 1e-2 for bf16/fp16
inputs with fp32 accumulation, <= 1e-3 for fp32 inputs; the oracle runs in
float64 on the same (already rounded) inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: 1e-2, torch.float16: 1e-2, torch.float32: 1e-3}


def _inputs(seed, b1, s1, b2, s2, k, d, dtype, scale=True):
    gen = torch.Generator().manual_seed(seed)
    def rnd(*shape, width):
        x = torch.randn(*shape, generator=gen)
        return (x / width**0.5 if scale else x).to(dtype)
    return (rnd(b1, s1, k, width=k), rnd(b1, s1, d, width=d),
            rnd(b2, s2, k, width=k), rnd(b2, s2, d, width=d))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [32, 16])
def test_mfma_lane_layout(device, dtype, shape):
    """The MFMA operand/accumulator conventions every kernel relies on."""
    from dattri_llm_amd import kernels

    chunk = 8 if dtype == torch.float32 else 16  # elements per 32 bytes
    rows, k = (32, chunk) if shape == 32 else (16, 2 * chunk)
    gen = torch.Generator().manual_seed(1)
    # small integers: every product and sum is exact in fp32
    a = torch.randint(-4, 5, (rows, k), generator=gen).to(dtype)
    b = torch.randint(-4, 5, (rows, k), generator=gen).to(dtype)
    raw = kernels.selftest_mfma(dtype, a.to(device), b.to(device), shape=shape).cpu()
    c = a.double() @ b.double().T
    lane = torch.arange(64)[:, None]
    if shape == 32:
        r = torch.arange(16)[None, :]
        rows_idx = 8 * (r // 4) + 4 * (lane // 32) + (r % 4)
        cols_idx = (lane % 32).expand(64, 16)
    else:
        r = torch.arange(4)[None, :]
        rows_idx = 4 * (lane // 16) + r
        cols_idx = (lane % 16).expand(64, 4)
    assert torch.equal(raw.double(), c[rows_idx, cols_idx])


CASES = [
    # (b1, s1, b2, s2, k, d, bias)
    (3, 128, 2, 128, 64, 64, False),
    (4, 96, 3, 200, 72, 40, True),       # ragged S, S1 != S2, K/D not multiples of 64
    (2, 300, 5, 17, 128, 256, True),
    (1, 1, 1, 1, 8, 8, False),           # single token
    (5, 64, 4, 64, 136, 48, False),
    (2, 257, 2, 129, 520, 264, True),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", CASES)
def test_ghost_gram_matches_oracle(device, dtype, case):
    from dattri_llm_amd import kernels

    b1, s1, b2, s2, k, d, bias = case
    a1, g1, a2, g2 = _inputs(hash(case) % 1000, b1, s1, b2, s2, k, d, dtype)
    print(f"ghost_gram case={case} dtype={dtype}", flush=True)
    got = kernels.ghost_gram(*(x.to(device) for x in (a1, g1, a2, g2)), bias=bias)
    ref = oracle.cross_gram_factorized(*(x.double().numpy() for x in (a1, g1, a2, g2)), bias=bias)
    assert got.shape == (b1, b2)
    assert rel_err(got.cpu().numpy(), ref) <= TOL[dtype]


def test_ghost_gram_accumulate_and_strided_out(device):
    from dattri_llm_amd import kernels

    a1, g1, a2, g2 = (x.to(device) for x in _inputs(7, 3, 64, 4, 80, 64, 32, torch.bfloat16))
    big = torch.zeros(3, 10, dtype=torch.float32, device=device)
    view = big[:, 2:6]
    kernels.ghost_gram(a1, g1, a2, g2, out=view)
    kernels.ghost_gram(a1, g1, a2, g2, out=view, accumulate=True)
    ref = oracle.cross_gram_factorized(*(x.double().cpu().numpy() for x in (a1, g1, a2, g2)))
    assert rel_err(view.cpu().numpy(), 2 * ref) <= 1e-2
    assert torch.count_nonzero(big[:, :2]) == 0 and torch.count_nonzero(big[:, 6:]) == 0


def test_ghost_gram_non_contiguous_views(device):
    """Sequence-first captures transposed to batch-first are strided views."""
    from dattri_llm_amd import kernels

    a1, g1, a2, g2 = _inputs(11, 3, 40, 2, 56, 64, 64, torch.bfloat16)
    t = [x.transpose(0, 1).contiguous().to(device).transpose(0, 1) for x in (a1, g1, a2, g2)]
    got = kernels.ghost_gram(*t)
    ref = oracle.cross_gram_factorized(*(x.double().numpy() for x in (a1, g1, a2, g2)))
    assert rel_err(got.cpu().numpy(), ref) <= 1e-2


def test_ghost_gram_c2_subset_pairs(device):
    """Full C2 geometry (T=512, d=4096) on a slice of the batch: 8 train x 4
    query pairs checked exactly against the float64 oracle."""
    from dattri_llm_amd import kernels

    a1, g1, a2, g2 = _inputs(2, 8, 512, 4, 512, 4096, 4096, torch.bfloat16)
    got = kernels.ghost_gram(*(x.to(device) for x in (a1, g1, a2, g2)))
    ref = oracle.cross_gram_factorized(*(x.double().numpy() for x in (a1, g1, a2, g2)))
    assert rel_err(got.cpu().numpy(), ref) <= 1e-2
