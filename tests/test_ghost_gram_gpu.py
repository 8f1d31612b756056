"""GPU parity of the fused ghost cross-gram (K1) against the oracle.

Bars (conftest.assert_parity): normwise relative error (max|got-ref| /
max|ref|) <= 1e-2 for bf16/fp16 inputs with fp32 accumulation, <= 1e-3 for
fp32 inputs, and a tight 1e-5 for what fp32 accumulation leaves against the
float64 oracle on the same (already rounded) inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_parity, stable_seed

pytestmark = pytest.mark.gpu



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
    a1, g1, a2, g2 = _inputs(stable_seed(case), b1, s1, b2, s2, k, d, dtype)
    print(f"ghost_gram case={case} dtype={dtype}", flush=True)
    got = kernels.ghost_gram(*(x.to(device) for x in (a1, g1, a2, g2)), bias=bias)
    ref = oracle.cross_gram_factorized(*(x.double().numpy() for x in (a1, g1, a2, g2)), bias=bias)
    assert got.shape == (b1, b2)
    assert_parity(got, ref, dtype)


def test_ghost_gram_accumulate_and_strided_out(device):
    from dattri_llm_amd import kernels

    a1, g1, a2, g2 = (x.to(device) for x in _inputs(7, 3, 64, 4, 80, 64, 32, torch.bfloat16))
    big = torch.zeros(3, 10, dtype=torch.float32, device=device)
    view = big[:, 2:6]
    kernels.ghost_gram(a1, g1, a2, g2, out=view)
    kernels.ghost_gram(a1, g1, a2, g2, out=view, accumulate=True)
    ref = oracle.cross_gram_factorized(*(x.double().cpu().numpy() for x in (a1, g1, a2, g2)))
    assert_parity(view, 2 * ref, torch.bfloat16)
    assert torch.count_nonzero(big[:, :2]) == 0 and torch.count_nonzero(big[:, 6:]) == 0


def test_ghost_gram_non_contiguous_views(device):
    """Sequence-first captures transposed to batch-first are strided views."""
    from dattri_llm_amd import kernels

    a1, g1, a2, g2 = _inputs(11, 3, 40, 2, 56, 64, 64, torch.bfloat16)
    t = [x.transpose(0, 1).contiguous().to(device).transpose(0, 1) for x in (a1, g1, a2, g2)]
    got = kernels.ghost_gram(*t)
    ref = oracle.cross_gram_factorized(*(x.double().numpy() for x in (a1, g1, a2, g2)))
    assert_parity(got, ref, torch.bfloat16)


def test_ghost_gram_c2_subset_pairs(device):
    """Full C2 geometry (T=512, d=4096) on a slice of the batch: 8 train x 4
    query pairs checked exactly against the float64 oracle."""
    from dattri_llm_amd import kernels

    a1, g1, a2, g2 = _inputs(2, 8, 512, 4, 512, 4096, 4096, torch.bfloat16)
    got = kernels.ghost_gram(*(x.to(device) for x in (a1, g1, a2, g2)))
    ref = oracle.cross_gram_factorized(*(x.double().numpy() for x in (a1, g1, a2, g2)))
    assert_parity(got, ref, torch.bfloat16)


# ---------------------------------------------------------------------------
# Grouped (MoE) form: packed expert rows, per-sample bins
# ---------------------------------------------------------------------------


def _rand(gen, *shape, dtype):
    return (torch.randn(*shape, generator=gen) / 4).to(dtype)


def _np(x):
    return x.double().cpu().numpy()


def _grouped_case(device, dtype, bias, n_exp, seed):
    """Experts with edge-case routing: one takes every token of side 1 (300-row
    samples span three tiles), one is empty, one sees a single sample, the rest
    a random 30%; rows arrive in a shuffled (routed) order."""
    from dattri_llm_amd.gradient import ops

    gen = torch.Generator().manual_seed(seed)
    b1, b2, tokens, k, d = 5, 3, 300, 64, 96
    groups1, groups2, ref = [], [], np.zeros((b1, b2))
    for e in range(n_exp):
        def pick(batch, side):
            flat = torch.arange(batch * tokens)
            if e == 0 and side == 1:
                keep = flat
            elif e == 1:
                keep = flat[:0]
            elif e == 2:
                keep = flat[(flat // tokens) == (batch - 1)]
            else:
                keep = flat[torch.rand(batch * tokens, generator=gen) < 0.3]
            return keep[torch.randperm(keep.numel(), generator=gen)]

        tok1, tok2 = pick(b1, 1), pick(b2, 2)
        a1, g1 = _rand(gen, tok1.numel(), k, dtype=dtype), _rand(gen, tok1.numel(), d, dtype=dtype)
        a2, g2 = _rand(gen, tok2.numel(), k, dtype=dtype), _rand(gen, tok2.numel(), d, dtype=dtype)
        ref += oracle.moe_segment_ghost(_np(a1), _np(g1), tok1.numpy(), _np(a2), _np(g2), tok2.numpy(),
                                        b1, b2, tokens, tokens, bias=bias)
        seg1, rows1 = ops.moe.segment_by_sample(tok1.to(device), b1, tokens)
        seg2, rows2 = ops.moe.segment_by_sample(tok2.to(device), b2, tokens)
        groups1.append((a1.to(device), g1.to(device), seg1, rows1))
        groups2.append((a2.to(device), g2.to(device), seg2, rows2))
    return groups1, groups2, ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("n_exp", [4, 11])  # 11 > 8 experts per launch: two launches
def test_ghost_gram_grouped(device, dtype, bias, n_exp):
    from dattri_llm_amd import kernels

    print(f"grouped dtype={dtype} bias={bias} n_exp={n_exp}", flush=True)
    groups1, groups2, ref = _grouped_case(device, dtype, bias, n_exp, seed=31 + n_exp)
    got = kernels.ghost_gram_grouped(groups1, groups2, bias=bias)
    assert_parity(got, ref, dtype)
    again = kernels.ghost_gram_grouped(groups1, groups2, bias=bias)
    assert torch.equal(got, again)  # fixed reduction order: bitwise repeatable
    acc = torch.ones_like(got)
    kernels.ghost_gram_grouped(groups1, groups2, bias=bias, out=acc, accumulate=True)
    assert_parity(acc, ref + 1.0, dtype)


@pytest.mark.parametrize("wide_first", [True, False])
def test_moe_layers_cross_gram(device, wide_first):
    """Experts of two routed layers (different widths, one with bias) in one
    launch.  The launch deals tiles longest reduction first, so the narrower
    layer first exercises the reordering of the groups."""
    from dattri_llm_amd.gradient import ops

    gen = torch.Generator().manual_seed(41)
    b, tokens, n_exp = 4, 200, 3
    shapes = [((64, 160), True), ((128, 64), False)]  # ((d_in, d_out), bias)
    if not wide_first:
        shapes = shapes[::-1]
    flat = torch.arange(b * tokens)
    toks = [[flat[torch.rand(b * tokens, generator=gen) < 0.4] for _ in range(n_exp)] for _ in range(2)]
    segs = [ops.moe.segment_experts([t.to(device) for t in side], b, tokens) for side in toks]
    ref = np.zeros((b, b))
    layers = []
    for (k, d), bias in shapes:
        experts = []
        for e in range(n_exp):
            t1, t2 = toks[0][e], toks[1][e]
            a1, g1 = _rand(gen, t1.numel(), k, dtype=torch.bfloat16), _rand(gen, t1.numel(), d, dtype=torch.bfloat16)
            a2, g2 = _rand(gen, t2.numel(), k, dtype=torch.bfloat16), _rand(gen, t2.numel(), d, dtype=torch.bfloat16)
            ref += oracle.moe_segment_ghost(_np(a1), _np(g1), t1.numpy(), _np(a2), _np(g2), t2.numpy(),
                                            b, b, tokens, tokens, bias=bias)
            experts.append(tuple(x.to(device) for x in (a1, g1, a2, g2)))
        layers.append((experts, bias))
    got = ops.moe.moe_layers_cross_gram(layers, segs[0], segs[1])
    assert_parity(got, ref, torch.bfloat16)


# ---------------------------------------------------------------------------
# per-token cross-gram (token decomposition of the score)
# ---------------------------------------------------------------------------

PT_CASES = [
    # (b1, t1, b2, t2, k, d, bias, dtype)
    (2, 300, 3, 200, 64, 48, True, torch.bfloat16),   # 2 row tiles x 2 column tiles, ragged
    (3, 64, 2, 129, 40, 24, False, torch.float32),
    (1, 513, 4, 64, 256, 512, True, torch.float16),    # 3 row tiles
    (4, 128, 5, 128, 136, 72, False, torch.bfloat16),
]


@pytest.mark.parametrize("case", PT_CASES)
def test_ghost_gram_per_token(device, case):
    from dattri_llm_amd import kernels

    b1, t1, b2, t2, k, d, bias, dtype = case
    print(f"ghost_gram_per_token case={case}", flush=True)
    a1, g1, a2, g2 = _inputs(31 + t1, b1, t1, b2, t2, k, d, dtype)
    dev = [x.to(device) for x in (a1, g1, a2, g2)]
    got = kernels.ghost_gram_per_token(*dev, bias=bias)
    assert got.shape == (b1, t1, b2)
    want = oracle.cross_gram_per_token(*(_np(x) for x in (a1, g1, a2, g2)), bias=bias)
    assert_parity(got, want, dtype)
    # the token sum is the ordinary cross-gram
    gram = kernels.ghost_gram(*dev, bias=bias)
    assert_parity(got.sum(1), gram, dtype)
    kernels.ghost_gram_per_token(*dev, bias=bias, out=got, accumulate=True)
    assert_parity(got, 2 * want, dtype)


DENSE_PT_CASES = [
    # (b1, t1, b2, k, d, bias, dtype)
    (2, 300, 3, 64, 136, True, torch.bfloat16),   # 2 output-channel tiles, ragged
    (3, 70, 2, 200, 48, False, torch.float32),
    (1, 257, 4, 520, 264, True, torch.float16),
]


@pytest.mark.parametrize("case", DENSE_PT_CASES)
def test_dense_per_token(device, case):
    from dattri_llm_amd import kernels

    b1, t1, b2, k, d, bias, dtype = case
    print(f"dense_per_token case={case}", flush=True)
    gen = torch.Generator().manual_seed(7 + k)
    a1 = (torch.randn(b1, t1, k, generator=gen) / k**0.5).to(dtype)
    g1 = (torch.randn(b1, t1, d, generator=gen) / d**0.5).to(dtype)
    m2 = (torch.randn(b2, d * (k + int(bias)), generator=gen) / (k * d) ** 0.25).to(dtype)
    got = kernels.dense_per_token(a1.to(device), g1.to(device), m2.to(device), bias=bias)
    want = oracle.cross_gram_per_token_dense(_np(a1), _np(g1), _np(m2), bias=bias)
    assert got.shape == (b1, t1, b2)
    assert_parity(got, want, dtype)


# (b1, s1, b2, s2, k, d, bias, dtype): short sequences, where the dense engine's
# 256 x 128-token tiles would be mostly padding, including single-token rows
SHORT_CASES = [
    (40, 64, 24, 64, 256, 128, False, torch.bfloat16),
    (9, 40, 7, 24, 72, 40, True, torch.bfloat16),
    (300, 1, 70, 1, 128, 96, True, torch.bfloat16),
    (6, 100, 5, 33, 64, 48, False, torch.float32),
]


@pytest.mark.parametrize("case", SHORT_CASES)
def test_short_sequences_take_the_packed_kernel(device, case, monkeypatch):
    """cross_gram's factorized route packs several samples into each tile when
    the dense tiles would hold few live token pairs: the packed (grouped)
    kernel runs, the dense one does not, and the scores match the oracle and
    the dense kernel.  A bias is the preprocessed form: a ones column."""
    from dattri_llm_amd import kernels
    from dattri_llm_amd.gradient import ops

    b1, s1, b2, s2, k, d, bias, dtype = case
    print(f"short-sequence packed route case={case}", flush=True)
    a1, g1, a2, g2 = (x.to(device) for x in _inputs(5, b1, s1, b2, s2, k, d, dtype))
    if bias:
        a1, a2 = (torch.cat([x, torch.ones_like(x[..., :1])], dim=-1) for x in (a1, a2))
    dense = kernels.ghost_gram(a1, g1, a2, g2)
    calls = {"dense": 0, "packed": 0}
    real_dense, real_packed = kernels.ghost_gram, kernels.ghost_gram_grouped

    def spy_dense(*a, **kw):
        calls["dense"] += 1
        return real_dense(*a, **kw)

    def spy_packed(*a, **kw):
        calls["packed"] += 1
        return real_packed(*a, **kw)

    monkeypatch.setattr(kernels, "ghost_gram", spy_dense)
    monkeypatch.setattr(kernels, "ghost_gram_grouped", spy_packed)
    got = ops.cross_gram(a1, g1, a2, g2, "nn.Linear", mode="factorized")  # in the inputs' dtype
    torch.cuda.synchronize()
    assert calls == {"dense": 0, "packed": 1}, calls
    assert got.dtype == dtype
    want = oracle.cross_gram(*(x.double().cpu().numpy() for x in (a1, g1, a2, g2)), "nn.Linear", mode="factorized")
    assert_parity(got, want, dtype, label=f"{case} packed")
    assert_parity(got, dense.double().cpu().numpy(), dtype, label=f"{case} vs dense")
