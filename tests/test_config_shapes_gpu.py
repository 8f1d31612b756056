"""Parity of whole launches at the benchmark configurations' own shapes.

* Ghost cross-gram, 256 train x 64 query samples, T = 512, d_in = d_out = 4096
  (bf16): one full launch (256 x 64 pair tiles over the whole grid and its
  XCD grouping), with 4 x 4 sampled pairs checked against the float64 oracle
  through the materialized reassociation <G_i^T A_i, G_j^T A_j>_F
  (dot.py:110-114, equal to the ghost sum dot.py:115-118).
* Llama-7B MLP projected capture: 640 samples x 128 tokens, projection to
  k = 64 on both sides, gate/up (4096 -> 11008) and down (11008 -> 4096),
  through da_project_outer (the stream-K projection over every piece of the
  640-sample grid, then the per-sample contraction); sampled samples of each
  layer against oracle.project_outer (hooks.py:631-648), then the 512 x 128
  score GEMM over the three layers against float64 products of the very rows
  it read (dot.py:114, :599-604).

Inputs are drawn on the device from a seeded generator; the oracle reads the
same bf16 values copied off it."""

from __future__ import annotations

import pytest
import torch

import oracle
from conftest import TIGHT_FP32, assert_parity

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _randn(gen, shape, scale, device):
    x = torch.empty(*shape, device=device)
    x.normal_(0.0, scale, generator=gen)
    return x.to(BF16)


def _f64(x):
    return x.double().cpu().numpy()


def test_ghost_gram_full_launch_256x64(device):
    from dattri_llm_amd import kernels

    n1, n2, t, d = 256, 64, 512, 4096
    print(f"ghost_gram full launch {n1}x{n2} T={t} d={d} bf16", flush=True)
    gen = torch.Generator(device=device).manual_seed(20)
    a1, g1 = _randn(gen, (n1, t, d), d**-0.5, device), _randn(gen, (n1, t, d), d**-0.5, device)
    a2, g2 = _randn(gen, (n2, t, d), d**-0.5, device), _randn(gen, (n2, t, d), d**-0.5, device)
    got = kernels.ghost_gram(a1, g1, a2, g2)
    torch.cuda.synchronize()
    assert got.shape == (n1, n2) and got.dtype == torch.float32
    assert bool(torch.isfinite(got).all())
    # one train row per XCD quarter of the grid, one query row per quarter
    rows, cols = [0, 85, 170, 255], [0, 21, 42, 63]
    want = oracle.cross_gram_materialized(_f64(a1[rows]), _f64(g1[rows]), _f64(a2[cols]), _f64(g2[cols]))
    assert_parity(got[rows][:, cols], want, BF16, label="ghost 256x64 sampled pairs")
    # the diagonal of one sample against itself is a squared norm: positive
    self_gram = kernels.ghost_gram(a1[:4], g1[:4], a1[:4], g1[:4])
    assert bool((torch.diagonal(self_gram) > 0).all())


PROJ_LAYERS = [("gate_proj", 4096, 11008), ("up_proj", 4096, 11008), ("down_proj", 11008, 4096)]


def test_projected_capture_llama7b_mlp_640_samples(device):
    from dattri_llm_amd import kernels
    from dattri_llm_amd.gradient.ops.projection import gaussian_matrix

    n_train, n_query, t, k = 512, 128, 128, 64
    n = n_train + n_query
    print(f"project_outer {n} samples x {t} tokens, k={k}, gate/up/down", flush=True)
    gen = torch.Generator(device=device).manual_seed(21)
    acts = {4096: _randn(gen, (n, t, 4096), 4096**-0.5, device),
            11008: _randn(gen, (n, t, 11008), 11008**-0.5, device)}
    sample = [0, 255, 511, 639]  # first / last train rows, first / last query rows
    feats = []
    for li, (name, din, dout) in enumerate(PROJ_LAYERS):
        g = _randn(gen, (n, t, dout), dout**-0.5, device)
        a = acts[din]
        # the projector's convention: activation side seed + 1, gradient side seed
        p_in = gaussian_matrix(din, k, 2 * li + 1).to(device, BF16)
        p_out = gaussian_matrix(dout, k, 2 * li).to(device, BF16)
        pin_t, pout_t = p_in.t().contiguous(), p_out.t().contiguous()
        got32 = kernels.project_outer(a, g, pin_t, pout_t, out_dtype=torch.float32)
        got = kernels.project_outer(a, g, pin_t, pout_t)
        torch.cuda.synchronize()
        assert got32.shape == (n, k * k) and got.dtype == BF16
        want = oracle.project_outer(_f64(a[sample]), _f64(g[sample]), _f64(p_in), _f64(p_out))
        assert_parity(got32[sample], want, BF16, tight=TIGHT_FP32, label=f"{name} fp32 rows")
        # the bf16 result is the same fp32 contraction rounded once (RNE)
        assert torch.equal(got, got32.to(BF16)), name
        feats.append(got)
        del g, got32

    scores = kernels.score_gemm([(f[:n_train], f[n_train:]) for f in feats])
    torch.cuda.synchronize()
    assert scores.shape == (n_train, n_query) and scores.dtype == torch.float32
    want = sum(_f64(f[:n_train]) @ _f64(f[n_train:]).T for f in feats)
    assert_parity(scores, want, BF16, tight=TIGHT_FP32, label="512x128 score GEMM over 3 layers")
