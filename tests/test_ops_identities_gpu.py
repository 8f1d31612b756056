"""The reference's algebraic identity suite (tests/gradient/test_ops.py:63-214)
on the MI355X kernels: for every supported layer type, with factors already in
preprocessed form and the reference's shapes (B=4, T=6, D_IN=8, D_OUT=12,
vocab 32, E=10),

    pairwise_dot_factors(a, g)[i, j] == mat[i] . mat[j]
    grad_norm_sq_factors(a, g)[i]    == |mat[i]|^2
    dot_factors(a1, g1, a2, g2)[i]   == mat1[i] . mat2[i]

where mat = materialize_factors(a, g) is the per-sample weight gradient, plus
symmetry, a non-negative diagonal, norm == diagonal and self-dot == norm, all
at the reference's fp32 tolerance (atol = rtol = 1e-4)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

B, T, D_IN, D_OUT, VOCAB, E = 4, 6, 8, 12, 32, 10
EMB_MK = {"has_bias": False, "num_embeddings": VOCAB, "padding_idx": None}


def _pair(gen, *shapes):
    return tuple(torch.randn(*s, generator=gen) for s in shapes)


def _factors(lt, gen):
    if lt in ("nn.Embedding", "nn.EmbeddingBag"):
        return torch.randint(0, VOCAB, (B, T), generator=gen), torch.randn(B, T, E, generator=gen)
    if lt in ("nn.LayerNorm", "nn.RMSNorm", "nn.GroupNorm", "nn.InstanceNorm1d"):
        return _pair(gen, (B, D_IN), (B, D_IN))
    if lt in ("nn.LayerNorm-3d",):
        return _pair(gen, (B, T, D_IN), (B, T, D_IN))
    if lt in ("nn.Linear", "nn.Bilinear"):
        return _pair(gen, (B, D_IN), (B, D_OUT))
    return _pair(gen, (B, T, D_IN), (B, T, D_OUT))  # Linear-3d, conv, conv-transpose


CASES = ["nn.Linear", "nn.Linear-3d", "nn.Bilinear", "nn.Conv1d", "nn.Conv2d", "nn.Conv3d", "nn.ConvTranspose1d",
         "nn.ConvTranspose2d", "nn.ConvTranspose3d", "nn.LayerNorm", "nn.LayerNorm-3d", "nn.RMSNorm", "nn.GroupNorm",
         "nn.InstanceNorm1d", "nn.Embedding", "nn.EmbeddingBag"]


def _lt(tag):
    return tag.replace("-3d", "")


def _mat(ops, a, g, lt):
    if lt in ("nn.Embedding", "nn.EmbeddingBag"):
        return ops.materialize_factors(a, g, "nn.Embedding", module_kwargs=EMB_MK)
    return ops.materialize_factors(a, g, lt)


def _close(actual, expected, what):
    assert torch.allclose(actual, expected, atol=1e-4, rtol=1e-4), (
        f"{what}: max diff {(actual - expected).abs().max().item():.2e}")


@pytest.mark.parametrize("tag", CASES)
def test_identities(device, tag):
    from dattri_llm_amd.gradient import ops

    lt = _lt(tag)
    gen = torch.Generator().manual_seed(CASES.index(tag))
    a, g = (t.to(device) for t in _factors(tag, gen))
    a2, g2 = (t.to(device) for t in _factors(tag, gen))
    print(f"identities {tag}", flush=True)
    mat = _mat(ops, a, g, lt).float()
    mat2 = _mat(ops, a2, g2, lt).float()
    assert mat.shape[0] == B and mat.dim() == 2

    k = ops.pairwise_dot_factors(a, g, lt).float()
    assert k.shape == (B, B)
    _close(k, mat @ mat.T, f"[{tag}] pairwise vs materialized Gram")
    _close(k, k.T, f"[{tag}] symmetry")
    assert (k.diagonal() >= -1e-6).all()

    norms = ops.grad_norm_sq_factors(a, g, lt).float()
    assert norms.shape == (B,)
    _close(norms, mat.pow(2).sum(-1), f"[{tag}] norm vs materialized")
    _close(norms, k.diagonal(), f"[{tag}] norm vs Gram diagonal")

    dots = ops.dot_factors(a, g, a2, g2, lt).float()
    assert dots.shape == (B,)
    _close(dots, (mat * mat2).sum(-1), f"[{tag}] dot vs materialized")
    _close(ops.dot_factors(a, g, a, g, lt).float(), norms, f"[{tag}] self-dot vs norm")

    cross = ops.cross_dot_factors(a, g, a2, g2, lt).float()
    _close(cross, mat @ mat2.T, f"[{tag}] cross Gram vs materialized")
