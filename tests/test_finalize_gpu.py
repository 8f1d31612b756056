"""finalize_factors on the device (the reference's
tests/attribution/test_utils.py:500-634): norm and convolution layers of a raw
capture are replaced once by their final factors and every kernel scores them
exactly as it scores the raw ones; embeddings stay raw; a layer whose final
form would outgrow the budget stays raw; final and dense blocks pass through.
Linear layers stay raw here by design -- their bias column is applied inside
the kernels -- which the reference's finalize would fold into the factors."""

from __future__ import annotations

import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu


def _raw_block(n, device, seed=0):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    gen = torch.Generator().manual_seed(seed)
    modules = {
        "linear": (nn.Linear(6, 5), "nn.Linear", (n, 3, 6), (n, 3, 5)),
        "nobias": (nn.Linear(6, 5, bias=False), "nn.Linear", (n, 3, 6), (n, 3, 5)),
        "norm": (nn.LayerNorm(6), "nn.LayerNorm", (n, 3, 6), (n, 3, 6)),
        "conv": (nn.Conv2d(2, 4, 3, padding=1), "nn.Conv2d", (n, 2, 5, 5), (n, 4, 5, 5)),
        "convT": (nn.ConvTranspose1d(3, 2, 2), "nn.ConvTranspose1d", (n, 3, 4), (n, 2, 5)),
    }
    data, types = {}, {}
    for name, (module, lt, a_shape, g_shape) in modules.items():
        data[name] = Factorized(torch.randn(*a_shape, generator=gen).to(device),
                                torch.randn(*g_shape, generator=gen).to(device),
                                module_kwargs=ops.extract_module_kwargs(module, lt))
        types[name] = lt
    emb = nn.Embedding(11, 8)
    data["emb"] = Factorized(torch.randint(0, 11, (n, 3), generator=gen).to(device),
                             torch.randn(n, 3, 8, generator=gen).to(device),
                             module_kwargs=ops.extract_module_kwargs(emb, "nn.Embedding"))
    types["emb"] = "nn.Embedding"
    return Gradient(dict.fromkeys(data, "factorized"), data, types, dict.fromkeys(data, "batch_token"),
                    validate_on_init=False)


def test_norm_and_conv_layers_become_final(device):
    from dattri_llm_amd.attribution.utils import finalize_factors

    final = finalize_factors(_raw_block(4, device))
    for name in ("norm", "conv", "convT"):
        assert final.data[name].module_kwargs is None, name
    for name in ("emb", "linear", "nobias"):
        assert final.data[name].module_kwargs is not None, name
    assert final.data["norm"].activation.shape[-1] == 12  # x_hat with the bias block
    assert final.data["conv"].activation.shape[-1] == 2 * 9 + 1  # unfolded patches and the ones column


def test_scores_match_the_raw_block(device):
    from dattri_llm_amd.attribution.utils import finalize_factors
    from dattri_llm_amd.gradient import ops

    raw = ops.layerwise_cross_dot(_raw_block(4, device, 1), _raw_block(2, device, 2), reduce="none")
    mixed = ops.layerwise_cross_dot(_raw_block(4, device, 1), finalize_factors(_raw_block(2, device, 2)),
                                    reduce="none")
    both = ops.layerwise_cross_dot(finalize_factors(_raw_block(4, device, 1)),
                                   finalize_factors(_raw_block(2, device, 2)), reduce="none")
    for name, want in raw.items():
        assert torch.allclose(mixed[name], want, atol=1e-5, rtol=1e-5), name
        assert torch.allclose(both[name], want, atol=1e-5, rtol=1e-5), name


def test_final_block_is_not_preprocessed_again(device, monkeypatch):
    """Scoring finalized blocks unfolds no convolution and normalizes no raw
    norm input (x_hat is not recomputed), however many times they are scored."""
    from dattri_llm_amd import kernels
    from dattri_llm_amd.attribution.utils import finalize_factors
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.ops import conv

    train, query = finalize_factors(_raw_block(4, device, 1)), finalize_factors(_raw_block(2, device, 2))
    calls = []

    def counting(name, real):
        def wrapped(*args, **kwargs):
            if kwargs.get("kind") != kernels.NORM_KIND_GIVEN:  # kind 2 takes x_hat as given
                calls.append(name)
            return real(*args, **kwargs)
        return wrapped

    monkeypatch.setattr(conv, "unfold_patches", counting("unfold", conv.unfold_patches))
    monkeypatch.setattr(kernels, "norm_weight_grad", counting("norm_weight_grad", kernels.norm_weight_grad))
    monkeypatch.setattr(kernels, "norm_xhat", counting("norm_xhat", kernels.norm_xhat))
    for _ in range(3):
        ops.layerwise_cross_dot(train, query)
    assert calls == []
    ops.layerwise_cross_dot(_raw_block(4, device, 1), _raw_block(2, device, 2))
    assert "unfold" in calls  # the raw blocks do run them


def test_budget_keeps_a_growing_layer_raw(device):
    from dattri_llm_amd.attribution.utils import finalize_factors
    from dattri_llm_amd.utils.cache import CacheBudget

    final = finalize_factors(_raw_block(4, device), budget=CacheBudget(limit_bytes=0))
    assert final.data["norm"].module_kwargs is not None  # x_hat plus the bias block: grows
    assert final.data["conv"].module_kwargs is not None  # the unfolded patches: grow


def test_final_and_dense_blocks_pass_through(device):
    from dattri_llm_amd.attribution.utils import finalize_factors
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    block = Gradient({"l1": "factorized"}, {"l1": Factorized(torch.randn(2, 4, 3, device=device),
                                                             torch.randn(2, 4, 5, device=device))},
                     {"l1": "nn.Linear"}, {"l1": "batch_token"})
    assert finalize_factors(block) is block
    dense = Gradient({"l1": "materialized"}, {"l1": torch.randn(2, 15, device=device)}, {"l1": "nn.Linear"})
    assert finalize_factors(dense) is dense
