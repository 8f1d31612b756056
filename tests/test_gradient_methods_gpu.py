"""Gradient block methods that run kernels, against the float64 oracle:
per-token similarity (dattri_llm/gradient/gradient.py:1072-1133) is the
token decomposition of the ordinary similarity; token aggregation of a
factorized layer is its materialized gradient (:838-886); pinning keeps
values (:516-537)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_parity, roundings

pytestmark = pytest.mark.gpu


def _blocks(device):
    from dattri_llm_amd.gradient import Factorized, Gradient

    gen = torch.Generator(device=device).manual_seed(11)

    def rnd(*shape, scale=0.1):
        return (torch.randn(*shape, generator=gen, device=device) * scale).bfloat16()

    def block(b, t):
        data = {"up": Factorized(rnd(b, t, 256), rnd(b, t, 384), module_kwargs={"has_bias": False}),
                "down": Factorized(rnd(b, t, 384), rnd(b, t, 256), module_kwargs={"has_bias": False})}
        return Gradient(dict.fromkeys(data, "factorized"), data, dict.fromkeys(data, "nn.Linear"),
                        dict.fromkeys(data, "batch_token"))

    return block(3, 96), block(4, 64)


def _np(t):
    return t.double().cpu().numpy()


def test_similarity_per_token_decomposes_similarity(device):
    print("similarity_per_token, 3x96 vs 4x64 tokens, 2 linears", flush=True)
    x, y = _blocks(device)
    per_tok = x.similarity_per_token(y)
    torch.cuda.synchronize()
    assert per_tok.shape == (3, 96, 4)
    want = sum(oracle.cross_gram_per_token(*(_np(t) for t in (x.data[n].activation, x.data[n].pre_activation_grad,
                                                             y.data[n].activation, y.data[n].pre_activation_grad)))
               for n in ("up", "down"))
    # bf16 roundings: side 2's dense gradient, each layer's (3, 96, 4) output, their sum
    assert_parity(per_tok, want, torch.bfloat16, tight=roundings(3), label="per-token similarity")
    # the decomposition in fp32 (no per-token bf16 rounding to accumulate)
    from dattri_llm_amd.gradient import ops

    with ops.compute_dtype(torch.float32):
        per_tok32 = x.similarity_per_token(y)
        total = x.similarity(y, reduce="all")
    assert per_tok32.dtype == torch.float32
    assert_parity(per_tok32.double().sum(1), total.double().cpu().numpy(), torch.float32,
                  label="sum over tokens == similarity")
    layers = x.similarity_per_token(y, reduce="none")
    assert set(layers) == {"up", "down"} and layers["up"].shape == (3, 96, 4)


def test_aggregate_materializes_factorized_token_layers(device):
    print("aggregate of factorized batch_token layers", flush=True)
    x, _ = _blocks(device)
    agg = x.aggregate()
    torch.cuda.synchronize()
    assert agg.representation == {"up": "materialized", "down": "materialized"}
    assert agg.indexing == {"up": "batch", "down": "batch"}
    for n in ("up", "down"):
        f = x.data[n]
        want = oracle.materialize_linear(_np(f.activation), _np(f.pre_activation_grad))
        assert_parity(agg.data[n].reshape(want.shape), want, torch.bfloat16, out_dtype=torch.bfloat16,
                      label=f"aggregate {n}")


def test_pin_memory_pins_host_payloads_and_keeps_values(device):
    x, _ = _blocks(device)
    host = x.to("cpu")
    pinned = host.pin_memory()
    for n in ("up", "down"):
        assert pinned.data[n].activation.is_pinned() and pinned.data[n].pre_activation_grad.is_pinned()
        assert torch.equal(pinned.data[n].activation, host.data[n].activation)
    again = pinned.pin_memory()
    assert again.data["up"].activation.data_ptr() == pinned.data["up"].activation.data_ptr()
    on_dev = x.pin_memory()
    assert on_dev.data["up"].activation is x.data["up"].activation
    assert np.isfinite(_np(pinned.data["down"].pre_activation_grad)).all()
