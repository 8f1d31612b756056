"""GPU parity of the projection styles on convolution and embedding layers
(projection.py:440-489, :687-775) against the oracle.

LoGRA ("logra"): both factors projected, the activation side with
``proj_seed + 1`` -- for an embedding, the one-hot ids times the
``(num_embeddings, k)`` matrix.  Mask ("mask"): fixed coordinates of the
materialized per-sample gradient, gathered from the factors.
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
K = 16


def _matrix(d, seed):
    from dattri_llm_amd.gradient.ops.projection import gaussian_matrix

    return gaussian_matrix(d, K, seed).double().numpy()


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_logra_and_mask(device, case):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.ops.projection import DattriProjector

    transpose, rank, _ci, _co, k, s, p, d, groups, bias, _sp = case
    lt = _NAMES[(transpose, rank)]
    mk = {"has_bias": bias, "kernel_size": k, "stride": s, "padding": p, "dilation": d, "groups": groups}
    x, gout = conv_inputs(case, n=3, seed=80)
    print(f"conv projection case={case}", flush=True)
    a_ref, g_ref = oracle.conv_preprocess(x, gout, transpose, k, s, p, d, groups, bias)
    xd, gd = torch.from_numpy(x).float().to(device), torch.from_numpy(gout).float().to(device)

    a_p, g_p = ops.project_factors(xd, gd, lt, None, mk, proj_dim=K, proj_seed=3)
    assert_parity(a_p, a_ref @ _matrix(a_ref.shape[-1], 4), torch.float32, label="a_p")
    assert_parity(g_p, g_ref @ _matrix(g_ref.shape[-1], 3), torch.float32, label="g_p")
    outer = ops.project_outer_factors(xd, gd, lt, None, mk, proj_dim=K, proj_seed=3)
    assert_parity(outer, oracle.conv_materialize(a_p.double().cpu().numpy(), g_p.double().cpu().numpy()),
                  torch.float32, label="outer")

    dense = oracle.conv_materialize(a_ref, g_ref, transpose)
    kept = min(40, dense.shape[1] - 1)
    idx = DattriProjector(None).mask_indices(dense.shape[1], proj_dim=kept, proj_seed=5, device="cpu").numpy()
    got = ops.mask_factors(xd, gd, lt, None, mk, proj_dim=kept, proj_seed=5)
    assert got.shape == (3, kept)
    assert_parity(got, dense[:, idx], torch.float32, label="mask")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layer_type", ["nn.Embedding", "nn.EmbeddingBag"])
def test_embedding_logra_and_mask(device, dtype, layer_type):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.ops.projection import DattriProjector

    vocab, e, b, t, pad = 300, 24, 4, 50, 0
    gen = torch.Generator().manual_seed(9)
    ids = torch.randint(1, vocab, (b, t), generator=gen)
    ids[:, -4:] = pad
    ids[:, 5:15] = 17  # a repeated id
    bag = layer_type == "nn.EmbeddingBag"
    g = torch.randn(*((b, e) if bag else (b, t, e)), generator=gen).to(dtype)
    mk = {"has_bias": False, "num_embeddings": vocab, "padding_idx": pad}
    if bag:
        mk["mode"] = "mean"
        a_ref, rows_ref = oracle.embedding_bag_expand(ids.numpy(), g.double().numpy(), "mean", pad)
    else:
        a_ref = ids.numpy()
        rows_ref = np.where((ids == pad)[..., None].numpy(), 0.0, g.double().numpy())
    print(f"embedding projection {layer_type} {dtype}", flush=True)
    ids_d, g_d = ids.to(device), g.to(device)

    a_p, g_p = ops.project_factors(ids_d, g_d, layer_type, None, mk, proj_dim=K, proj_seed=1)
    onehot = np.eye(vocab)[ids.numpy()]  # the reference's one-hot, times the input-side matrix
    assert a_p.dtype == torch.float32
    assert np.array_equal(a_p.double().cpu().numpy(), onehot @ _matrix(vocab, 2))
    assert_parity(g_p, rows_ref @ _matrix(e, 1), dtype, label="g_p")

    dense = oracle.embedding_materialize(a_ref, rows_ref, vocab)
    idx = DattriProjector(None).mask_indices(vocab * e, proj_dim=200, proj_seed=2, device="cpu").numpy()
    idx[:8] = 17 * e + np.arange(8)  # some coordinates of the repeated id's row
    idx.sort()
    got = ops.mask_factors(ids_d, g_d, layer_type, None, mk, proj_dim=200, proj_seed=2)
    ref = dense[:, DattriProjector(None).mask_indices(vocab * e, proj_dim=200, proj_seed=2, device="cpu").numpy()]
    assert got.shape == (b, 200) and got.dtype == dtype
    assert_parity(got, ref, dtype, label="mask")
    # the kernel on chosen coordinates (a repeated id's row and a pad row)
    from dattri_llm_amd import kernels
    from dattri_llm_amd.gradient.ops import embedding as emb_ops

    emb_ids, emb_rows = emb_ops.side(ids_d, g_d, layer_type, mk)
    rows_t, cols_t = torch.from_numpy(idx // e).to(device), torch.from_numpy(idx % e).to(device)
    direct = kernels.gather_embedding_entries(emb_ids, emb_rows, rows_t, cols_t)
    # fp32 entries of the bag's divided rows, which the product holds in g's dtype (one rounding)
    assert_parity(direct, dense[:, idx], dtype, tight=roundings(1) if dtype == torch.bfloat16 else None,
                  label="entries")
    with pytest.raises(ValueError, match="num_embeddings"):
        ops.project_factors(ids_d, g_d, layer_type, None, None, proj_dim=K)
