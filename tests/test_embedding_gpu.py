"""GPU parity of the embedding layer family against the oracle.

* ``da_materialize_embedding`` (materialize.py:22-48) is bit-exact against the
  oracle's restatement of the CPU scatter_add_ (fp32 sums in ascending token
  order, one rounding), in bf16, fp16 and fp32;
* the embedding cross-gram kernels (dot.py:58-74, :189-203, :325-337, :383-384)
  and the dense per-token product (dot.py:239-245) meet the two parity bars
  of conftest.assert_parity against the float64 oracle;
* the ops entry points (padding_idx, EmbeddingBag sum/mean) route there.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_parity, roundings, stable_seed

pytestmark = pytest.mark.gpu

_ODT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def _ids(gen, b, t, vocab, repeat_from=None):
    ids = torch.randint(0, vocab, (b, t), generator=gen)
    if repeat_from is not None:  # a run of one id: long sums into one row
        ids[:, repeat_from:repeat_from + 64] = 3 % vocab
    return ids


def _grad(gen, *shape, dtype):
    return (torch.randn(*shape, generator=gen) * 2).to(dtype)


MAT_CASES = [
    # (b, t, e, vocab)
    (3, 200, 64, 7),        # many repeats of few ids
    (2, 2500, 40, 50),      # more tokens than one LDS run of ids
    (4, 6, 10, 32),         # the reference test's sizes: E padded to a 16-byte chunk
    (1, 1, 8, 1),
    (5, 300, 136, 4000),    # mostly distinct ids
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", MAT_CASES)
def test_materialize_embedding_bit_exact(device, dtype, case):
    from dattri_llm_amd import kernels

    b, t, e, vocab = case
    gen = torch.Generator().manual_seed(stable_seed(case))
    ids = _ids(gen, b, t, vocab, repeat_from=t // 3 if t > 100 else None)
    g = _grad(gen, b, t, e, dtype=dtype)
    print(f"materialize_embedding case={case} dtype={dtype}", flush=True)
    got = kernels.materialize_embedding(ids.to(device), g.to(device), vocab)
    assert got.shape == (b, vocab * e) and got.dtype == dtype
    ref = oracle.embedding_materialize(ids.numpy(), g.float().numpy(), vocab, dtype=_ODT[dtype])
    assert np.array_equal(got.float().cpu().numpy(), ref)


def test_materialize_embedding_empty_and_negative_ids(device):
    from dattri_llm_amd import kernels

    g = torch.randn(2, 0, 8).to(device, torch.bfloat16)
    out = kernels.materialize_embedding(torch.zeros(2, 0, dtype=torch.int64, device=device), g, 5)
    assert out.shape == (2, 40) and not out.any()
    # a negative id (a padding position) adds nothing
    ids = torch.tensor([[1, -1, 1, 2]], device=device)
    g = torch.randn(1, 4, 8).to(device, torch.bfloat16)
    got = kernels.materialize_embedding(ids, g, 3).view(1, 3, 8).float().cpu()
    assert torch.equal(got[0, 0], torch.zeros(8))
    ref = oracle.embedding_materialize(np.array([[1, 1, 2]]), g.float().cpu().numpy()[:, [0, 2, 3]], 3, dtype="bf16")
    assert np.array_equal(got.numpy().reshape(1, -1), ref)


def test_materialize_embedding_llama_vocab_rows(device):
    """Full-size shape (vocab 128256, E 4096, 2 x 2048 bf16 tokens): every row
    of an id that no token uses is zero, and the rows of sampled ids equal the
    oracle's bit for bit."""
    from dattri_llm_amd import kernels

    vocab, e, b, t = 128256, 4096, 2, 2048
    gen = torch.Generator().manual_seed(7)
    ids = torch.randint(0, vocab, (b, t), generator=gen)
    ids[:, 100:400] = 42  # one frequent id
    g = _grad(gen, b, t, e, dtype=torch.bfloat16)
    print("materialize_embedding full-size", flush=True)
    got = kernels.materialize_embedding(ids.to(device), g.to(device), vocab).view(b, vocab, e)
    used = torch.zeros(b, vocab, dtype=torch.bool)
    used[torch.arange(b)[:, None], ids] = True
    nonzero = got.ne(0).any(-1).cpu()
    assert not (nonzero & ~used).any()
    for i in range(b):
        for v in (42, int(ids[i, 0]), int(ids[i, -1])):
            sel = (ids[i] == v).numpy()
            row = g[i][torch.from_numpy(sel)].float().numpy().sum(axis=0, dtype=np.float32)
            # ascending-t fp32 sum, then one rounding
            acc = np.zeros(e, dtype=np.float32)
            for r in g[i][torch.from_numpy(sel)].float().numpy():
                acc = acc + r
            ref = oracle.ops._round_to(acc, "bf16")
            assert np.array_equal(got[i, v].float().cpu().numpy(), ref), (i, v)
            assert np.allclose(ref, row, rtol=1e-2, atol=1e-2)
    del got


GRAM_CASES = [
    # (b1, t1, b2, t2, e, vocab)
    (3, 128, 2, 128, 64, 50),
    (4, 300, 3, 200, 40, 30),     # ragged tiles, T1 != T2
    (2, 257, 5, 17, 256, 9),      # few ids: most pairs match
    (1, 1, 1, 1, 8, 3),
    (2, 64, 3, 96, 10, 1000),     # E padded to a 16-byte chunk
]


def _gram_inputs(case, dtype, pad=True):
    b1, t1, b2, t2, e, vocab = case
    gen = torch.Generator().manual_seed(stable_seed(case))
    tok1, tok2 = _ids(gen, b1, t1, vocab), _ids(gen, b2, t2, vocab)
    if pad and t1 > 4:
        tok1[:, -3:] = -1  # padding positions match nothing
        tok2[0, :2] = -1
    g1, g2 = _grad(gen, b1, t1, e, dtype=dtype), _grad(gen, b2, t2, e, dtype=dtype)
    return tok1, g1, tok2, g2


def _oracle_ids(tok, side):
    """The oracle's ids for a side with padding: -1 positions get ids that
    match nothing on either side (numpy equality would pair two -1s)."""
    tok = tok.numpy().copy()
    neg = tok < 0
    tok[neg] = -np.arange(1, neg.sum() + 1) - side * 10**9
    return tok


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", GRAM_CASES)
def test_embedding_cross_gram_matches_oracle(device, dtype, case):
    from dattri_llm_amd import kernels

    tok1, g1, tok2, g2 = _gram_inputs(case, dtype)
    print(f"embedding_cross_gram case={case} dtype={dtype}", flush=True)
    d = [x.to(device) for x in (tok1, g1, tok2, g2)]
    t1, t2 = _oracle_ids(tok1, 1), _oracle_ids(tok2, 2)
    got = kernels.embedding_cross_gram(*d)
    ref = oracle.embedding_cross_gram(t1, g1.double().numpy(), t2, g2.double().numpy())
    assert_parity(got, ref, dtype, label="gram")
    per_tok = kernels.embedding_cross_gram_per_token(*d)
    ref_pt = oracle.embedding_cross_gram_per_token(t1, g1.double().numpy(), t2, g2.double().numpy())
    assert per_tok.shape == ref_pt.shape
    assert_parity(per_tok, ref_pt, dtype, label="per_token")
    # accumulate adds into out
    out = torch.ones_like(got)
    kernels.embedding_cross_gram(*d, out=out, accumulate=True)
    assert_parity(out, ref + 1.0, dtype, label="accumulate")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", [(4, 300, 4, 200, 40, 30), (3, 77, 3, 77, 64, 5)])
def test_embedding_cross_gram_diag(device, dtype, case):
    from dattri_llm_amd import kernels

    tok1, g1, tok2, g2 = _gram_inputs(case, dtype)
    d = [x.to(device) for x in (tok1, g1, tok2, g2)]
    got = kernels.embedding_cross_gram(*d, diag=True)
    full = oracle.embedding_cross_gram(_oracle_ids(tok1, 1), g1.double().numpy(), _oracle_ids(tok2, 2),
                                       g2.double().numpy())
    assert got.shape == (case[0],)
    assert_parity(got, np.diagonal(full).copy(), dtype, label="diag")
    # one block with itself: the squared norms of the materialized gradients
    sq = kernels.embedding_cross_gram(d[0], d[1], d[0], d[1], diag=True)
    m = oracle.embedding_materialize(tok1.clamp_min(0).numpy(), np.where((tok1 < 0)[..., None].numpy(), 0.0,
                                     g1.double().numpy()), case[5])
    assert_parity(sq, (m * m).sum(-1), dtype, label="norm")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dense_per_token_embedding(device, dtype):
    from dattri_llm_amd import kernels

    case = (3, 150, 4, 90, 48, 40)
    tok1, g1, tok2, g2 = _gram_inputs(case, dtype)
    vocab = case[5]
    m2 = oracle.embedding_materialize(tok2.clamp_min(0).numpy(),
                                      np.where((tok2 < 0)[..., None].numpy(), 0.0, g2.float().numpy()), vocab,
                                      dtype=_ODT[dtype])
    m2_t = torch.from_numpy(m2).to(dtype)
    got = kernels.dense_per_token_embedding(tok1.to(device), g1.to(device), m2_t.to(device), vocab)
    ref = oracle.embedding_per_token_dense(np.where(tok1.numpy() < 0, 0, tok1.numpy()),
                                           np.where((tok1 < 0)[..., None].numpy(), 0.0, g1.double().numpy()),
                                           m2_t.double().numpy(), vocab)
    assert_parity(got, ref, dtype, label="dense_per_token")


# ---------------------------------------------------------------------------
# the ops layer
# ---------------------------------------------------------------------------


def test_ops_embedding_padding_idx(device):
    """materialize_factors / dot_factors / grad_norm_sq_factors / cross_dot_factors
    with a padding_idx: pad positions contribute nothing (preprocess.py:403-408)."""
    from dattri_llm_amd.gradient import ops

    vocab, e, b, t, pad = 32, 16, 4, 40, 0
    gen = torch.Generator().manual_seed(11)
    ids = torch.randint(1, vocab, (b, t), generator=gen)
    ids[:, -5:] = pad
    g = torch.randn(b, t, e, generator=gen)
    mk = {"has_bias": False, "num_embeddings": vocab, "padding_idx": pad}
    gp = np.where((ids == pad)[..., None].numpy(), 0.0, g.double().numpy())
    mat_ref = oracle.embedding_materialize(ids.numpy(), gp, vocab)
    ids_d, g_d = ids.to(device), g.to(device)
    mat = ops.materialize_factors(ids_d, g_d, "nn.Embedding", module_kwargs=mk)
    assert mat.shape == (b, vocab * e) and mat.dtype == torch.float32
    assert_parity(mat, mat_ref, torch.float32, label="materialize")
    # the public preprocess returns the reference's masked factors
    a_p, g_p = ops.preprocess_factors(ids_d, g_d, "nn.Embedding", mk)
    assert torch.equal(a_p.cpu(), ids) and np.array_equal(g_p.double().cpu().numpy(), gp)
    sq = ops.grad_norm_sq_factors(ids_d, g_d, "nn.Embedding", module_kwargs=mk)
    assert_parity(sq, (mat_ref * mat_ref).sum(-1), torch.float32, label="norm")
    dots = ops.dot_factors(ids_d, g_d, ids_d.flip(0), g_d.flip(0), "nn.Embedding", mk, mk)
    assert_parity(dots, (mat_ref * mat_ref[::-1]).sum(-1), torch.float32, label="dot")
    cross = ops.cross_dot_factors(ids_d, g_d, ids_d[:2], g_d[:2], "nn.Embedding", mk, mk)
    assert_parity(cross, mat_ref @ mat_ref[:2].T, torch.float32, label="cross")


@pytest.mark.parametrize("mode", ["sum", "mean"])
@pytest.mark.parametrize("pad", [None, 0])
def test_ops_embedding_bag(device, mode, pad):
    from dattri_llm_amd.gradient import ops

    vocab, e, n, t = 20, 24, 5, 9
    gen = torch.Generator().manual_seed(12)
    ids = torch.randint(1, vocab, (n, t), generator=gen)
    if pad is not None:
        ids[:, -2:] = pad
        ids[1, -4] = pad
    g = torch.randn(n, e, generator=gen)
    mk = {"has_bias": False, "num_embeddings": vocab, "mode": mode, "padding_idx": pad}
    a, rows = oracle.embedding_bag_expand(ids.numpy(), g.double().numpy(), mode, pad)
    mat_ref = oracle.embedding_materialize(a, rows, vocab)
    ids_d, g_d = ids.to(device), g.to(device)
    mat = ops.materialize_factors(ids_d, g_d, "nn.EmbeddingBag", module_kwargs=mk)
    assert_parity(mat, mat_ref, torch.float32, label="materialize")
    a_p, g_p = ops.preprocess_factors(ids_d, g_d, "nn.EmbeddingBag", mk)
    assert g_p.shape == (n, t, e)
    assert_parity(g_p, rows, torch.float32, label="preprocess")
    gram = ops.cross_dot_factors(ids_d, g_d, ids_d, g_d, "nn.EmbeddingBag", mk, mk)
    assert_parity(gram, mat_ref @ mat_ref.T, torch.float32, label="gram")
    sq = ops.grad_norm_sq_factors(ids_d, g_d, "nn.EmbeddingBag", module_kwargs=mk)
    assert_parity(sq, (mat_ref * mat_ref).sum(-1), torch.float32, label="norm")


def test_ops_embedding_cross_gram_and_per_token(device):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized

    vocab, e = 60, 32
    gen = torch.Generator().manual_seed(13)
    tok1, tok2 = torch.randint(0, vocab, (3, 70), generator=gen), torch.randint(0, vocab, (4, 50), generator=gen)
    g1, g2 = (torch.randn(3, 70, e, generator=gen).to(torch.bfloat16),
              torch.randn(4, 50, e, generator=gen).to(torch.bfloat16))
    d1, d2 = (tok1.to(device), g1.to(device)), (tok2.to(device), g2.to(device))
    ref = oracle.embedding_cross_gram(tok1.numpy(), g1.double().numpy(), tok2.numpy(), g2.double().numpy())
    got = ops.cross_gram(*d1, *d2, "nn.Embedding")
    assert got.dtype == torch.bfloat16
    assert_parity(got, ref, torch.bfloat16, tight=roundings(1), label="cross_gram")
    ref_pt = oracle.embedding_cross_gram_per_token(tok1.numpy(), g1.double().numpy(), tok2.numpy(),
                                                   g2.double().numpy())
    pt = ops.cross_gram_per_token(*d1, *d2, "nn.Embedding")
    assert_parity(pt, ref_pt, torch.bfloat16, tight=roundings(1), label="per_token")
    # side 2 dense (materialize's layout): the gathered-row product
    mk = {"has_bias": False, "num_embeddings": vocab, "padding_idx": None}
    m2 = ops.materialize_factors(*d2, "nn.Embedding", module_kwargs=mk)
    ptd = ops.cross_gram_per_token_dense(*d1, m2, "nn.Embedding")
    assert_parity(ptd, ref_pt, torch.bfloat16, tight=roundings(2), label="per_token_dense")
    f1 = Factorized(activation=d1[0], pre_activation_grad=d1[1], module_kwargs=mk)
    f2 = Factorized(activation=d2[0], pre_activation_grad=d2[1], module_kwargs=mk)
    assert_parity(ops.cross_dot_per_token(f1, f2, "nn.Embedding"), ref_pt, torch.bfloat16, tight=roundings(1),
                  label="cross_dot_per_token")
    assert_parity(ops.cross_dot_per_token(f1, m2, "nn.Embedding"), ref_pt, torch.bfloat16, tight=roundings(2),
                  label="cross_dot_per_token dense")


def test_ops_embedding_width_and_range(device):
    """Materialized widths are num_embeddings * E whatever ids a batch touches;
    disjoint id ranges give exactly orthogonal gradients; ids beyond the
    declared vocab raise (the reference's test_embedding_width_is_batch_independent)."""
    from dattri_llm_amd.gradient import ops

    vocab, e, b, t = 32, 10, 4, 6
    gen = torch.Generator().manual_seed(14)
    mk = {"has_bias": False, "num_embeddings": vocab, "padding_idx": None}
    lo = torch.randint(0, 5, (b, t), generator=gen).to(device)
    hi = torch.randint(vocab - 5, vocab, (b, t), generator=gen).to(device)
    g_lo, g_hi = torch.randn(b, t, e, generator=gen).to(device), torch.randn(b, t, e, generator=gen).to(device)
    m_lo = ops.materialize_factors(lo, g_lo, "nn.Embedding", module_kwargs=mk)
    m_hi = ops.materialize_factors(hi, g_hi, "nn.Embedding", module_kwargs=mk)
    assert m_lo.shape == m_hi.shape == (b, vocab * e)
    assert torch.equal((m_lo * m_hi).sum(-1).cpu(), torch.zeros(b))
    with pytest.raises(ValueError, match="out of range"):
        ops.materialize_factors(hi, g_hi, "nn.Embedding", module_kwargs=dict(mk, num_embeddings=5))
    with pytest.raises(ValueError, match="module_kwargs"):
        ops.materialize_factors(hi, g_hi, "nn.Embedding")
    with pytest.raises(ValueError, match="negative"):
        ops.cross_gram(lo - 3, g_lo, hi, g_hi, "nn.Embedding")


def test_embedding_cross_gram_at_scale(device):
    """Long sequences with a Zipf-like id distribution (8 x 2048 against 16 x 512
    tokens, E = 1024, vocab 32000): the cross-gram, its diagonal and the
    per-token sums against the product of the materialized gradients, an fp32
    torch matmul of this build's bit-exact scatter."""
    from dattri_llm_amd import kernels

    vocab, e = 32000, 1024
    gen = torch.Generator().manual_seed(21)
    ranks = torch.arange(1, vocab + 1, dtype=torch.float64)
    probs = (1.0 / ranks) / (1.0 / ranks).sum()
    tok1 = torch.multinomial(probs, 8 * 2048, replacement=True, generator=gen).view(8, 2048)
    tok2 = torch.multinomial(probs, 16 * 512, replacement=True, generator=gen).view(16, 512)
    g1 = torch.randn(8, 2048, e, generator=gen) * 0.1
    g2 = torch.randn(16, 512, e, generator=gen) * 0.1
    d = [x.to(device) for x in (tok1, g1, tok2, g2)]
    print("embedding cross-gram at scale", flush=True)
    m1 = kernels.materialize_embedding(d[0], d[1], vocab)
    m2 = kernels.materialize_embedding(d[2], d[3], vocab)
    ref = (m1.double() @ m2.double().T).cpu().numpy()
    got = kernels.embedding_cross_gram(*d)
    assert_parity(got, ref, torch.float32, label="gram")
    per_tok = kernels.embedding_cross_gram_per_token(*d)
    assert_parity(per_tok.double().sum(1), ref, torch.float32, label="per-token sum")
    sq = kernels.embedding_cross_gram(d[0], d[1], d[0], d[1], diag=True)
    assert_parity(sq, (m1.double() ** 2).sum(-1).cpu().numpy(), torch.float32, label="norms")
    del m1, m2
