"""GPU parity of the K-FAC / EK-FAC ops (gradient/ops/kronecker.py) against the
oracle: covariances and Fisher through the dW kernel, the whitened cross-gram
through cross_gram, the EK-FAC eigenbasis coordinates through the dW kernel.

Bars (conftest.assert_parity): normwise relative error <= 1e-2 for bf16
inputs, <= 1e-3 for fp32, and a tight bound for what fp32 accumulation leaves
(1e-5, plus half an ulp of a bf16 result); the oracle runs in float64 on the
same rounded inputs."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_parity, rel_err, roundings

pytestmark = pytest.mark.gpu

LIN = "nn.Linear"


def _factors(seed, b, t, k, d, dtype):
    gen = torch.Generator().manual_seed(seed)
    a = (torch.randn(b, t, k, generator=gen) / k**0.5).to(dtype)
    g = (torch.randn(b, t, d, generator=gen) / d**0.5).to(dtype)
    return a, g


def _np(x):
    return x.double().cpu().numpy()


def _ones(a):
    return np.concatenate([a, np.ones(a.shape[:-1] + (1,))], axis=-1)


def _spd_inv(seed, n):
    rng = np.random.default_rng(seed)
    m = rng.standard_normal((n, n))
    return np.linalg.inv(m @ m.T / n + 0.5 * np.eye(n))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bias", [False, True])
def test_kfac_factors(device, dtype, bias):
    from dattri_llm_amd.gradient import ops

    print(f"kfac_factors {dtype} bias={bias}", flush=True)
    a, g = _factors(1, 4, 96, 72, 40, dtype)
    g[1, 5:20] = 0  # gradient-free rows are dropped from both factors and the count
    mk = {"has_bias": bias}
    big_a, big_g = ops.kfac_factors(a.to(device), g.to(device), LIN, mk)
    a_np = _ones(_np(a)) if bias else _np(a)
    ref_a, ref_g = oracle.kfac_factors(a_np, _np(g))
    assert big_a.dtype == torch.float32 and big_a.shape == ref_a.shape
    assert_parity(big_a, ref_a, dtype)
    assert_parity(big_g, ref_g, dtype)


def test_kfac_factors_row_chunks_and_errors(device, monkeypatch):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.ops import kronecker

    a, g = _factors(2, 3, 200, 64, 48, torch.bfloat16)
    whole = ops.kfac_factors(a.to(device), g.to(device), LIN)
    monkeypatch.setattr(kronecker, "_GRAM_BYTES", 64 * 2 * 37)  # 37-row chunks
    chunked = ops.kfac_factors(a.to(device), g.to(device), LIN)
    for x, y in zip(whole, chunked):
        assert rel_err(y.cpu().double().numpy(), x.cpu().double().numpy()) < 1e-5
    with pytest.raises(ValueError):
        ops.kfac_factors(a.to(device), torch.zeros_like(g).to(device), LIN)
    with pytest.raises(NotImplementedError):
        ops.kfac_factors(a.to(device), g.to(device), "nn.RMSNorm", None)


def test_fim_factors(device):
    from dattri_llm_amd.gradient import ops

    a, g = _factors(3, 6, 64, 24, 16, torch.bfloat16)
    f = ops.fim_factors(a.to(device), g.to(device), LIN)
    ref = oracle.fim_factors(oracle.materialize_linear(_np(a), _np(g)))
    assert f.dtype == torch.float32
    # the per-sample gradients are formed in bf16 (the compute dtype), then squared
    assert_parity(f, ref, torch.bfloat16, tight=roundings(2))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bias", [False, True])
def test_kfac_cross_factors(device, dtype, bias):
    from dattri_llm_amd.gradient import ops

    print(f"kfac_cross_factors {dtype} bias={bias}", flush=True)
    a1, g1 = _factors(4, 3, 80, 64, 48, dtype)
    a2, g2 = _factors(5, 2, 112, 64, 48, dtype)
    kb = 64 + int(bias)
    a_inv, g_inv = _spd_inv(6, kb), _spd_inv(7, 48)
    mk = {"has_bias": bias}
    got = ops.kfac_cross_factors(
        a1.to(device), g1.to(device), a2.to(device), g2.to(device), LIN,
        torch.tensor(a_inv, dtype=torch.float32, device=device),
        torch.tensor(g_inv, dtype=torch.float32, device=device), mk, mk,
    )
    f = (lambda x: _ones(x)) if bias else (lambda x: x)
    ref = oracle.kfac_cross_factors(f(_np(a1)), _np(g1), f(_np(a2)), _np(g2),
                                    np.float32(a_inv).astype(np.float64), np.float32(g_inv).astype(np.float64))
    assert got.shape == ref.shape
    assert_parity(got, ref, dtype)

    # whitening one side once (kfac_precondition) then a plain cross_gram gives the same scores
    from dattri_llm_amd.gradient.gradient import Factorized

    f1 = Factorized(a1.to(device), g1.to(device), module_kwargs=mk)
    wa, wg = ops.kfac_precondition(f1, LIN, torch.tensor(a_inv, dtype=torch.float32, device=device),
                                   torch.tensor(g_inv, dtype=torch.float32, device=device))
    a2p, g2p = ops.preprocess_factors(a2.to(device), g2.to(device), LIN, mk)
    again = ops.cross_gram(wa, wg, a2p, g2p, LIN)
    assert_parity(again, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ekfac_rotation_and_precondition(device, dtype):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized

    a, g = _factors(8, 3, 64, 32, 24, dtype)
    _, u_a = np.linalg.eigh(np.linalg.inv(_spd_inv(9, 32)))
    _, u_g = np.linalg.eigh(np.linalg.inv(_spd_inv(10, 24)))
    ua = torch.tensor(u_a, dtype=torch.float32, device=device)
    ug = torch.tensor(u_g, dtype=torch.float32, device=device)
    u_a32, u_g32 = np.float32(u_a).astype(np.float64), np.float32(u_g).astype(np.float64)
    rot = ops.ekfac_materialize(Factorized(a.to(device), g.to(device)), LIN, ua, ug)
    ref = oracle.ekfac_materialize_factors(_np(a), _np(g), u_a32, u_g32)
    assert_parity(rot, ref, dtype)
    # a materialized block rotates to the same coordinates
    dense = ops.materialize_factors(a.to(device), g.to(device), LIN)
    rot_d = ops.ekfac_materialize(dense, LIN, ua, ug)
    # the dense block is stored in the compute dtype before the rotation
    assert_parity(rot_d, ref, dtype, tight=roundings(1) if dtype == torch.bfloat16 else None)
    lam = torch.linspace(0.5, 2.0, 24 * 32, device=device)
    pre = ops.ekfac_precondition(rot, ua, ug, lam, LIN)
    ref_pre = oracle.ekfac_precondition(ref, u_a32, u_g32, _np(lam))
    assert_parity(pre, ref_pre, dtype)


def test_kfac_precondition_materialized(device):
    from dattri_llm_amd.gradient import ops

    gen = torch.Generator().manual_seed(11)
    block = torch.randn(5, 16 * 12, generator=gen)
    a_inv, g_inv = _spd_inv(12, 12), _spd_inv(13, 16)
    got = ops.kfac_precondition_materialized(block.to(device), torch.tensor(a_inv, dtype=torch.float32, device=device),
                                             torch.tensor(g_inv, dtype=torch.float32, device=device))
    ref = oracle.kfac_precondition_materialized(_np(block), np.float32(a_inv), np.float32(g_inv))
    assert_parity(got, ref, torch.float32)


def test_accumulators_match_one_shot(device):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.gradient import Factorized, Gradient

    blocks = [_factors(20 + i, 3, 48, 40, 24, torch.bfloat16) for i in range(3)]
    kacc, facc = ops.KroneckerAccumulator(), ops.FisherAccumulator()
    for a, g in blocks:
        grad = Gradient({"fc": "factorized"}, {"fc": Factorized(a.to(device), g.to(device))}, {"fc": LIN})
        kacc.update(grad, ["fc"])
        facc.update(grad, ["fc"])
    big_a, big_g = kacc.result()["fc"]
    a_all = np.concatenate([_np(a) for a, _ in blocks])
    g_all = np.concatenate([_np(g) for _, g in blocks])
    ref_a, ref_g = oracle.kfac_factors(a_all, g_all)
    assert_parity(big_a, ref_a, torch.bfloat16)
    assert_parity(big_g, ref_g, torch.bfloat16)
    ref_f = oracle.fim_factors(oracle.materialize_linear(a_all, g_all))
    # bf16 per-sample gradients, squared, and a bf16 result (the reference keeps the gradients' dtype)
    assert_parity(facc.result()["fc"], ref_f, torch.bfloat16, tight=roundings(3))
    capped = ops.FisherAccumulator(max_params=100)
    capped.update(Gradient({"fc": "factorized"}, {"fc": Factorized(*[x.to(device) for x in blocks[0]])},
                           {"fc": LIN}), ["fc"])
    assert capped.skipped == {"fc": 40 * 24} and capped.result() == {}


# ---- the symmetric row Gram (da_row_gram) on its own -------------------------

def _rows(seed, n, p, dtype):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(n, p, generator=gen) / p**0.25).to(dtype)


def _off_diagonal_tiles_mirrored(out, tile=256):
    """Tiles below the diagonal are copies of the ones above it, bit for bit."""
    p = out.shape[0]
    for i in range(tile, p, tile):
        for j in range(0, i, tile):
            if not torch.equal(out[i:i + tile, j:j + tile], out[j:j + tile, i:i + tile].T):
                return False
    return True


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,p", [(1000, 40), (5000, 264), (777, 520), (3000, 1032), (64, 300), (1, 8)])
def test_row_gram_kernel(device, dtype, n, p):
    from dattri_llm_amd import kernels

    x = _rows(n + p, n, p, dtype)
    want = x.double().T @ x.double()
    got = kernels.row_gram(x.to(device))
    torch.cuda.synchronize()
    assert got.shape == (p, p) and got.dtype == torch.float32
    # exactly representable inputs, fp32 accumulation: far inside the fp32 bar
    assert_parity(got, want, torch.bfloat16)
    assert _off_diagonal_tiles_mirrored(got.cpu())


def test_row_gram_accumulate_and_out_stride(device):
    from dattri_llm_amd import kernels

    p = 520
    x1, x2 = _rows(1, 900, p, torch.bfloat16), _rows(2, 1300, p, torch.bfloat16)
    base = torch.full((p, p + 8), float("nan"), device=device)
    out = base[:, :p]  # row stride p + 8: the 8 columns past p must stay untouched
    kernels.row_gram(x1.to(device), out=out)
    kernels.row_gram(x2.to(device), out=out, accumulate=True)
    want = x1.double().T @ x1.double() + x2.double().T @ x2.double()
    assert_parity(out, want, torch.bfloat16)
    assert torch.isnan(base[:, p:]).all()
    kernels.row_gram(x1[:0].to(device), out=out, accumulate=True)  # no rows: unchanged
    assert_parity(out, want, torch.bfloat16)
    assert torch.equal(kernels.row_gram(x1[:0].to(device)).cpu(), torch.zeros(p, p))
    with pytest.raises(ValueError):
        kernels.row_gram(x1.float().to(device))
    with pytest.raises(ValueError):
        kernels.row_gram(x1.to(device), accumulate=True)


def _row_gram_raw(x, ws, out=None, accumulate=False):
    """da_row_gram through the C ABI with an explicit workspace (None: none)."""
    from dattri_llm_amd import _native as nat

    p = x.shape[1]
    out = torch.empty(p, p, dtype=torch.float32, device=x.device) if out is None else out
    nat.check(nat.load().da_row_gram(x.data_ptr(), nat.DA_BF16, x.shape[0], p, x.stride(0), out.data_ptr(),
                                     out.stride(0), int(accumulate), None if ws is None else ws.data_ptr(),
                                     0 if ws is None else ws.numel(), torch.cuda.current_stream().cuda_stream),
              "row_gram")
    return out


def _row_gram_ws(n, p):
    import ctypes

    from dattri_llm_amd import _native as nat

    need = ctypes.c_size_t(0)
    nat.check(nat.load().da_row_gram_workspace(n, p, nat.DA_BF16, ctypes.byref(need)), "row_gram_workspace")
    return need.value


def test_row_gram_row_chunks(device):
    """Rows 4 MiB apart.  Without a workspace the entry point takes the rows in
    chunks whose buffer offsets stay below 2^31 bytes (479 + 479 + 42 rows),
    each adding to the output; with one, in token splits of at most 479 rows
    summed by the second pass.  Both equal the float64 product."""
    n, p, stride = 1000, 264, 1 << 21
    x = _rows(7, n, p, torch.bfloat16)
    big = torch.zeros(n, stride, dtype=torch.bfloat16, device=device)
    big[:, :p] = x.to(device)
    want = x.double().T @ x.double()
    chunked = _row_gram_raw(big[:, :p], None)
    need = _row_gram_ws(n, p)
    assert need > 0  # a 2 x 2 triangle of tiles: splits pay
    split = _row_gram_raw(big[:, :p], torch.empty(need, dtype=torch.uint8, device=device))
    torch.cuda.synchronize()
    assert_parity(chunked, want, torch.bfloat16)
    assert_parity(split, want, torch.bfloat16)
    del big


def _dev_rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


@pytest.mark.parametrize("n,p", [(16384, 1024), (16384, 4096), (3000, 520), (700, 8), (4096, 5888)])
def test_row_gram_token_splits(device, n, p):
    """Token splits (workspace) against one pass (no workspace): the same
    product to fp32 rounding, with and without accumulation, twice in a row on
    one workspace (each call rewrites every partial it reads), and a workspace
    too small for the planned splits falls back to fewer.  Width 5888 has 276
    tiles: 256 run over all rows and the last 20 as splits."""
    x = _rows(11 + p, n, p, torch.bfloat16).to(device)
    need = _row_gram_ws(n, p)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
    one = _row_gram_raw(x, None)
    split = _row_gram_raw(x, ws)
    again = _row_gram_raw(x, ws)
    base = torch.randn(p, p, device=device)
    base = base + base.T  # an accumulator of Grams is symmetric (the lower tiles are rewritten by the mirror)
    acc = _row_gram_raw(x, ws, out=base.clone(), accumulate=True)
    small = _row_gram_raw(x, ws[: need // 2] if need > 1 else None)
    torch.cuda.synchronize()
    assert need > 0  # every case here plans splits
    assert torch.equal(split, again)
    for got in (split, small):
        assert _dev_rel(got, one) <= 1e-5
    assert _dev_rel(acc, one + base) <= 1e-5
    assert _off_diagonal_tiles_mirrored(split)


def test_gradient_free_rows_match_the_reference_rule(device):
    """Token rows are dropped exactly when every gradient entry compares equal
    to zero (kronecker.py:65-81: (g != 0).any(1)); -0.0 rows go, rows holding
    only a NaN, an inf or a subnormal stay."""
    from dattri_llm_amd.gradient.ops import kronecker

    g = torch.randn(9, 40).bfloat16()
    g[1] = 0
    g[2] = -0.0
    g[3] = 0
    g[3, 5] = float("nan")
    g[4] = 0
    g[4, 0] = -1e-38  # subnormal in bf16
    g[5] = 0
    g[5, 7] = float("inf")
    g[6] = 0
    a = torch.randn(9, 24).bfloat16()
    want = (g != 0).any(dim=1)
    a_f, g_f = kronecker._drop_gradient_free_rows(a.to(device), g.to(device))
    assert torch.equal(a_f.cpu(), a[want])  # the activation rows kept are exactly the reference's
    got, ref = g_f.cpu(), g[want]  # (NaN != NaN, so compare with the NaNs replaced)
    assert torch.equal(torch.isnan(got), torch.isnan(ref)) and torch.equal(got.nan_to_num(7.0), ref.nan_to_num(7.0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("width", [8, 40, 300, 14336])
def test_nonzero_rows_kernel(device, dtype, width):
    """da_nonzero_rows against (x != 0).any(1) on the CPU: random rows, all-zero
    and -0.0 rows, rows whose only nonzero is a NaN, an inf, a subnormal or
    the last column (past padding when the width is not a chunk multiple)."""
    from dattri_llm_amd import kernels

    gen = torch.Generator().manual_seed(width)
    x = torch.randn(64, width, generator=gen).to(dtype)
    x[1:9] = 0
    x[2] = -0.0
    x[3, width // 2] = float("nan")
    x[4, 0] = float("-inf")
    x[5, 1] = torch.finfo(dtype).tiny / 4  # subnormal (a nonzero bit pattern in every dtype)
    x[6, width - 1] = 1.0
    want = (x != 0).any(dim=1)
    got = kernels.nonzero_rows(x.to(device))
    assert got.dtype == torch.bool and torch.equal(got.cpu(), want)
    assert kernels.nonzero_rows(x[:0].to(device)).numel() == 0
    view = torch.zeros(16, width + 8, dtype=dtype)
    view[3, 2] = 5
    got_view = kernels.nonzero_rows(view.to(device)[:, :width])  # strided rows
    assert torch.equal(got_view.cpu(), (view[:, :width] != 0).any(dim=1))
