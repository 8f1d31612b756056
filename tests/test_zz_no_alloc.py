"""The allocation-free score GEMM (``da_score_gemm_noalloc``) against
``da_score_gemm`` with a caller workspace, through the C ABI.

Both entry points run the same kernels and the same fixed-order reduction,
so their outputs must be bit-identical.  Two calls in a row, the second on a
smaller problem, check that nothing left in the shared device scratch by the
first call leaks into the second.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


def _lib():
    from dattri_llm_amd import _native as nat

    return nat, nat.load()


def _layer_array(nat, pairs):
    layers = [nat.DenseLayer(m1.data_ptr(), m2.data_ptr(), m1.shape[1], m1.stride(0), m2.stride(0), 64, 64)
              for m1, m2 in pairs]
    return (nat.DenseLayer * len(layers))(*layers)


def _pairs(b1, b2, widths, dtype, device, seed):
    gen = torch.Generator().manual_seed(seed)
    return [(torch.randn(b1, w, generator=gen).to(dtype).to(device),
             torch.randn(b2, w, generator=gen).to(dtype).to(device)) for w in widths]


def _run_both(b1, b2, pairs, dtype, device, accumulate=False, seed=0):
    nat, lib = _lib()
    arr = _layer_array(nat, pairs)
    code = nat.dtype_code(dtype)
    stream = torch.cuda.current_stream(device).cuda_stream
    init = torch.randn(b1, b2, generator=torch.Generator().manual_seed(seed + 99)).to(device)
    out_ws = init.clone()
    out_na = init.clone()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_score_gemm_workspace(b1, b2, arr, len(pairs), code, ctypes.byref(nbytes)), "workspace")
    ws = torch.empty(max(nbytes.value, 16), dtype=torch.uint8, device=device)
    nat.check(lib.da_score_gemm(b1, b2, arr, len(pairs), code, out_ws.data_ptr(), out_ws.stride(0), 1,
                                int(accumulate), ws.data_ptr(), ws.numel(), stream), "da_score_gemm")
    nat.check(lib.da_score_gemm_noalloc(b1, b2, arr, len(pairs), code, out_na.data_ptr(), out_na.stride(0), 1,
                                        int(accumulate), stream), "da_score_gemm_noalloc")
    torch.cuda.synchronize(device)
    ref = sum(m1.double().cpu() @ m2.double().cpu().T for m1, m2 in pairs)
    if accumulate:
        ref = ref + init.double().cpu()
    return out_ws.cpu(), out_na.cpu(), ref, nbytes.value


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_on_two_calls(device, dtype):
    """A large call, then a smaller one: bit-identical to da_score_gemm both times."""
    cases = [
        (8, 64, [65536, 4096, 12288]) if dtype == torch.bfloat16 else (4, 8, [20000, 512]),
        (3, 17, [1024, 192]) if dtype == torch.bfloat16 else (2, 3, [256]),
    ]
    used = []
    for n, (b1, b2, widths) in enumerate(cases):
        print(f"noalloc case {n}: {dtype} {b1}x{b2} widths {widths}", flush=True)
        pairs = _pairs(b1, b2, widths, dtype, device, seed=n)
        out_ws, out_na, ref, nbytes = _run_both(b1, b2, pairs, dtype, device, seed=n)
        used.append(nbytes)
        assert torch.equal(out_ws, out_na), float((out_ws - out_na).abs().max())
        assert rel_err(out_na.numpy(), ref.numpy()) <= 1e-5
    assert used[1] < used[0]  # the second call is the smaller problem


def test_noalloc_accumulates_like_workspace_entry(device):
    pairs = _pairs(5, 40, [8192, 64], torch.bfloat16, device, seed=7)
    out_ws, out_na, ref, _ = _run_both(5, 40, pairs, torch.bfloat16, device, accumulate=True, seed=7)
    assert torch.equal(out_ws, out_na)
    assert rel_err(out_na.numpy(), ref.numpy()) <= 1e-5


def test_noalloc_rejects_problems_beyond_its_scratch(device):
    """Every output keeps at least one fp32 partial per workgroup of its tile:
    2048 x 2048 outputs need 16 MiB of partials at one workgroup per tile,
    more than the scratch holds.  The call fails before any launch and leaves
    out untouched."""
    nat, lib = _lib()
    n = 2048
    pairs = _pairs(n, n, [64], torch.float32, device, seed=3)
    arr = _layer_array(nat, pairs)
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_score_gemm_workspace(n, n, arr, 1, nat.DA_F32, ctypes.byref(nbytes)), "workspace")
    assert nbytes.value > 8 << 20
    out = torch.full((n, n), 3.0, device=device)
    status = lib.da_score_gemm_noalloc(n, n, arr, 1, nat.DA_F32, out.data_ptr(), n, 1, 0,
                                       torch.cuda.current_stream(device).cuda_stream)
    assert status == nat.DA_ERR_WORKSPACE
    assert b"scratch" in lib.da_last_error()
    torch.cuda.synchronize(device)
    assert bool((out == 3.0).all())
