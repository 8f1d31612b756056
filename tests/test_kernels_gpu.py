"""GPU parity of the materialize, score-GEMM and norm kernels against the oracle.

Bars (conftest.assert_parity): normwise relative error <= 1e-2 for bf16/fp16
inputs (fp32 accumulation), <= 1e-3 for fp32 inputs, and a tight 1e-5 (plus
half an ulp of a 2-byte output) for what fp32 accumulation leaves against the
float64 oracle on the same rounded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_parity

pytestmark = pytest.mark.gpu



def _rand(gen, *shape, dtype, scale=None):
    x = torch.randn(*shape, generator=gen)
    if scale is not None:
        x = x * scale
    return x.to(dtype)


def _np(x):
    return x.double().cpu().numpy()


MAT_CASES = [
    # (b, t, k, d, bias)
    (2, 64, 128, 128, False),
    (3, 100, 72, 200, True),      # ragged T, partial tiles, bias column
    (1, 1, 8, 8, False),
    (2, 130, 256, 136, True),
    (4, 33, 100, 60, False),      # widths not multiples of 8 -> padded path
    (2, 100, 264, 520, False),    # 256x256-tile kernel, partial tiles on both axes
    (1, 2048, 512, 768, False),   # 256x256-tile kernel, long token axis
    (3, 77, 512, 264, True),      # 256x256 tiles, ragged last stage, bias column
    (2, 31, 256, 256, False),     # 256x256 tiles, a single partial stage
    # one side at most 64 wide (LoRA-like adapters): the narrow-layer kernel
    (3, 77, 1024, 16, False),     # narrow d, ragged last stage
    (2, 300, 16, 1000, True),     # narrow k, wide side past its last 64-column tile, bias column
    (5, 64, 64, 520, False),      # narrow k at the 64-column limit
    (4, 33, 48, 40, True),        # both sides narrow
    (6, 130, 2048, 56, False),    # narrow d of four 16-row blocks, the last partial
    (3, 77, 1024, 128, True),     # narrow d up to 128 (eight 16-row blocks)
    (2, 100, 200, 1000, False),   # narrow k up to 256 (sixteen blocks, the last partial)
    (4, 50, 136, 96, True),       # both under 256: the narrower side whole
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("out_dtype", [None, torch.float32])
@pytest.mark.parametrize("case", MAT_CASES)
def test_materialize_linear(device, dtype, out_dtype, case):
    from dattri_llm_amd import kernels

    b, t, k, d, bias = case
    gen = torch.Generator().manual_seed(sum(case))
    a = _rand(gen, b, t, k, dtype=dtype)
    g = _rand(gen, b, t, d, dtype=dtype)
    print(f"materialize case={case} dtype={dtype} out={out_dtype}", flush=True)
    got = kernels.materialize_linear(a.to(device), g.to(device), bias=bias, out_dtype=out_dtype)
    ref = oracle.materialize_linear(_np(a), _np(g), bias=bias)
    assert got.shape == ref.shape
    assert got.dtype == (out_dtype or dtype)
    assert_parity(got, ref, dtype)


def test_materialize_linear_strided(device):
    from dattri_llm_amd import kernels

    gen = torch.Generator().manual_seed(5)
    a = _rand(gen, 40, 3, 64, dtype=torch.bfloat16)  # (T, B, K) sequence-first
    g = _rand(gen, 40, 3, 32, dtype=torch.bfloat16)
    got = kernels.materialize_linear(a.to(device).transpose(0, 1), g.to(device).transpose(0, 1))
    ref = oracle.materialize_linear(_np(a.transpose(0, 1)), _np(g.transpose(0, 1)))
    assert_parity(got, ref, torch.bfloat16)


def test_materialize_linear_strided_large(device):
    """Sequence-first captures on the 256x256-tile path: token stride 3x the row."""
    from dattri_llm_amd import kernels

    gen = torch.Generator().manual_seed(6)
    a = _rand(gen, 300, 3, 512, dtype=torch.bfloat16)  # (T, B, K)
    g = _rand(gen, 300, 3, 768, dtype=torch.bfloat16)
    print("materialize strided large (3, 300, 512, 768)", flush=True)
    got = kernels.materialize_linear(a.to(device).transpose(0, 1), g.to(device).transpose(0, 1),
                                     out_dtype=torch.float32)
    ref = oracle.materialize_linear(_np(a.transpose(0, 1)), _np(g.transpose(0, 1)))
    assert_parity(got, ref, torch.bfloat16)


SCORE_CASES = [
    # (b1, b2, widths)
    (8, 64, [4096, 1024, 136]),
    (3, 5, [64]),
    (70, 20, [520, 8, 2000]),        # b1 > b2 -> transposed launch; b1 > 32
    (1, 1, [8]),
    (33, 130, [4104]),
    (4, 64, [16384] * 6 + [0, 136] + [16384] * 6),  # workgroup ranges across layers, an empty layer
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", SCORE_CASES)
def test_score_gemm(device, dtype, case):
    from dattri_llm_amd import kernels

    b1, b2, widths = case
    gen = torch.Generator().manual_seed(b1 * 7 + b2)
    pairs = [(_rand(gen, b1, w, dtype=dtype), _rand(gen, b2, w, dtype=dtype)) for w in widths]
    print(f"score_gemm case={case} dtype={dtype}", flush=True)
    got = kernels.score_gemm([(m1.to(device), m2.to(device)) for m1, m2 in pairs])
    ref = oracle.score_gemm([_np(m1) for m1, _ in pairs], [_np(m2) for _, m2 in pairs])
    assert got.shape == (b1, b2)
    assert_parity(got, ref, dtype)
    # accumulate into an existing result
    kernels.score_gemm([(m1.to(device), m2.to(device)) for m1, m2 in pairs], out=got, accumulate=True)
    assert_parity(got, 2 * ref, dtype)


NORM_CASES = [
    # (b, t, d, layer_type, bias, eps)
    (2, 70, 4096, "nn.RMSNorm", False, 1e-6),
    (3, 33, 128, "nn.RMSNorm", False, None),      # eps=None -> dtype machine eps
    (2, 64, 136, "nn.LayerNorm", True, 1e-5),
    (4, 1, 64, "nn.LayerNorm", False, 1e-5),
    (1, 300, 1024, "nn.RMSNorm", False, 1e-5),
    # widths that end inside a 16-byte chunk: zero-padded rows, masked in the kernels
    (3, 40, 6, "nn.LayerNorm", True, 1e-5),
    (2, 33, 101, "nn.RMSNorm", False, 1e-6),
    (2, 70, 4099, "nn.LayerNorm", False, 1e-5),  # fp32: past the register form, the wide form
    (2, 37, 9000, "nn.LayerNorm", True, 1e-5),   # both dtypes in the wide form
    # 16-bit rows of 8 KB in the LDS ring: 64, 32 and 16 token rows per workgroup on 256 CUs
    (8, 2048, 4096, "nn.RMSNorm", False, 1e-6),
    (1, 8192, 4096, "nn.RMSNorm", False, 1e-6),
    (3, 1000, 4096, "nn.LayerNorm", True, 1e-5),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", NORM_CASES)
def test_norm_weight_grad(device, dtype, case):
    from dattri_llm_amd import kernels

    b, t, d, lt, bias, eps = case
    eps_v = torch.finfo(dtype).eps if eps is None else eps
    gen = torch.Generator().manual_seed(b + t + d)
    x = _rand(gen, b, t, d, dtype=dtype)
    g = _rand(gen, b, t, d, dtype=dtype)
    print(f"norm case={case} dtype={dtype}", flush=True)
    got = kernels.norm_weight_grad(x.to(device), g.to(device), kind=kernels.NORM_KIND[lt],
                                   eps=eps_v, bias=bias, out_dtype=torch.float32)
    ref = oracle.norm_weight_grad(_np(x), _np(g), lt, eps_v, bias)
    assert got.shape == ref.shape
    assert_parity(got, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("lt", ["nn.RMSNorm", "nn.LayerNorm"])
@pytest.mark.parametrize("d", [256, 6, 203, 9001])
def test_norm_xhat(device, dtype, lt, d):
    from dattri_llm_amd import kernels

    gen = torch.Generator().manual_seed(3)
    x = _rand(gen, 3, 17, d, dtype=dtype, scale=3.0)
    fn = oracle.rms_x_hat if lt == "nn.RMSNorm" else oracle.layer_norm_x_hat
    got = kernels.norm_xhat(x.to(device), kind=kernels.NORM_KIND[lt], eps=1e-5, out_dtype=torch.float32)
    assert_parity(got, fn(_np(x), 1e-5), dtype)


@pytest.mark.parametrize("shape", [(3, 70, 128, 200), (8, 256, 512, 520), (2, 33, 64, 8)])
def test_blocked_materialize_equals_plain(device, shape):
    """The k-blocked dW layout holds exactly the plain layout's values."""
    from dattri_llm_amd import kernels

    b, t, k, d = shape
    gen = torch.Generator().manual_seed(b * t)
    a = _rand(gen, b, t, k, dtype=torch.bfloat16).to(device)
    g = _rand(gen, b, t, d, dtype=torch.bfloat16).to(device)
    plain = kernels.materialize_linear(a, g)
    blk = kernels.materialize_linear(a, g, blocked=True)
    assert kernels.is_blocked(blk) and blk.shape == (b, d * k // 64, 64)
    assert blk.stride() == (64, b * 64, 1)
    assert torch.equal(blk.reshape(b, -1), plain)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b1", [8, 17, 64, 100])
def test_score_gemm_blocked_operands(device, dtype, b1):
    """k-blocked and row-major layers mixed in one launch.  b1 <= 16 takes the
    16 x 64 ring tile; taller side-1 blocks the 64 x 64 tile (one tile at 17
    and 64 rows, two row tiles at 100, whose side-2 rows then keep the default
    load policy)."""
    from dattri_llm_amd import kernels

    gen = torch.Generator().manual_seed(21 + b1)
    pairs, m1s, m2s = [], [], []
    for w, (bl1, bl2) in [(4096, (True, True)), (1024, (False, True)), (192, (True, False)), (136, (False, False))]:
        m1, m2 = _rand(gen, b1, w, dtype=dtype), _rand(gen, 64, w, dtype=dtype)
        m1s.append(_np(m1))
        m2s.append(_np(m2))

        def block(m, on):
            if not on:
                return m.to(device)
            buf = kernels.blocked_storage(m.shape[0], m.shape[1], dtype, device)
            buf.copy_(m.view(m.shape[0], -1, 64).to(device))
            return buf

        pairs.append((block(m1, bl1), block(m2, bl2)))
    got = kernels.score_gemm(pairs)
    assert_parity(got, oracle.score_gemm(m1s, m2s), dtype)
    got_t = kernels.score_gemm([(q, p) for p, q in pairs])  # transposed launch (B1 > B2)
    assert_parity(got_t, oracle.score_gemm(m2s, m1s), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b1", [8, 64])
def test_score_gemm_wide_row_strides(device, dtype, b1):
    """Layers sliced out of 64 MiB rows: 63 row strides exceed a 32-bit buffer
    offset, so the rings give every DMA instruction its own base (8 rows of
    offsets).  b1 = 8 takes the 16 x 64 tile, b1 = 64 the 64 x 64 tile."""
    from dattri_llm_amd import kernels

    ld = (64 << 20) // torch.tensor([], dtype=dtype).element_size()
    gen = torch.Generator().manual_seed(31 + b1)
    widths = [4096, 136]
    m1s = [_rand(gen, b1, w, dtype=dtype) for w in widths]
    m2s = [_rand(gen, 64, w, dtype=dtype) for w in widths]
    buf1 = torch.empty(b1, ld, dtype=dtype, device=device)
    buf2 = torch.empty(64, ld, dtype=dtype, device=device)
    pairs, off = [], 0
    for m1, m2, w in zip(m1s, m2s, widths):
        buf1[:, off:off + w] = m1.to(device)
        buf2[:, off:off + w] = m2.to(device)
        pairs.append((buf1[:, off:off + w], buf2[:, off:off + w]))
        off += w
    print(f"score_gemm wide strides b1={b1} dtype={dtype} ld={ld}", flush=True)
    got = kernels.score_gemm(pairs)
    assert_parity(got, oracle.score_gemm([_np(m) for m in m1s], [_np(m) for m in m2s]), dtype)
    del buf1, buf2


PROJ_CASES = [
    # (b, t, k, d, ka, kg, bias, dtype, seq_first)
    (3, 300, 200, 136, 24, 40, True, torch.bfloat16, False),   # 3 chunks, ragged; widths not whole stages
    (2, 128, 4096, 1024, 64, 64, False, torch.bfloat16, False),
    (2, 77, 100, 36, 64, 16, True, torch.float32, False),      # fp32 rows
    (3, 50, 512, 264, 32, 64, False, torch.bfloat16, True),    # sequence-first captures (token stride B*width)
    (9, 260, 2048, 4096, 64, 64, True, torch.float16, False),  # 3 chunks per sample, fp16
    (40, 128, 1024, 2752, 64, 48, False, torch.bfloat16, False),  # more stages than workgroups
    # short samples packed into 128-row items (several samples per item)
    (40, 16, 512, 264, 64, 48, True, torch.bfloat16, False),
    (7, 100, 1024, 2752, 64, 64, True, torch.float16, False),  # samples straddle items
    (33, 1, 256, 128, 32, 16, True, torch.float32, False),     # one token per sample
    (9, 127, 2048, 512, 48, 64, False, torch.bfloat16, False),
    (6, 40, 512, 264, 64, 32, True, torch.bfloat16, "slice"),  # batch stride above T rows: not packed
    (12, 30, 256, 136, 24, 40, False, torch.bfloat16, True),   # sequence-first: not packed
    # samples over several items (partial blocks of M), contracted items and split ones
    (4, 256, 512, 264, 64, 48, True, torch.bfloat16, False),
    (5, 300, 256, 136, 32, 64, True, torch.bfloat16, "slice"),
    (3, 4096, 4096, 1024, 64, 64, False, torch.bfloat16, False),
    (1, 1000, 1024, 512, 64, 64, True, torch.float16, False),
    (50, 10, 256, 128, 64, 64, False, torch.bfloat16, False),  # under 16 rows a sample: pieces only
]


@pytest.mark.parametrize("case", PROJ_CASES)
def test_project_outer_kernel(device, case):
    from dattri_llm_amd import kernels

    b, t, k, d, ka, kg, bias, dtype, seq_first = case
    print(f"project_outer case={case}", flush=True)
    gen = torch.Generator().manual_seed(b * t + k)
    if seq_first == "slice":  # sliced on the device: a copy would be made dense
        a_full, g_full = _rand(gen, b, t + 8, k, dtype=dtype), _rand(gen, b, t + 8, d, dtype=dtype)
        a, g = a_full[:, 3:3 + t], g_full[:, 5:5 + t]
        a_dev, g_dev = a_full.to(device)[:, 3:3 + t], g_full.to(device)[:, 5:5 + t]
        assert a_dev.stride(0) != t * a_dev.stride(1)
    elif seq_first:
        a = _rand(gen, t, b, k, dtype=dtype).transpose(0, 1)
        g = _rand(gen, t, b, d, dtype=dtype).transpose(0, 1)
    else:
        a, g = _rand(gen, b, t, k, dtype=dtype), _rand(gen, b, t, d, dtype=dtype)
    p_in = _rand(gen, k, ka, dtype=dtype, scale=k**-0.5)
    p_out = _rand(gen, d, kg, dtype=dtype, scale=d**-0.5)
    bias_in = torch.randn(ka, generator=gen) if bias else None
    if seq_first != "slice":
        a_dev, g_dev = a.to(device), g.to(device)
    got = kernels.project_outer(a_dev, g_dev, p_in.t().contiguous().to(device),
                                p_out.t().contiguous().to(device),
                                bias_in=bias_in.to(device) if bias else None, out_dtype=torch.float32)
    p_in_np = _np(p_in)
    if bias:
        p_in_np = np.concatenate([p_in_np, bias_in.double().numpy()[None, :]], axis=0)
    want = oracle.project_outer(_np(a), _np(g), p_in_np, _np(p_out), bias=bias)
    assert got.shape == (b, kg * ka)
    assert_parity(got, want, dtype)


DIAG_CASES = [
    # (b, s1, s2, k, d, bias, same_block)
    (5, 128, 128, 64, 64, False, True),
    (3, 300, 300, 72, 40, True, True),     # ragged S, two row tiles
    (4, 96, 200, 128, 256, True, False),   # two blocks of one batch, S1 != S2
    (1, 1, 1, 8, 8, False, True),
    (6, 520, 77, 264, 136, False, False),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", DIAG_CASES)
def test_ghost_gram_diag(device, dtype, case):
    """The ghost product on the diagonal pairs (per-sample dots / norms) equals
    the diagonal of the oracle's full cross-gram."""
    from dattri_llm_amd import kernels

    b, s1, s2, k, d, bias, same = case
    gen = torch.Generator().manual_seed(b * s1 + k)
    a1, g1 = _rand(gen, b, s1, k, dtype=dtype, scale=k**-0.5), _rand(gen, b, s1, d, dtype=dtype, scale=d**-0.5)
    a2, g2 = (a1, g1) if same else (_rand(gen, b, s2, k, dtype=dtype, scale=k**-0.5),
                                    _rand(gen, b, s2, d, dtype=dtype, scale=d**-0.5))
    print(f"ghost_gram_diag case={case} dtype={dtype}", flush=True)
    x1, y1 = a1.to(device), g1.to(device)
    x2, y2 = (x1, y1) if same else (a2.to(device), g2.to(device))
    got = kernels.ghost_gram_diag(x1, y1, x2, y2, bias=bias)
    want = np.diag(oracle.cross_gram_factorized(_np(a1), _np(g1), _np(a2), _np(g2), bias=bias))
    assert got.shape == (b,)
    assert_parity(got, want, dtype)
    kernels.ghost_gram_diag(x1, y1, x2, y2, bias=bias, out=got, accumulate=True)
    assert_parity(got, 2 * want, dtype)


ROW_DOT_CASES = [
    # (rows, [(width, blocked1, blocked2 or None for a squared norm)])
    (8, [(4096, True, True), (1024, False, False), (136, False, None)]),
    (64, [(16384, True, None), (4096, True, False)]),
    (3, [(64, False, None)]),
    (130, [(2048, True, True), (200, False, False)]),   # two row tiles (bf16), ragged widths
    (1, [(8192, True, None)]),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", ROW_DOT_CASES)
def test_row_dots(device, dtype, case):
    """Per-row dot products (or squared norms) summed over dense layers, row-major
    and k-blocked operands read in place, against float64 sums."""
    from dattri_llm_amd import kernels

    rows, spec = case
    gen = torch.Generator().manual_seed(rows + len(spec))
    layers, want = [], np.zeros(rows)
    for w, bl1, bl2 in spec:
        m1 = _rand(gen, rows, w, dtype=dtype)
        m2 = None if bl2 is None else _rand(gen, rows, w, dtype=dtype)
        want += (_np(m1) * (_np(m1) if m2 is None else _np(m2))).sum(1)

        def place(m, blocked):
            if not blocked or w % 64:
                return m.to(device)
            buf = kernels.blocked_storage(rows, w, dtype, device)
            buf.copy_(m.view(rows, -1, 64).to(device))
            return buf

        layers.append((place(m1, bl1), None if m2 is None else place(m2, bl2)))
    print(f"row_dots rows={rows} layers={spec} dtype={dtype}", flush=True)
    got = kernels.row_dots(layers)
    assert got.shape == (rows,)
    assert_parity(got, want, dtype)
    kernels.row_dots(layers, out=got, accumulate=True)
    assert_parity(got, 2 * want, dtype)
