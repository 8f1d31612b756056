"""Typed torch-tensor wrappers over the C-ABI entry points.

Each wrapper checks shapes, brings operands into the layout the kernel
requires (16-byte aligned rows, widths a multiple of one 16-byte chunk --
padding with zero features when needed, which changes no product), allocates
outputs and workspace from torch's caching allocator and launches on the
current stream of the tensors' device.  No arithmetic happens here.
"""

from __future__ import annotations

import ctypes

import torch

from dattri_llm_amd import _native as nat


def _chunk_elems(dtype: torch.dtype) -> int:
    return 16 // nat.ELEM_BYTES[dtype]


def _aligned(x: torch.Tensor) -> bool:
    es = x.element_size()
    if x.stride(-1) != 1 or x.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 for s in x.stride()[:-1])


def prepare_rows(x: torch.Tensor, width: int | None = None) -> torch.Tensor:
    """Return *x* (..., K) with 16-byte aligned rows whose width is a multiple
    of one 16-byte chunk: *x* itself when it already is, else a zero-padded copy
    of width ``width`` (default: K rounded up to a chunk)."""
    k = x.shape[-1]
    vec = _chunk_elems(x.dtype)
    target = width if width is not None else -(-k // vec) * vec
    if target == k and _aligned(x):
        return x
    out = torch.zeros(*x.shape[:-1], target, dtype=x.dtype, device=x.device)
    out[..., :k] = x
    return out


def _side(a: torch.Tensor, g: torch.Tensor, bias: bool, seg=None, index=None, tokens=None):
    side = nat.FactorSide()
    side.act = a.data_ptr()
    side.grad = g.data_ptr()
    if seg is None:
        side.batch = a.shape[0]
        side.tokens = a.shape[1]
        side.act_bstride, side.act_tstride = a.stride(0), a.stride(1)
        side.grad_bstride, side.grad_tstride = g.stride(0), g.stride(1)
        side.seg_offsets = None
        side.row_index = None
    else:
        side.batch = seg.numel() - 1
        side.tokens = int(tokens)
        side.act_bstride, side.act_tstride = 0, a.stride(0)
        side.grad_bstride, side.grad_tstride = 0, g.stride(0)
        side.seg_offsets = seg.data_ptr()
        side.row_index = index.data_ptr() if index is not None else None
    side.has_bias = int(bool(bias))
    side.reserved = 0
    return side


def ghost_gram(
    a1: torch.Tensor,
    g1: torch.Tensor,
    a2: torch.Tensor,
    g2: torch.Tensor,
    *,
    bias: bool = False,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """Fused factorized cross-gram of one linear layer, fp32 ``(B1, B2)``.

    ``a*`` are (B, S, K), ``g*`` (B, S, D) in one of fp32/fp16/bf16; the two
    sides may differ in S.  ``bias`` adds the implicit ones column on both
    activations.  With ``out`` given (fp32, (B1, B2) with unit column stride)
    the result is written -- or added, with ``accumulate`` -- in place.
    """
    dev = nat.require_device(a1, g1, a2, g2)
    if a1.dim() != 3 or g1.dim() != 3 or a2.dim() != 3 or g2.dim() != 3:
        raise ValueError("ghost_gram expects 3-D (B, S, width) factors")
    if not (a1.dtype == g1.dtype == a2.dtype == g2.dtype):
        raise ValueError("ghost_gram factors must share one dtype")
    if a1.shape[:2] != g1.shape[:2] or a2.shape[:2] != g2.shape[:2]:
        raise ValueError("activation and gradient factors disagree on (B, S)")
    if a1.shape[-1] != a2.shape[-1] or g1.shape[-1] != g2.shape[-1]:
        raise ValueError("the two sides disagree on the layer widths")
    code = nat.dtype_code(a1.dtype)
    vec = _chunk_elems(a1.dtype)
    k = -(-a1.shape[-1] // vec) * vec
    d = -(-g1.shape[-1] // vec) * vec
    a1, a2 = prepare_rows(a1, k), prepare_rows(a2, k)
    g1, g2 = prepare_rows(g1, d), prepare_rows(g2, d)
    b1, b2 = a1.shape[0], a2.shape[0]
    if out is None:
        out = torch.empty(b1, b2, dtype=torch.float32, device=dev)
        accumulate = False
    elif out.dtype != torch.float32 or tuple(out.shape) != (b1, b2) or out.stride(1) != 1:
        raise ValueError("out must be a float32 (B1, B2) tensor with unit column stride")
    s1 = _side(a1, g1, bias)
    s2 = _side(a2, g2, bias)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_ghost_gram_workspace(s1, s2, k, d, code, ctypes.byref(nbytes)), "ghost_gram")
    ws = nat.workspace(nbytes.value, dev)
    nat.check(
        lib.da_ghost_gram(
            s1, s2, k, d, code, out.data_ptr(), out.stride(0), int(accumulate),
            ws.data_ptr(), ws.numel(), nat.stream_ptr(dev),
        ),
        "ghost_gram",
    )
    return out


def selftest_mfma(dtype: torch.dtype, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Raw accumulator dump of one 32x32 MFMA (see da_selftest_mfma)."""
    dev = nat.require_device(a, b)
    out = torch.empty(64 * 16, dtype=torch.float32, device=dev)
    nat.check(
        nat.load().da_selftest_mfma(nat.dtype_code(dtype), a.data_ptr(), b.data_ptr(),
                                    out.data_ptr(), nat.stream_ptr(dev)),
        "selftest_mfma",
    )
    return out.view(64, 16)
