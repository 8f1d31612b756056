"""Typed torch-tensor wrappers over the C-ABI entry points.

Each wrapper checks shapes, brings operands into the layout the kernel
requires (16-byte aligned rows, widths a multiple of one 16-byte chunk --
padding with zero features when needed, which changes no product), allocates
outputs and workspace from torch's caching allocator and launches on the
current stream of the tensors' device.  No arithmetic happens here.
"""

from __future__ import annotations

import contextlib
import ctypes
import math

import numpy as np
import torch

from dattri_llm_amd import _native as nat


_launch_log: dict | None = None


@contextlib.contextmanager
def launch_events():
    """While active, every kernel launch made through this module is bracketed
    by HIP events on the stream it is launched on; yields ``{entry point:
    [(start, end), ...]}``.  Used to time kernels inside a measured region
    without changing what runs."""
    global _launch_log  # noqa: PLW0603
    prev, _launch_log = _launch_log, {}
    try:
        yield _launch_log
    finally:
        _launch_log = prev


def _run(dev: torch.device, what: str, fn, *args) -> None:
    """Call the C entry point ``fn(*args)`` (it enqueues work on ``dev``'s
    current stream) and map its status to an exception."""
    log = _launch_log
    if log is None:
        nat.check(fn(*args), what)
        return
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    nat.check(fn(*args), what)
    end.record(stream)
    log.setdefault(what, []).append((start, end))


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
    _run(dev, "ghost_gram", lib.da_ghost_gram,
         s1, s2, k, d, code, out.data_ptr(), out.stride(0), int(accumulate), ws.data_ptr(), ws.numel(),
         nat.stream_ptr(dev))
    return out


def ghost_gram_diag(
    a1: torch.Tensor,
    g1: torch.Tensor,
    a2: torch.Tensor,
    g2: torch.Tensor,
    *,
    bias: bool = False,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """The ghost product on the diagonal pairs only, fp32 ``(B,)``: sample i of
    side 1 against sample i of side 2 (per-sample dots; per-sample squared
    norms when both sides are one block), all samples in one launch."""
    dev = nat.require_device(a1, g1, a2, g2)
    if a1.dim() != 3 or g1.dim() != 3 or a2.dim() != 3 or g2.dim() != 3:
        raise ValueError("ghost_gram_diag expects 3-D (B, S, width) factors")
    if not (a1.dtype == g1.dtype == a2.dtype == g2.dtype):
        raise ValueError("ghost_gram_diag factors must share one dtype")
    if a1.shape[:2] != g1.shape[:2] or a2.shape[:2] != g2.shape[:2]:
        raise ValueError("activation and gradient factors disagree on (B, S)")
    if a1.shape[0] != a2.shape[0]:
        raise ValueError("ghost_gram_diag needs two blocks of one batch size")
    if a1.shape[-1] != a2.shape[-1] or g1.shape[-1] != g2.shape[-1]:
        raise ValueError("the two sides disagree on the layer widths")
    code = nat.dtype_code(a1.dtype)
    vec = _chunk_elems(a1.dtype)
    k = -(-a1.shape[-1] // vec) * vec
    d = -(-g1.shape[-1] // vec) * vec
    same = a1 is a2 and g1 is g2
    a1, g1 = prepare_rows(a1, k), prepare_rows(g1, d)
    a2, g2 = (a1, g1) if same else (prepare_rows(a2, k), prepare_rows(g2, d))
    b = a1.shape[0]
    if out is None:
        out = torch.empty(b, dtype=torch.float32, device=dev)
        accumulate = False
    elif out.dtype != torch.float32 or tuple(out.shape) != (b,):
        raise ValueError("out must be a float32 (B,) tensor")
    s1, s2 = _side(a1, g1, bias), _side(a2, g2, bias)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_ghost_gram_diag_workspace(s1, s2, k, d, code, ctypes.byref(nbytes)), "ghost_gram_diag")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "ghost_gram_diag", lib.da_ghost_gram_diag,
         s1, s2, k, d, code, out.data_ptr(), out.stride(0), int(accumulate), ws.data_ptr(), ws.numel(),
         nat.stream_ptr(dev))
    return out


def _token_ids(tok: torch.Tensor) -> torch.Tensor:
    """int64 (B, T) token ids, 8-byte aligned (a copy only when they are not)."""
    if tok.dtype != torch.int64 or tok.data_ptr() % 8:
        tok = tok.to(torch.int64).contiguous() if tok.dtype != torch.int64 else tok.clone()
    return tok


def embedding_cross_gram(
    tok1: torch.Tensor,
    g1: torch.Tensor,
    tok2: torch.Tensor,
    g2: torch.Tensor,
    *,
    diag: bool = False,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """Cross-gram of one embedding layer, fp32 ``(B1, B2)``:
    ``sum over (t, s) with tok1[i,t] == tok2[j,s] of g1[i,t] . g2[j,s]`` --
    side 2 compacted to its distinct ids, each side-1 token looked up.

    ``tok*`` are integer (B, T) ids (negative ids match nothing), ``g*`` the
    (B, T, E) gradient rows in one of fp32/fp16/bf16.  With ``diag`` only the
    pairs (i, i) are formed and the result is ``(B,)``."""
    dev = nat.require_device(tok1, g1, tok2, g2)
    if diag and tok1.shape[0] != tok2.shape[0]:
        raise ValueError("embedding_cross_gram(diag=True) needs two blocks of one batch size")
    tok1, g1, tok2, g2, e = _embedding_sides("embedding_cross_gram", tok1, g1, tok2, g2)
    code = nat.dtype_code(g1.dtype)
    b1, b2 = tok1.shape[0], tok2.shape[0]
    shape = (b1,) if diag else (b1, b2)
    if out is None:
        out = torch.empty(*shape, dtype=torch.float32, device=dev)
        accumulate = False
    elif out.dtype != torch.float32 or tuple(out.shape) != shape or out.stride(-1) != 1:
        raise ValueError(f"out must be a float32 {shape} tensor with unit column stride")
    s1, s2 = _side(tok1, g1, False), _side(tok2, g2, False)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_embedding_cross_gram_workspace(s1, s2, e, code, int(diag), ctypes.byref(nbytes)),
              "embedding_cross_gram")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "embedding_cross_gram", lib.da_embedding_cross_gram,
         s1, s2, e, code, int(diag), out.data_ptr(), out.stride(0), int(accumulate), ws.data_ptr(), ws.numel(),
         nat.stream_ptr(dev))
    return out


def materialize_embedding(tok: torch.Tensor, g: torch.Tensor, vocab: int) -> torch.Tensor:
    """Per-sample embedding weight gradient ``(B, vocab*E)`` in g's dtype:
    row v of sample b is the sum of the gradient rows whose id is v, in fp32
    in ascending token order, rounded once.  Ids must lie in ``[0, vocab)``
    (the caller checks); a negative id adds nothing."""
    dev = nat.require_device(tok, g)
    if tok.dim() != 2 or g.dim() != 3 or tok.shape != g.shape[:2]:
        raise ValueError("materialize_embedding expects (B, T) ids and (B, T, E) gradients")
    b, t = tok.shape
    e = g.shape[-1]
    out = torch.empty(b, vocab * e, dtype=g.dtype, device=dev)
    if b == 0 or e == 0 or vocab == 0:
        return out
    ep = -(-e // _chunk_elems(g.dtype)) * _chunk_elems(g.dtype)
    if ep != e:  # padded width: scatter into a padded table, then drop the padding
        full = materialize_embedding(tok, prepare_rows(g, ep), vocab)
        out.view(b, vocab, e).copy_(full.view(b, vocab, ep)[:, :, :e])
        return out
    tok, g = _token_ids(tok), prepare_rows(g, e)
    code = nat.dtype_code(g.dtype)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_materialize_embedding_workspace(b, t, e, code, ctypes.byref(nbytes)), "materialize_embedding")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "materialize_embedding", lib.da_materialize_embedding,
         tok.data_ptr(), g.data_ptr(), code, b, t, e, vocab, tok.stride(0), tok.stride(1),
         g.stride(0), g.stride(1), out.data_ptr(), vocab * e, ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


def _per_token_out(out, b1, t1, b2, dev, accumulate):
    if out is None:
        return torch.empty(b1, t1, b2, dtype=torch.float32, device=dev), False
    if out.dtype != torch.float32 or tuple(out.shape) != (b1, t1, b2):
        raise ValueError("out must be a float32 (B1, T1, B2) tensor")
    return out, accumulate


def ghost_gram_per_token(
    a1: torch.Tensor,
    g1: torch.Tensor,
    a2: torch.Tensor,
    g2: torch.Tensor,
    *,
    bias: bool = False,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """Per-token cross-gram of one linear layer, fp32 ``(B1, T1, B2)``:
    ``K[i, t, j] = sum_s (a1_it . a2_js + bias)(g1_it . g2_js)``, i.e. side 1's
    token t against side 2's whole per-sample gradient (``da_ghost_gram_per_token``).
    Factors as for :func:`ghost_gram`."""
    dev = nat.require_device(a1, g1, a2, g2)
    if a1.dim() != 3 or g1.dim() != 3 or a2.dim() != 3 or g2.dim() != 3:
        raise ValueError("ghost_gram_per_token expects 3-D (B, S, width) factors")
    if not (a1.dtype == g1.dtype == a2.dtype == g2.dtype):
        raise ValueError("ghost_gram_per_token factors must share one dtype")
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
    b1, t1, b2 = a1.shape[0], a1.shape[1], a2.shape[0]
    out, accumulate = _per_token_out(out, b1, t1, b2, dev, accumulate)
    o0 = out.stride(0)
    if _flatten_side1(a1, g1, out):
        # Side 1's token rows are independent outputs: as one sample of
        # B1*T1 tokens they fill the kernel's 256-row tiles instead of padding
        # each short sample to a tile (out row i*T1 + t is token t of sample i).
        a1, g1 = a1.reshape(1, b1 * t1, k), g1.reshape(1, b1 * t1, d)
        o0 = b1 * t1 * out.stride(1)
    s1, s2 = _side(a1, g1, bias), _side(a2, g2, bias)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_ghost_gram_per_token_workspace(s1, s2, k, d, code, ctypes.byref(nbytes)),
              "ghost_gram_per_token")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "ghost_gram_per_token", lib.da_ghost_gram_per_token,
         s1, s2, k, d, code, out.data_ptr(), o0, out.stride(1), out.stride(2), int(accumulate),
         ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


def _flatten_side1(a1: torch.Tensor, g1: torch.Tensor, out: torch.Tensor) -> bool:
    """Whether the per-token kernel should see side 1 as one sample of B1*T1
    tokens: several samples shorter than the 256-row tile, whose rows (and out
    rows) lie at one stride, within the kernel's 32-bit row offsets."""
    b1, t1 = a1.shape[:2]
    if b1 < 2 or t1 >= 256:
        return False
    if a1.stride(0) != t1 * a1.stride(1) or g1.stride(0) != t1 * g1.stride(1):
        return False
    if out.stride(0) != t1 * out.stride(1):
        return False
    row_bytes = max(a1.stride(1), g1.stride(1)) * a1.element_size()
    return b1 * t1 * row_bytes + max(a1.shape[-1], g1.shape[-1]) * a1.element_size() < (1 << 31) - (1 << 20)


def _embedding_sides(name, tok1, g1, tok2, g2):
    if tok1.dim() != 2 or tok2.dim() != 2 or g1.dim() != 3 or g2.dim() != 3:
        raise ValueError(f"{name} expects (B, T) ids and (B, T, E) gradients")
    if tok1.shape != g1.shape[:2] or tok2.shape != g2.shape[:2]:
        raise ValueError("ids and gradients disagree on (B, T)")
    if g1.dtype != g2.dtype:
        raise ValueError(f"{name} gradients must share one dtype")
    if g1.shape[-1] != g2.shape[-1]:
        raise ValueError("the two sides disagree on the embedding width")
    e = -(-g1.shape[-1] // _chunk_elems(g1.dtype)) * _chunk_elems(g1.dtype)
    same = tok1 is tok2 and g1 is g2
    tok1, g1 = _token_ids(tok1), prepare_rows(g1, e)
    tok2, g2 = (tok1, g1) if same else (_token_ids(tok2), prepare_rows(g2, e))
    return tok1, g1, tok2, g2, e


def embedding_cross_gram_per_token(
    tok1: torch.Tensor,
    g1: torch.Tensor,
    tok2: torch.Tensor,
    g2: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """Per-token embedding cross-gram, fp32 ``(B1, T1, B2)``: side 1's token t
    against side 2's whole per-sample gradient, ``sum over s with
    tok2[j,s] == tok1[i,t] of g1[i,t] . g2[j,s]``."""
    dev = nat.require_device(tok1, g1, tok2, g2)
    tok1, g1, tok2, g2, e = _embedding_sides("embedding_cross_gram_per_token", tok1, g1, tok2, g2)
    code = nat.dtype_code(g1.dtype)
    b1, t1, b2 = tok1.shape[0], tok1.shape[1], tok2.shape[0]
    out, accumulate = _per_token_out(out, b1, t1, b2, dev, accumulate)
    s1, s2 = _side(tok1, g1, False), _side(tok2, g2, False)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_embedding_cross_gram_per_token_workspace(s1, s2, e, code, ctypes.byref(nbytes)),
              "embedding_cross_gram_per_token")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "embedding_cross_gram_per_token", lib.da_embedding_cross_gram_per_token,
         s1, s2, e, code, out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), int(accumulate),
         ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


def dense_per_token_embedding(
    tok1: torch.Tensor,
    g1: torch.Tensor,
    m2: torch.Tensor,
    vocab: int,
    *,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """Per-token product of an embedding side against dense per-sample
    gradients ``m2 (B2, vocab*E)``, fp32 ``(B1, T1, B2)``:
    ``sum_e g1[i,t,e] * m2[j, tok1[i,t]*E + e]`` (0 for a negative id; ids
    must be below ``vocab``)."""
    dev = nat.require_device(tok1, g1, m2)
    if tok1.dim() != 2 or g1.dim() != 3 or tok1.shape != g1.shape[:2]:
        raise ValueError("dense_per_token_embedding expects (B, T) ids and (B, T, E) gradients")
    if m2.dtype != g1.dtype:
        raise ValueError("dense_per_token_embedding operands must share one dtype")
    b1, t1, e = g1.shape
    b2 = m2.shape[0]
    if m2.reshape(b2, -1).shape[1] != vocab * e:
        raise ValueError(f"m2 rows hold {m2.reshape(b2, -1).shape[1]} values, expected vocab*E = {vocab * e}")
    vec = _chunk_elems(g1.dtype)
    ep = -(-e // vec) * vec
    m2 = m2.reshape(b2, vocab, e)
    if ep != e:
        m2 = prepare_rows(m2, ep)
    m2 = m2.reshape(b2, vocab * ep)
    if m2.stride(1) != 1 or m2.data_ptr() % 16 or (m2.stride(0) * m2.element_size()) % 16:
        m2 = m2.contiguous()
    tok1, g1 = _token_ids(tok1), prepare_rows(g1, ep)
    out, accumulate = _per_token_out(out, b1, t1, b2, dev, accumulate)
    _run(dev, "dense_per_token_embedding", nat.load().da_dense_per_token_embedding,
         tok1.data_ptr(), g1.data_ptr(), nat.dtype_code(g1.dtype), b1, t1, ep, vocab, tok1.stride(0),
         tok1.stride(1), g1.stride(0), g1.stride(1), m2.data_ptr(), m2.stride(0), b2, out.data_ptr(),
         out.stride(0), out.stride(1), out.stride(2), int(accumulate), nat.stream_ptr(dev))
    return out


def gather_embedding_entries(tok: torch.Tensor, g: torch.Tensor, rows: torch.Tensor,
                             cols: torch.Tensor) -> torch.Tensor:
    """fp32 ``(B, k)``: entry q of sample b is the sum of ``g[b, t, cols[q]]``
    over the tokens whose id is ``rows[q]`` (ascending t) -- the kept
    coordinates of the per-sample embedding gradient."""
    dev = nat.require_device(tok, g, rows, cols)
    if tok.dim() != 2 or g.dim() != 3 or tok.shape != g.shape[:2]:
        raise ValueError("gather_embedding_entries expects (B, T) ids and (B, T, E) gradients")
    if rows.shape != cols.shape or rows.dim() != 1:
        raise ValueError("rows and cols must be matching 1-D index tensors")
    b, t, e = g.shape
    k = rows.numel()
    out = torch.empty(b, k, dtype=torch.float32, device=dev)
    if b == 0 or k == 0:
        return out
    tok = _token_ids(tok)
    if g.stride(-1) != 1:
        g = g.contiguous()
    rows, cols = rows.to(torch.int64).contiguous(), cols.to(torch.int64).contiguous()
    _run(dev, "gather_embedding_entries", nat.load().da_gather_embedding_entries,
         tok.data_ptr(), g.data_ptr(), nat.dtype_code(g.dtype), b, t, e, tok.stride(0), tok.stride(1),
         g.stride(0), g.stride(1), rows.data_ptr(), cols.data_ptr(), k, out.data_ptr(), out.stride(0),
         nat.stream_ptr(dev))
    return out


def dense_per_token(
    a1: torch.Tensor,
    g1: torch.Tensor,
    m2: torch.Tensor,
    *,
    bias: bool = False,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """Per-token cross-gram against dense per-sample gradients, fp32
    ``(B1, T1, B2)``: ``K[i, t, j] = g1_it^T M2_j a1_it`` (``da_dense_per_token``).

    ``m2`` is (B2, D, K) -- or (B2, D, K+1) with ``bias``, the last column the
    bias gradient -- in materialize's ``o*(K+bias) + i`` order; a flat
    (B2, D*(K+bias)) block is reshaped."""
    dev = nat.require_device(a1, g1, m2)
    if a1.dim() != 3 or g1.dim() != 3 or a1.shape[:2] != g1.shape[:2]:
        raise ValueError("dense_per_token expects (B, T, K) and (B, T, D) factors")
    if a1.dtype != g1.dtype or m2.dtype != a1.dtype:
        raise ValueError("dense_per_token operands must share one dtype")
    kk, dd = a1.shape[-1], g1.shape[-1]
    kb = kk + int(bias)
    if m2.numel() != m2.shape[0] * dd * kb:
        raise ValueError(f"m2 must hold (B2, {dd}, {kb}) values")
    m2 = m2.reshape(m2.shape[0], dd, kb)
    bias_grad = m2[:, :, kk].float().contiguous() if bias else None
    code = nat.dtype_code(a1.dtype)
    vec = _chunk_elems(a1.dtype)
    k = -(-kk // vec) * vec
    d = -(-dd // vec) * vec
    a1, g1 = prepare_rows(a1, k), prepare_rows(g1, d)
    w = m2[:, :, :kk]
    if k != kk or d != dd or not _aligned(w) or w.stride(2) != 1:
        padded = torch.zeros(w.shape[0], d, k, dtype=w.dtype, device=dev)
        padded[:, :dd, :kk] = w
        w = padded
    if bias_grad is not None and d != dd:
        bias_grad = torch.nn.functional.pad(bias_grad, (0, d - dd))
    b1, t1, b2 = a1.shape[0], a1.shape[1], w.shape[0]
    out, accumulate = _per_token_out(out, b1, t1, b2, dev, accumulate)
    o0 = out.stride(0)
    if _flatten_side1(a1, g1, out):  # short samples as one long one (see ghost_gram_per_token)
        a1, g1 = a1.reshape(1, b1 * t1, k), g1.reshape(1, b1 * t1, d)
        o0 = b1 * t1 * out.stride(1)
    s1 = _side(a1, g1, bias)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_dense_per_token_workspace(s1, b2, k, d, code, ctypes.byref(nbytes)), "dense_per_token")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "dense_per_token", lib.da_dense_per_token,
         s1, w.data_ptr(), b2, w.stride(0), w.stride(1),
         bias_grad.data_ptr() if bias_grad is not None else None,
         bias_grad.stride(0) if bias_grad is not None else 0, k, d, code, out.data_ptr(), o0,
         out.stride(1), out.stride(2), int(accumulate), ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


# FactorSide as a numpy record, so a grouped launch's side arrays are filled
# column by column instead of one ctypes structure per group (a launch may
# carry hundreds of groups: the experts of an MoE layer, a depthwise conv).
# numpy record with FactorSide's layout (field names, offsets and size taken from the ctypes struct)
_CTYPE_FORMAT = {ctypes.c_void_p: "<u8", ctypes.c_int64: "<i8", ctypes.c_int32: "<i4"}
_SIDE_RECORD = np.dtype({"names": [f for f, _t in nat.FactorSide._fields_],
                         "formats": [_CTYPE_FORMAT[t] for _f, t in nat.FactorSide._fields_],
                         "offsets": [getattr(nat.FactorSide, f).offset for f, _t in nat.FactorSide._fields_],
                         "itemsize": ctypes.sizeof(nat.FactorSide)})


def _grouped_sides(groups, nb, ks, ds, biases, dev_index, dtype, vec, es, keep):
    """One side's FactorSide array for :func:`ghost_gram_grouped`, checked."""
    n = len(groups)
    cols = {f: [0] * n for f in ("act", "grad", "tokens", "act_tstride", "grad_tstride", "seg_offsets",
                                  "row_index")}
    for e, (a, g, seg, idx) in enumerate(groups):
        if a.dim() != 2 or g.dim() != 2:
            raise ValueError("grouped factors must be (rows, width) with matching rows")
        (ra, wa), (rg, wg) = a.shape, g.shape
        if ra != rg:
            raise ValueError("grouped factors must be (rows, width) with matching rows")
        if a.dtype != dtype or g.dtype != dtype:
            raise ValueError("grouped factors must share one dtype")
        if seg.dtype != torch.int32 or seg.numel() != nb + 1 or (idx is not None and idx.dtype != torch.int32):
            raise ValueError("segment offsets (B+1) and row indices must be int32, one batch per side")
        for t in (a, g, seg, idx):
            if t is not None and t.get_device() != dev_index:
                nat.require_device(*[x for grp in groups for x in grp])  # raises with the reason
                raise ValueError("grouped operands on different devices")
        pa, pg = a.data_ptr(), g.data_ptr()
        sa, sg = a.stride(), g.stride()
        if not (wa == ks[e] and sa[1] == 1 and pa % 16 == 0 and (sa[0] * es) % 16 == 0):
            a = prepare_rows(a, ks[e])
            keep.append(a)
            pa, sa = a.data_ptr(), a.stride()
        if not (wg == ds[e] and sg[1] == 1 and pg % 16 == 0 and (sg[0] * es) % 16 == 0):
            g = prepare_rows(g, ds[e])
            keep.append(g)
            pg, sg = g.data_ptr(), g.stride()
        if not seg.is_contiguous():
            seg = seg.contiguous()
            keep.append(seg)
        if idx is not None and not idx.is_contiguous():
            idx = idx.contiguous()
            keep.append(idx)
        cols["act"][e], cols["grad"][e] = pa, pg
        cols["tokens"][e] = ra
        cols["act_tstride"][e], cols["grad_tstride"][e] = sa[0], sg[0]
        cols["seg_offsets"][e] = seg.data_ptr()
        cols["row_index"][e] = idx.data_ptr() if idx is not None else 0
    rec = np.zeros(n, dtype=_SIDE_RECORD)
    for f, v in cols.items():
        rec[f] = v
    rec["batch"] = nb
    rec["has_bias"] = biases
    keep.append(rec)
    return (nat.FactorSide * n).from_buffer(rec)


def ghost_gram_grouped(groups1, groups2, *, bias=False, out: torch.Tensor | None = None,
                       accumulate: bool = False) -> torch.Tensor:
    """Segment-summed ghost product over groups (experts of one or several
    linear layers), fp32 ``(B1, B2)``.

    ``groups*`` are equally long lists of ``(a, g, seg, idx)``: a group's
    (rows, K) activation and (rows, D) gradient captures, its int32 per-sample
    offsets ``seg`` (B+1 entries, non-decreasing, ``seg[B] <= rows``) and an
    optional int32 row index (packed row r is physical row ``idx[r]``).  Group
    e's two sides share K and D; groups may differ in widths (the experts of
    several layers in one launch, widest first) and ``bias`` may be one bool or
    one per group.  All groups share B1 / B2 and the dtype."""
    n = len(groups1)
    if len(groups2) != n or n == 0:
        raise ValueError("ghost_gram_grouped needs the same, non-zero number of groups on both sides")
    biases = [int(bool(x)) for x in bias] if isinstance(bias, (list, tuple)) else [int(bool(bias))] * n
    if len(biases) != n:
        raise ValueError("one bias flag per group")
    dev = nat.require_device(groups1[0][0])
    dev_index = groups1[0][0].get_device()
    dtype = groups1[0][0].dtype
    b1, b2 = groups1[0][2].numel() - 1, groups2[0][2].numel() - 1
    code = nat.dtype_code(dtype)  # raises for a dtype the kernels do not read
    es = nat.ELEM_BYTES[dtype]
    vec = 16 // es
    ks, ds = [0] * n, [0] * n
    for e in range(n):
        kw, dw = groups1[e][0].shape[-1], groups1[e][1].shape[-1]
        if groups2[e][0].shape[-1] != kw or groups2[e][1].shape[-1] != dw:
            raise ValueError(f"group {e}: the two sides disagree on the layer widths")
        ks[e] = -(-kw // vec) * vec
        ds[e] = -(-dw // vec) * vec
    keep: list = []
    sides = [_grouped_sides(groups, nb, ks, ds, biases, dev_index, dtype, vec, es, keep)
             for groups, nb in ((groups1, b1), (groups2, b2))]
    if out is None:
        out = torch.empty(b1, b2, dtype=torch.float32, device=dev)
        accumulate = False
    elif out.dtype != torch.float32 or tuple(out.shape) != (b1, b2) or out.stride(1) != 1:
        raise ValueError("out must be a float32 (B1, B2) tensor with unit column stride")
    karr, darr = (ctypes.c_int64 * n)(*ks), (ctypes.c_int64 * n)(*ds)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_ghost_gram_grouped_workspace(sides[0], sides[1], n, karr, darr, code, ctypes.byref(nbytes)),
              "ghost_gram_grouped")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "ghost_gram_grouped", lib.da_ghost_gram_grouped,
         sides[0], sides[1], n, karr, darr, code, out.data_ptr(), out.stride(0), int(accumulate),
         ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    del keep
    return out


def is_blocked(x: torch.Tensor) -> bool:
    """A (B, W/64, 64) view of a dense (B, W) block stored in 64-element blocks."""
    return x.dim() == 3 and x.shape[2] == 64 and x.stride(2) == 1


def blocked_storage(b: int, width: int, dtype: torch.dtype, device) -> torch.Tensor:
    """An uninitialised k-blocked (B, width) block: the (B, width/64, 64) view
    of a (width/64, B, 64) buffer, so block j of every sample is one run."""
    return torch.empty(width // 64, b, 64, dtype=dtype, device=device).permute(1, 0, 2)


def materialize_linear(
    a: torch.Tensor,
    g: torch.Tensor,
    *,
    bias: bool = False,
    out_dtype: torch.dtype | None = None,
    blocked: bool = False,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-sample linear weight gradient ``(B, D*(K+bias))``, index o*(K+bias)+k.

    With ``blocked`` (and K a multiple of 64, no bias) the result is written in
    the k-blocked layout and returned as its ``(B, D*K/64, 64)`` view (see
    :func:`is_blocked`); otherwise ``blocked`` is ignored.  ``out`` (blocked
    only) is a row slice ``view[b0:b0+B]`` of a larger :func:`blocked_storage`
    buffer, so several blocks can be written into one."""
    dev = nat.require_device(a, g)
    if a.dim() != 3 or g.dim() != 3 or a.shape[:2] != g.shape[:2]:
        raise ValueError("materialize_linear expects a (B, T, K) and g (B, T, D)")
    if a.dtype != g.dtype:
        raise ValueError("materialize_linear factors must share one dtype")
    out_dtype = out_dtype or a.dtype
    b, t, k = a.shape
    d = g.shape[-1]
    kb = k + int(bias)
    if blocked and not bias and k % 64 == 0 and d % _chunk_elems(a.dtype) == 0 and b > 0 and t > 0:
        if out is None:
            out = blocked_storage(b, d * k, out_dtype, dev)
        elif not (is_blocked(out) and out.shape == (b, d * k // 64, 64) and out.stride(0) == 64
                  and out.stride(1) >= b * 64 and out.dtype == out_dtype and out.device == dev):
            raise ValueError("materialize_linear out must be a (B, D*K/64, 64) row slice of a blocked buffer "
                             "in out_dtype")
        a, g = prepare_rows(a, k), prepare_rows(g, d)
        _run(dev, "materialize_linear", nat.load().da_materialize_linear,
             a.data_ptr(), g.data_ptr(), nat.dtype_code(a.dtype), b, t, k, d, a.stride(0), a.stride(1),
             g.stride(0), g.stride(1), 0, out.data_ptr(), nat.dtype_code(out_dtype), 64, k, out.stride(1),
             nat.stream_ptr(dev))
        return out
    if out is not None:
        raise ValueError("materialize_linear out is for the blocked layout only")
    out = torch.empty(b, d * kb, dtype=out_dtype, device=dev)
    if b == 0 or d == 0 or kb == 0:
        return out
    if t == 0:
        return out.zero_()
    vec = _chunk_elems(a.dtype)
    kp = -(-k // vec) * vec
    dp = -(-d // vec) * vec
    if kp != k or dp != d:
        # padded widths: compute into a padded buffer, then drop the padding
        full = materialize_linear(prepare_rows(a, kp), prepare_rows(g, dp), out_dtype=out_dtype)
        full = full.view(b, dp, kp)[:, :d, :k]
        out.view(b, d, kb)[:, :, :k] = full
        if bias:
            out.view(b, d, kb)[:, :, k] = _column_sums(g, out_dtype)
        return out
    a, g = prepare_rows(a, k), prepare_rows(g, d)
    _run(dev, "materialize_linear", nat.load().da_materialize_linear,
         a.data_ptr(), g.data_ptr(), nat.dtype_code(a.dtype), b, t, k, d, a.stride(0), a.stride(1),
         g.stride(0), g.stride(1), int(bias), out.data_ptr(), nat.dtype_code(out_dtype), d * kb, kb, 64,
         nat.stream_ptr(dev))
    return out


def row_gram(x: torch.Tensor, *, out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """fp32 ``x^T x`` of bf16/fp16 rows ``x (N, p)`` -> ``(p, p)``; with
    ``accumulate`` it is added to ``out``, which must be symmetric (its lower
    tiles are rewritten as the mirror of the upper ones).  The product is
    computed once per tile pair on or above the diagonal and mirrored; a small
    triangle of tiles runs as token splits summed by a second pass."""
    dev = nat.require_device(x, out)
    if x.dim() != 2 or x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("row_gram expects bf16/fp16 rows (N, p)")
    n, p = x.shape
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = torch.empty(p, p, dtype=torch.float32, device=dev)
    elif out.dtype != torch.float32 or out.shape != (p, p) or out.stride(1) != 1:
        raise ValueError("row_gram out must be (p, p) fp32 with unit column stride")
    if p == 0:
        return out
    vec = _chunk_elems(x.dtype)
    xp = prepare_rows(x, -(-p // vec) * vec)
    if xp.shape[-1] != p:  # padded columns: the product of the padded rows, then the (p, p) corner
        full = row_gram(xp)
        if accumulate:
            out += full[:p, :p]
        else:
            out.copy_(full[:p, :p])
        return out
    if xp.stride(1) != 1:
        xp = xp.contiguous()
    lib = nat.load()
    need = ctypes.c_size_t(0)
    nat.check(lib.da_row_gram_workspace(n, p, nat.dtype_code(xp.dtype), ctypes.byref(need)), "row_gram")
    ws = torch.empty(need.value, dtype=torch.uint8, device=dev) if need.value else None
    _run(dev, "row_gram", lib.da_row_gram,
         xp.data_ptr(), nat.dtype_code(xp.dtype), n, p, xp.stride(0), out.data_ptr(), out.stride(0),
         int(accumulate), ws.data_ptr() if ws is not None else None, need.value, nat.stream_ptr(dev))
    return out


def nonzero_rows(x: torch.Tensor) -> torch.Tensor:
    """``(x != 0).any(dim=1)`` of a 2-D tensor as a bool vector (one read of
    ``x``; -0.0 counts as zero, NaN as nonzero)."""
    dev = nat.require_device(x)
    if x.dim() != 2:
        raise ValueError("nonzero_rows expects a 2-D tensor")
    n = x.shape[0]
    out = torch.empty(n, dtype=torch.uint8, device=dev)
    if n == 0:
        return out.bool()
    xp = prepare_rows(x)  # zero padding changes no row's answer
    if xp.stride(1) != 1:
        xp = xp.contiguous()
    _run(dev, "nonzero_rows", nat.load().da_nonzero_rows,
         xp.data_ptr(), nat.dtype_code(xp.dtype), n, xp.shape[1], xp.stride(0), out.data_ptr(),
         nat.stream_ptr(dev))
    return out.view(torch.bool)


def _column_sums(g: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """sum_t g[b, t, :] through the materialize kernel with a ones activation."""
    b, t, _ = g.shape
    vec = _chunk_elems(g.dtype)
    ones = torch.zeros(b, t, vec, dtype=g.dtype, device=g.device)
    ones[..., 0] = 1
    dp = -(-g.shape[-1] // vec) * vec
    m = materialize_linear(ones, prepare_rows(g, dp), out_dtype=out_dtype)
    return m.view(b, dp, vec)[:, : g.shape[-1], 0]


def score_gemm(
    pairs: list[tuple[torch.Tensor, torch.Tensor]],
    *,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
) -> torch.Tensor:
    """``sum_L m1_L @ m2_L.T`` over dense layer pairs, fp32 ``(B1, B2)``.

    Each ``m*`` is (B, width...) and is flattened to (B, width); all pairs
    share one dtype.  The side with fewer rows is put on the kernel's 32-row
    side (the result is written transposed through the output strides).
    """
    if not pairs:
        raise ValueError("score_gemm needs at least one layer pair")

    def rows(m):  # k-blocked views pass as they are; anything else as (B, W)
        return m if is_blocked(m) else m.reshape(m.shape[0], -1)

    def width(m):
        return m.shape[1] * 64 if is_blocked(m) else m.shape[1]

    flat = [(rows(m1), rows(m2)) for m1, m2 in pairs]
    dev = nat.require_device(*[t for p in flat for t in p])
    dtype = flat[0][0].dtype
    b1, b2 = flat[0][0].shape[0], flat[0][1].shape[0]
    for m1, m2 in flat:
        if m1.dtype != dtype or m2.dtype != dtype:
            raise ValueError("score_gemm layers must share one dtype")
        if m1.shape[0] != b1 or m2.shape[0] != b2 or width(m1) != width(m2):
            raise ValueError("score_gemm layer shapes disagree")
    if out is None:
        out = torch.empty(b1, b2, dtype=torch.float32, device=dev)
        accumulate = False
    elif out.dtype != torch.float32 or tuple(out.shape) != (b1, b2):
        raise ValueError("out must be float32 (B1, B2)")
    vec = _chunk_elems(dtype)
    swap = b1 > b2
    layers = []
    keep = []
    def operand(m, w):
        """(tensor, row stride, block stride) in elements for the kernel."""
        if is_blocked(m) and m.data_ptr() % 16 == 0 and all(
                (st * m.element_size()) % 16 == 0 for st in m.stride()[:2]):
            return m, m.stride(0), m.stride(1)
        if is_blocked(m):
            m = m.reshape(m.shape[0], -1)
        m = prepare_rows(m, w)
        return m, m.stride(0), 64

    for m1, m2 in flat:
        if width(m1) == 0:  # contributes nothing (and an empty tensor's strides are arbitrary)
            continue
        w = -(-width(m1) // vec) * vec
        (m1, ld1, bk1), (m2, ld2, bk2) = operand(m1, w), operand(m2, w)
        keep += [m1, m2]
        if swap:
            m1, ld1, bk1, m2, ld2, bk2 = m2, ld2, bk2, m1, ld1, bk1
        layers.append(nat.DenseLayer(m1.data_ptr(), m2.data_ptr(), w, ld1, ld2, bk1, bk2))
    n1, n2 = (b2, b1) if swap else (b1, b2)
    ld_row, ld_col = (out.stride(1), out.stride(0)) if swap else (out.stride(0), out.stride(1))
    lib = nat.load()
    code = nat.dtype_code(dtype)
    if not layers:  # every layer empty: the library writes the zero product (or leaves out to accumulate)
        _run(dev, "score_gemm", lib.da_score_gemm,
             n1, n2, None, 0, code, out.data_ptr(), ld_row, ld_col, int(accumulate), None, 0,
             nat.stream_ptr(dev))
        return out
    for start in range(0, len(layers), 32):
        group = layers[start : start + 32]
        arr = (nat.DenseLayer * len(group))(*group)
        nbytes = ctypes.c_size_t(0)
        nat.check(lib.da_score_gemm_workspace(n1, n2, arr, len(group), code, ctypes.byref(nbytes)), "score_gemm")
        ws = nat.workspace(nbytes.value, dev)
        _run(dev, "score_gemm", lib.da_score_gemm,
             n1, n2, arr, len(group), code, out.data_ptr(), ld_row, ld_col, int(accumulate or start > 0),
             ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    del keep
    return out


def _dense_operand(m: torch.Tensor, width: int):
    """(tensor, row stride, block stride) in elements of a dense (B, W) block
    as the dense-layer kernels address it: k-blocked views as they are,
    anything else as 16-byte aligned (B, width) rows."""
    if is_blocked(m) and m.data_ptr() % 16 == 0 and all((st * m.element_size()) % 16 == 0 for st in m.stride()[:2]):
        return m, m.stride(0), m.stride(1)
    if is_blocked(m):
        m = m.reshape(m.shape[0], -1)
    m = prepare_rows(m, width)
    return m, m.stride(0), 64


def row_dots(layers: list, *, out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """``sum_L (m1_L * m2_L).sum(-1)`` over dense layer pairs ``(m1, m2)``,
    fp32 ``(B,)``; a pair whose ``m2`` is None contributes ``m1``'s squared
    row norms.  Each ``m`` is (B, width...) -- k-blocked views are read in
    place, never reshaped -- and all layers share one dtype."""
    if not layers:
        raise ValueError("row_dots needs at least one layer")

    def width(m):
        return m.shape[1] * 64 if is_blocked(m) else math.prod(m.shape[1:])

    tensors = [t for pair in layers for t in pair if t is not None]
    dev = nat.require_device(*tensors)
    dtype = tensors[0].dtype
    b = layers[0][0].shape[0]
    for m1, m2 in layers:
        if m1.dtype != dtype or (m2 is not None and m2.dtype != dtype):
            raise ValueError("row_dots layers must share one dtype")
        if m1.shape[0] != b or (m2 is not None and (m2.shape[0] != b or width(m2) != width(m1))):
            raise ValueError("row_dots layer shapes disagree")
    if out is None:
        out = torch.empty(b, dtype=torch.float32, device=dev)
        accumulate = False
    elif out.dtype != torch.float32 or tuple(out.shape) != (b,):
        raise ValueError("out must be a float32 (B,) tensor")
    vec = _chunk_elems(dtype)
    descs, keep = [], []
    for m1, m2 in layers:
        w = width(m1)
        if w == 0:
            continue
        wp = -(-w // vec) * vec
        t1, ld1, bk1 = _dense_operand(m1, wp)
        t2, ld2, bk2 = _dense_operand(m2, wp) if m2 is not None else (None, 0, 0)
        keep += [t1, t2]
        descs.append(nat.DenseLayer(t1.data_ptr(), t2.data_ptr() if t2 is not None else None, wp, ld1, ld2, bk1, bk2))
    lib = nat.load()
    code = nat.dtype_code(dtype)
    if not descs:
        if not accumulate:
            out.zero_()
        return out
    for start in range(0, len(descs), 32):
        group = descs[start : start + 32]
        arr = (nat.DenseLayer * len(group))(*group)
        nbytes = ctypes.c_size_t(0)
        nat.check(lib.da_row_dots_workspace(b, arr, len(group), code, ctypes.byref(nbytes)), "row_dots")
        ws = nat.workspace(nbytes.value, dev)
        _run(dev, "row_dots", lib.da_row_dots,
             b, arr, len(group), code, out.data_ptr(), out.stride(0), int(accumulate or start > 0), ws.data_ptr(),
             ws.numel(), nat.stream_ptr(dev))
    del keep
    return out


NORM_KIND = {"nn.RMSNorm": 0, "nn.LayerNorm": 1}
NORM_KIND_GIVEN = 2  # x is already normalised: x_hat = x


def norm_weight_grad(
    x: torch.Tensor,
    g: torch.Tensor,
    *,
    kind: int,
    eps: float,
    bias: bool = False,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Per-sample norm weight gradient (B, d) -- or (B, 2d) = [dgamma, dbeta]."""
    dev = nat.require_device(x, g)
    if x.dim() != 3 or x.shape != g.shape:
        raise ValueError("norm_weight_grad expects x and g of one (B, T, d) shape")
    if x.dtype != g.dtype:
        raise ValueError("norm_weight_grad factors must share one dtype")
    out_dtype = out_dtype or x.dtype
    b, t, d = x.shape
    width = d * (1 + int(bias))
    out = torch.empty(b, width, dtype=out_dtype, device=dev)
    if b == 0:
        return out
    if t == 0:
        return out.zero_()
    if d % _chunk_elems(x.dtype) or not (_aligned(x) and _aligned(g)):
        # rows of whole 16-byte chunks; the kernels mask the padding
        x, g = prepare_rows(x), prepare_rows(g)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_norm_weight_grad_workspace(b, t, d, int(bias), ctypes.byref(nbytes)), "norm_weight_grad")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "norm_weight_grad", lib.da_norm_weight_grad,
         x.data_ptr(), g.data_ptr(), nat.dtype_code(x.dtype), b, t, d, x.stride(0), x.stride(1), g.stride(0),
         g.stride(1), int(kind), float(eps), int(bias), out.data_ptr(), nat.dtype_code(out_dtype), width,
         ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


def norm_xhat(x: torch.Tensor, *, kind: int, eps: float, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Normalised rows of a token norm layer over the last axis."""
    dev = nat.require_device(x)
    out_dtype = out_dtype or x.dtype
    d = x.shape[-1]
    rows = x.numel() // d if d else 0
    out = torch.empty(*x.shape, dtype=out_dtype, device=dev)
    if rows == 0:
        return out
    flat = x.reshape(rows, d)
    if d % _chunk_elems(x.dtype) or not _aligned(flat):
        flat = prepare_rows(flat)  # rows of whole 16-byte chunks; the kernel masks the padding
    _run(dev, "norm_xhat", nat.load().da_norm_xhat,
         flat.data_ptr(), nat.dtype_code(x.dtype), rows, d, flat.stride(0), int(kind), float(eps),
         out.data_ptr(), nat.dtype_code(out_dtype), d, nat.stream_ptr(dev))
    return out


def _channel_rows(x: torch.Tensor):
    n, c = x.shape[:2]
    s = x.numel() // max(n * c, 1) if n * c else 0
    return x.contiguous(), n, c, s


def channel_norm_weight_grad(x: torch.Tensor, g: torch.Tensor, *, groups: int, eps: float, bias: bool = False,
                             out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Per-sample weight gradient of a channel norm, ``(N, C)`` or with
    ``bias`` ``(N, 2C)`` = ``[dgamma | dbeta]``: the x_hat of each (sample,
    group) block times g, summed over the spatial positions (fp32)."""
    dev = nat.require_device(x, g)
    if x.shape != g.shape or x.dim() < 2:
        raise ValueError("channel_norm_weight_grad expects x and g of one (N, C, *spatial) shape")
    if x.dtype != g.dtype:
        raise ValueError("channel_norm_weight_grad operands must share one dtype")
    out_dtype = out_dtype or x.dtype
    x, n, c, s = _channel_rows(x)
    g = g.contiguous()
    width = c * (2 if bias else 1)
    if s == 0 or n == 0:
        return torch.zeros(n, width, dtype=out_dtype, device=dev)
    out = torch.empty(n, width, dtype=out_dtype, device=dev)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_channel_norm_workspace(n, groups, ctypes.byref(nbytes)), "channel_norm_weight_grad")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "channel_norm_weight_grad", lib.da_channel_norm_weight_grad,
         x.data_ptr(), g.data_ptr(), nat.dtype_code(x.dtype), n, c, s, groups, float(eps), int(bias),
         out.data_ptr(), nat.dtype_code(out_dtype), width, ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


def channel_norm_xhat(x: torch.Tensor, *, groups: int, eps: float, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """A channel norm's normalised input, in x's (N, C, *spatial) layout."""
    dev = nat.require_device(x)
    out_dtype = out_dtype or x.dtype
    x, n, c, s = _channel_rows(x)
    out = torch.empty(x.shape, dtype=out_dtype, device=dev)
    if n * c * s == 0:
        return out
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_channel_norm_workspace(n, groups, ctypes.byref(nbytes)), "channel_norm_xhat")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "channel_norm_xhat", lib.da_channel_norm_xhat,
         x.data_ptr(), nat.dtype_code(x.dtype), n, c, s, groups, float(eps), out.data_ptr(),
         nat.dtype_code(out_dtype), ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


def match_rows(src: torch.Tensor, x: torch.Tensor) -> torch.Tensor | None:
    """int64 ``(n_x,)``: the row of ``src (n_src, d)`` each row of ``x (n_x, d)``
    was gathered from -- the k-th occurrence of a value in x takes the k-th
    (ascending) src row holding it, verified by float equality -- or None when
    some row cannot be placed (one host read of the status word)."""
    dev = nat.require_device(src, x)
    if src.dim() != 2 or x.dim() != 2 or src.shape[1] != x.shape[1]:
        raise ValueError("match_rows expects (n_src, d) and (n_x, d) rows of one width")
    if src.dtype != x.dtype:
        raise ValueError("match_rows operands must share one dtype")
    n_src, n_x = src.shape[0], x.shape[0]
    token = torch.empty(n_x, dtype=torch.int64, device=dev)
    if n_x == 0:
        return token
    if n_src == 0:
        return None
    d = -(-src.shape[1] // _chunk_elems(src.dtype)) * _chunk_elems(src.dtype)
    src, x = prepare_rows(src, d), prepare_rows(x, d)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_match_rows_workspace(n_src, n_x, ctypes.byref(nbytes)), "match_rows")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "match_rows", lib.da_match_rows,
         src.data_ptr(), n_src, src.stride(0), x.data_ptr(), n_x, x.stride(0), d, nat.dtype_code(src.dtype),
         token.data_ptr(), status.data_ptr(), ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return None if int(status.item()) else token


def selftest_mfma(dtype: torch.dtype, a: torch.Tensor, b: torch.Tensor, shape: int = 32) -> torch.Tensor:
    """Raw accumulator dump of one MFMA block (see da_selftest_mfma)."""
    dev = nat.require_device(a, b)
    regs = 16 if shape == 32 else 4
    out = torch.empty(64 * regs, dtype=torch.float32, device=dev)
    nat.check(
        nat.load().da_selftest_mfma(nat.dtype_code(dtype), shape, a.data_ptr(), b.data_ptr(),
                                    out.data_ptr(), nat.stream_ptr(dev)),
        "selftest_mfma",
    )
    return out.view(64, regs)


def project_rows(x: torch.Tensor, pt: torch.Tensor, *, bias: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """``x @ pt.T (+ bias)`` over the last axis: x (..., d), pt (k, d) -- the
    transposed projection matrix -- bias (k,) fp32 or None."""
    dev = nat.require_device(x, pt, bias)
    if pt.dim() != 2 or x.shape[-1] > pt.shape[1]:
        raise ValueError("project_rows: pt must be (k, >= d)")
    if x.dtype != pt.dtype:
        raise ValueError("project_rows: x and the matrix must share one dtype")
    out_dtype = out_dtype or x.dtype
    d = x.shape[-1]
    k = pt.shape[0]
    rows = x.numel() // d if d else 0
    out = torch.empty(*x.shape[:-1], k, dtype=out_dtype, device=dev)
    if rows == 0 or k == 0:
        return out
    vec = _chunk_elems(x.dtype)
    dp = -(-d // vec) * vec
    flat = prepare_rows(x.reshape(rows, d), dp)
    ptp = prepare_rows(pt[:, :d] if pt.shape[1] != dp else pt, dp)
    if bias is not None:
        bias = bias.to(torch.float32).contiguous()
        if bias.numel() != k:
            raise ValueError("project_rows: bias must have k entries")
    _run(dev, "project_rows", nat.load().da_project_rows,
         flat.data_ptr(), nat.dtype_code(x.dtype), rows, dp, flat.stride(0), ptp.data_ptr(), k, ptp.stride(0),
         bias.data_ptr() if bias is not None else None, out.data_ptr(), nat.dtype_code(out_dtype), k,
         nat.stream_ptr(dev))
    return out


def project_outer(a: torch.Tensor, g: torch.Tensor, pin_t: torch.Tensor, pout_t: torch.Tensor, *,
                  bias_in: torch.Tensor | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Fused ``bmm((g @ P_out)^T, a @ P_in (+ bias_in))`` flattened to (B, kg*ka).

    a (B, T, K), g (B, T, D); pin_t (ka, K) and pout_t (kg, D) are the
    transposed projection matrices; ka, kg <= 64."""
    dev = nat.require_device(a, g, pin_t, pout_t, bias_in)
    if a.dim() != 3 or g.dim() != 3 or a.shape[:2] != g.shape[:2]:
        raise ValueError("project_outer expects a (B, T, K) and g (B, T, D)")
    if not (a.dtype == g.dtype == pin_t.dtype == pout_t.dtype):
        raise ValueError("project_outer operands must share one dtype")
    out_dtype = out_dtype or a.dtype
    b, t, k = a.shape
    d = g.shape[-1]
    ka, kg = pin_t.shape[0], pout_t.shape[0]
    out = torch.empty(b, kg * ka, dtype=out_dtype, device=dev)
    if b == 0 or ka == 0 or kg == 0:
        return out
    if t == 0:
        return out.zero_()
    vec = _chunk_elems(a.dtype)
    kp, dp = -(-k // vec) * vec, -(-d // vec) * vec
    a, g = prepare_rows(a, kp), prepare_rows(g, dp)
    pin_t, pout_t = prepare_rows(pin_t[:, :k], kp), prepare_rows(pout_t[:, :d], dp)
    if bias_in is not None:
        bias_in = bias_in.to(torch.float32).contiguous()
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_project_outer_workspace(b, t, ka, kg, ctypes.byref(nbytes)), "project_outer")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "project_outer", lib.da_project_outer,
         a.data_ptr(), g.data_ptr(), nat.dtype_code(a.dtype), b, t, kp, dp, a.stride(0), a.stride(1),
         g.stride(0), g.stride(1), pin_t.data_ptr(), ka, pin_t.stride(0),
         bias_in.data_ptr() if bias_in is not None else None, pout_t.data_ptr(), kg, pout_t.stride(0),
         out.data_ptr(), nat.dtype_code(out_dtype), kg * ka, ws.data_ptr(), ws.numel(), nat.stream_ptr(dev))
    return out


def gather_entries(a: torch.Tensor, g: torch.Tensor, rows: torch.Tensor, cols: torch.Tensor, *,
                   bias: bool = False) -> torch.Tensor:
    """fp32 ``(B, n)``: entries ``(rows[k], cols[k])`` of every sample's linear
    weight gradient ``sum_t g[b,t,:]^T [a[b,t,:], 1]``, gathered from the
    factors (a (B, T, K), g (B, T, D); column K is the bias column)."""
    dev = nat.require_device(a, g, rows, cols)
    if a.dim() != 3 or g.dim() != 3 or a.shape[:2] != g.shape[:2]:
        raise ValueError("gather_entries expects a (B, T, K) and g (B, T, D)")
    if a.dtype != g.dtype:
        raise ValueError("gather_entries factors must share one dtype")
    if rows.shape != cols.shape or rows.dim() != 1:
        raise ValueError("rows and cols must be matching 1-D index tensors")
    if a.stride(-1) != 1 or g.stride(-1) != 1:
        a, g = a.contiguous(), g.contiguous()
    rows, cols = rows.to(torch.int64).contiguous(), cols.to(torch.int64).contiguous()
    b, t, k = a.shape
    n = rows.numel()
    out = torch.empty(b, n, dtype=torch.float32, device=dev)
    if b == 0 or n == 0:
        return out
    _run(dev, "gather_entries", nat.load().da_gather_entries,
         a.data_ptr(), g.data_ptr(), nat.dtype_code(a.dtype), b, t, k, g.shape[-1], a.stride(0), a.stride(1),
         g.stride(0), g.stride(1), int(bias), rows.data_ptr(), cols.data_ptr(), n, out.data_ptr(), out.stride(0),
         nat.stream_ptr(dev))
    return out


def moe_topk(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Router top-k of softmax(logits) -> (weights (N, k) fp32, indices (N, k) int64)."""
    dev = nat.require_device(logits)
    if logits.dim() != 2:
        raise ValueError("moe_topk expects (tokens, experts) logits")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    n, e = logits.shape
    weights = torch.empty(n, k, dtype=torch.float32, device=dev)
    index = torch.empty(n, k, dtype=torch.int64, device=dev)
    _run(dev, "moe_topk", nat.load().da_moe_topk,
         logits.data_ptr(), nat.dtype_code(logits.dtype), n, e, k, logits.stride(0), weights.data_ptr(),
         index.data_ptr(), nat.stream_ptr(dev))
    return weights, index


def counting_sort(keys: torch.Tensor, bins: int, *, slot_major: bool = False,
                  key_div: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    """Stable counting sort -> (offsets (bins+1) int32, perm (n) int32).

    ``keys`` is int32/int64 (flattened), or with ``slot_major`` an int64
    (rows, k) matrix read column by column."""
    dev = nat.require_device(keys)
    if keys.dtype not in (torch.int32, torch.int64):
        raise ValueError("counting_sort keys must be int32 or int64")
    keys = keys.contiguous()
    if slot_major:
        if keys.dim() != 2 or keys.dtype != torch.int64:
            raise ValueError("slot-major keys must be an int64 (rows, k) matrix")
        rows, k = keys.shape
    else:
        keys = keys.reshape(-1)
        rows, k = keys.numel(), 1
    n = keys.numel()
    offsets = torch.empty(bins + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    k32 = keys.data_ptr() if keys.dtype == torch.int32 else None
    k64 = keys.data_ptr() if keys.dtype == torch.int64 else None
    _run(dev, "counting_sort", nat.load().da_counting_sort,
         k32, k64, n, rows, k, int(slot_major), key_div, bins, offsets.data_ptr(), perm.data_ptr(),
         nat.stream_ptr(dev))
    return offsets, perm[:n]


def compact_rows(mask: torch.Tensor, batch: int, tokens: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``(seg (B+1) int32, rows (B*T) int32)``: the rows whose mask entry is set,
    in order, grouped by sample (row ``b*T + t``); the first ``seg[B]`` entries
    of ``rows`` are written."""
    dev = nat.require_device(mask)
    n = batch * tokens
    if mask.numel() != n:
        raise ValueError(f"compact_rows: mask has {mask.numel()} entries, expected {n}")
    flags = mask.contiguous().view(torch.uint8) if mask.dtype == torch.bool else mask.to(torch.uint8).contiguous()
    seg = torch.empty(batch + 1, dtype=torch.int32, device=dev)
    rows = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    _run(dev, "compact_rows", nat.load().da_compact_rows,
         flags.data_ptr() if n else None, batch, tokens, seg.data_ptr(), rows.data_ptr(), nat.stream_ptr(dev))
    return seg, rows


def moe_route(index: torch.Tensor, n_experts: int, batch: int, tokens: int):
    """Expert routing of one side: ``(offsets (E+1), entries (N*k), seg (E, B+1),
    rows (N*k))`` int32, as documented for ``da_moe_route``."""
    dev = nat.require_device(index)
    if index.dim() != 2 or index.dtype != torch.int64:
        raise ValueError("moe_route expects the (N, k) int64 top-k index matrix")
    index = index.contiguous()
    n, k = index.shape
    total = max(n * k, 1)
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    entries = torch.empty(total, dtype=torch.int32, device=dev)
    seg = torch.empty(n_experts, batch + 1, dtype=torch.int32, device=dev)
    rows = torch.empty(total, dtype=torch.int32, device=dev)
    _run(dev, "moe_route", nat.load().da_moe_route,
         index.data_ptr(), n, k, n_experts, batch, tokens, offsets.data_ptr(), entries.data_ptr(),
         seg.data_ptr(), rows.data_ptr(), nat.stream_ptr(dev))
    return offsets, entries[: n * k], seg, rows[: n * k]


def ghost_gram_segmented(a1, g1, seg1, idx1, tokens1, a2, g2, seg2, idx2, tokens2, *,
                         bias: bool = False, out: torch.Tensor | None = None,
                         accumulate: bool = False) -> torch.Tensor:
    """Ghost cross-gram over row segments: side s sample b owns flat rows
    [seg_s[b], seg_s[b+1]) of the (rows, width) factors, gathered through idx_s
    (int32 row ids, or None for identity); ``tokens_s`` >= the longest segment."""
    dev = nat.require_device(a1, g1, a2, g2, seg1, seg2)
    if not (a1.dtype == g1.dtype == a2.dtype == g2.dtype):
        raise ValueError("ghost_gram_segmented factors must share one dtype")
    for t in (seg1, seg2) + tuple(x for x in (idx1, idx2) if x is not None):
        if t.dtype != torch.int32:
            raise ValueError("segment offsets and row indices must be int32")
    code = nat.dtype_code(a1.dtype)
    vec = _chunk_elems(a1.dtype)
    k = -(-a1.shape[-1] // vec) * vec
    d = -(-g1.shape[-1] // vec) * vec
    a1, a2 = prepare_rows(a1, k), prepare_rows(a2, k)
    g1, g2 = prepare_rows(g1, d), prepare_rows(g2, d)
    b1, b2 = seg1.numel() - 1, seg2.numel() - 1
    if out is None:
        out = torch.empty(b1, b2, dtype=torch.float32, device=dev)
        accumulate = False
    s1 = _side(a1, g1, bias, seg=seg1.contiguous(), index=idx1, tokens=max(int(tokens1), 1))
    s2 = _side(a2, g2, bias, seg=seg2.contiguous(), index=idx2, tokens=max(int(tokens2), 1))
    lib = nat.load()
    nbytes = ctypes.c_size_t(0)
    nat.check(lib.da_ghost_gram_workspace(s1, s2, k, d, code, ctypes.byref(nbytes)), "ghost_gram_segmented")
    ws = nat.workspace(nbytes.value, dev)
    _run(dev, "ghost_gram_segmented", lib.da_ghost_gram,
         s1, s2, k, d, code, out.data_ptr(), out.stride(0), int(accumulate), ws.data_ptr(), ws.numel(),
         nat.stream_ptr(dev))
    return out
