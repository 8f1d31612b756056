"""ctypes binding of ``libdattri_amd.so`` (the gfx950 HIP kernels).

The library is built in-tree by ``dattri-llm_amd/build.py`` (``__graft_entry__.build()``).
There is no fallback: every op that needs a kernel raises
:class:`NativeLibraryError` when the library is missing or the tensors are not
on a ROCm device.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libdattri_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 13

DA_F32, DA_F16, DA_BF16 = 0, 1, 2
DA_OK, DA_ERR_INVALID, DA_ERR_UNSUPPORTED, DA_ERR_HIP, DA_ERR_WORKSPACE = 0, 1, 2, 3, 4

DTYPE_CODE = {torch.float32: DA_F32, torch.float16: DA_F16, torch.bfloat16: DA_BF16}
ELEM_BYTES = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}


class NativeLibraryError(RuntimeError):
    """The HIP library is unavailable or was handed tensors it cannot run on."""


class FactorSide(ctypes.Structure):
    """Mirror of ``da_factor_side`` (include/dattri_amd.h)."""

    _fields_ = [
        ("act", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("batch", ctypes.c_int64),
        ("tokens", ctypes.c_int64),
        ("act_bstride", ctypes.c_int64),
        ("act_tstride", ctypes.c_int64),
        ("grad_bstride", ctypes.c_int64),
        ("grad_tstride", ctypes.c_int64),
        ("seg_offsets", ctypes.c_void_p),
        ("row_index", ctypes.c_void_p),
        ("has_bias", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_SZ = ctypes.c_size_t
_SIDE = ctypes.POINTER(FactorSide)

# name -> (restype, argtypes).  Every symbol include/dattri_amd.h declares.
SIGNATURES: dict[str, tuple[object, list]] = {
    "da_abi_version": (_I32, []),
    "da_last_error": (ctypes.c_char_p, []),
    "da_selftest_mfma": (_I32, [_I32, _I32, _P, _P, _P, _P]),
    "da_ghost_gram_workspace": (_I32, [_SIDE, _SIDE, _I64, _I64, _I32, ctypes.POINTER(_SZ)]),
    "da_ghost_gram": (_I32, [_SIDE, _SIDE, _I64, _I64, _I32, _P, _I64, _I32, _P, _SZ, _P]),
    "da_ghost_gram_diag_workspace": (_I32, [_SIDE, _SIDE, _I64, _I64, _I32, ctypes.POINTER(_SZ)]),
    "da_ghost_gram_diag": (_I32, [_SIDE, _SIDE, _I64, _I64, _I32, _P, _I64, _I32, _P, _SZ, _P]),
    "da_ghost_gram_grouped_workspace": (_I32, [_SIDE, _SIDE, _I32, _P, _P, _I32, ctypes.POINTER(_SZ)]),
    "da_ghost_gram_grouped": (_I32, [_SIDE, _SIDE, _I32, _P, _P, _I32, _P, _I64, _I32, _P, _SZ, _P]),
    "da_ghost_gram_per_token_workspace": (_I32, [_SIDE, _SIDE, _I64, _I64, _I32, ctypes.POINTER(_SZ)]),
    "da_ghost_gram_per_token": (
        _I32, [_SIDE, _SIDE, _I64, _I64, _I32, _P, _I64, _I64, _I64, _I32, _P, _SZ, _P]),
    "da_embedding_cross_gram_workspace": (_I32, [_SIDE, _SIDE, _I64, _I32, _I32, ctypes.POINTER(_SZ)]),
    "da_embedding_cross_gram": (_I32, [_SIDE, _SIDE, _I64, _I32, _I32, _P, _I64, _I32, _P, _SZ, _P]),
    "da_embedding_cross_gram_per_token_workspace": (_I32, [_SIDE, _SIDE, _I64, _I32, ctypes.POINTER(_SZ)]),
    "da_embedding_cross_gram_per_token": (
        _I32, [_SIDE, _SIDE, _I64, _I32, _P, _I64, _I64, _I64, _I32, _P, _SZ, _P]),
    "da_dense_per_token_embedding": (
        _I32, [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64,
               _I32, _P]),
    "da_dense_per_token_workspace": (_I32, [_SIDE, _I64, _I64, _I64, _I32, ctypes.POINTER(_SZ)]),
    "da_dense_per_token": (
        _I32, [_SIDE, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _I32, _P, _I64, _I64, _I64, _I32, _P, _SZ, _P]),
}

class DenseLayer(ctypes.Structure):
    """Mirror of ``da_dense_layer`` (include/dattri_amd.h)."""

    _fields_ = [
        ("m1", ctypes.c_void_p),
        ("m2", ctypes.c_void_p),
        ("width", ctypes.c_int64),
        ("ld1", ctypes.c_int64),
        ("ld2", ctypes.c_int64),
        ("blk1", ctypes.c_int64),
        ("blk2", ctypes.c_int64),
    ]


_LAYERS = ctypes.POINTER(DenseLayer)
SIGNATURES.update(
    {
        "da_materialize_linear": (
            _I32,
            [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _I32, _I64, _I64, _I64, _P],
        ),
        "da_gather_embedding_entries": (
            _I32, [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P]),
        "da_materialize_embedding_workspace": (_I32, [_I64, _I64, _I64, _I32, ctypes.POINTER(_SZ)]),
        "da_materialize_embedding": (
            _I32, [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _SZ, _P]),
        "da_row_gram": (_I32, [_P, _I32, _I64, _I64, _I64, _P, _I64, _I32, _P, _SZ, _P]),
        "da_row_gram_workspace": (_I32, [_I64, _I64, _I32, ctypes.POINTER(_SZ)]),
        "da_nonzero_rows": (_I32, [_P, _I32, _I64, _I64, _I64, _P, _P]),
        "da_score_gemm_workspace": (_I32, [_I64, _I64, _LAYERS, _I32, _I32, ctypes.POINTER(_SZ)]),
        "da_row_dots_workspace": (_I32, [_I64, _LAYERS, _I32, _I32, ctypes.POINTER(_SZ)]),
        "da_row_dots": (_I32, [_I64, _LAYERS, _I32, _I32, _P, _I64, _I32, _P, _SZ, _P]),
        "da_score_gemm_noalloc": (_I32, [_I64, _I64, _LAYERS, _I32, _I32, _P, _I64, _I64, _I32, _P]),
        "da_score_gemm": (
            _I32,
            [_I64, _I64, _LAYERS, _I32, _I32, _P, _I64, _I64, _I32, _P, _SZ, _P],
        ),
        "da_norm_weight_grad_workspace": (_I32, [_I64, _I64, _I64, _I32, ctypes.POINTER(_SZ)]),
        "da_norm_weight_grad": (
            _I32,
            [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, ctypes.c_float, _I32,
             _P, _I32, _I64, _P, _SZ, _P],
        ),
        "da_match_rows_workspace": (_I32, [_I64, _I64, ctypes.POINTER(_SZ)]),
        "da_match_rows": (_I32, [_P, _I64, _I64, _P, _I64, _I64, _I64, _I32, _P, _P, _P, _SZ, _P]),
        "da_channel_norm_workspace": (_I32, [_I64, _I64, ctypes.POINTER(_SZ)]),
        "da_channel_norm_weight_grad": (
            _I32, [_P, _P, _I32, _I64, _I64, _I64, _I64, ctypes.c_float, _I32, _P, _I32, _I64, _P, _SZ, _P]),
        "da_channel_norm_xhat": (
            _I32, [_P, _I32, _I64, _I64, _I64, _I64, ctypes.c_float, _P, _I32, _P, _SZ, _P]),
        "da_norm_xhat": (
            _I32,
            [_P, _I32, _I64, _I64, _I64, _I32, ctypes.c_float, _P, _I32, _I64, _P],
        ),
    }
)

_FP = ctypes.POINTER(ctypes.c_float)
SIGNATURES.update(
    {
        "da_project_rows": (
            _I32,
            [_P, _I32, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _I32, _I64, _P],
        ),
        "da_project_outer_workspace": (_I32, [_I64, _I64, _I64, _I64, ctypes.POINTER(_SZ)]),
        "da_project_outer": (
            _I32,
            [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _P,
             _I64, _I64, _P, _I32, _I64, _P, _SZ, _P],
        ),
        "da_moe_topk": (_I32, [_P, _I32, _I64, _I32, _I32, _I64, _P, _P, _P]),
        "da_gather_entries": (
            _I32,
            [_P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _I64, _P, _I64, _P],
        ),
        "da_moe_route": (_I32, [_P, _I64, _I32, _I32, _I64, _I64, _P, _P, _P, _P, _P]),
    "da_counting_sort": (_I32, [_P, _P, _I64, _I64, _I64, _I32, _I64, _I32, _P, _P, _P]),
        "da_compact_rows": (_I32, [_P, _I64, _I64, _P, _P, _P]),
    }
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> str:
    return os.environ.get("DATTRI_AMD_LIB", LIB_PATH)


def load() -> ctypes.CDLL:
    """Load (once) and type the shared library; raise if it is absent."""
    global _lib  # noqa: PLW0603
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise NativeLibraryError(
                f"{LIB_NAME} not found at {path}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` "
                "(hipcc --offload-arch=gfx950)."
            )
        lib = ctypes.CDLL(path)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.da_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f"{path} has ABI {version}, expected {ABI_VERSION}; rebuild it.")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Map a non-zero status to the reference's exception types."""
    if status == DA_OK:
        return
    msg = (load().da_last_error() or b"").decode(errors="replace")
    text = f"{what}: {msg}" if msg else f"{what}: status {status}"
    if status == DA_ERR_INVALID:
        raise ValueError(text)
    if status == DA_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise NativeLibraryError(text)


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise NativeLibraryError(
                "dattri_llm_amd kernels run on a ROCm GPU (gfx950); got a tensor on "
                f"{t.device}. Move the gradients to the GPU first."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise NotImplementedError(f"dtype {dtype} is not supported by the HIP kernels") from None


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-side workspace from torch's caching allocator (16-byte aligned)."""
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)
