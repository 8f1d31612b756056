"""Compute-dtype policy (same contract as ``dattri_llm/gradient/ops/dtypes.py``).

``"auto"`` resolves to the promoted dtype of the floating operands (bf16 in
stays bf16), an explicit dtype forces it.  On this path every kernel
accumulates in fp32 whatever the policy; the policy decides the operand dtype
the kernels read and the dtype results are returned in.
"""

from __future__ import annotations

from contextlib import contextmanager

import torch

_POLICY: str | torch.dtype = "auto"
_NAMED = {
    "auto": "auto",
    "float32": torch.float32,
    "fp32": torch.float32,
    "float64": torch.float64,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
    "float16": torch.float16,
    "fp16": torch.float16,
}


def _as_policy(policy):
    if isinstance(policy, torch.dtype):
        return policy
    if isinstance(policy, str) and policy in _NAMED:
        return _NAMED[policy]
    raise ValueError(
        "compute dtype policy must be 'auto', a torch.dtype, or one of "
        f"{sorted(k for k in _NAMED if k != 'auto')}; got {policy!r}"
    )


def set_compute_dtype(policy):
    """Set the process-wide compute dtype; returns the policy it replaces."""
    global _POLICY  # noqa: PLW0603
    previous, _POLICY = _POLICY, _as_policy(policy)
    return previous


def get_compute_dtype():
    return _POLICY


@contextmanager
def compute_dtype(policy):
    """Scope a compute-dtype policy to a block."""
    previous = set_compute_dtype(policy)
    try:
        yield
    finally:
        set_compute_dtype(previous)


def resolve(*tensors, minimum: torch.dtype | None = None) -> torch.dtype:
    """dtypes.py:84-107: the policy dtype, or the promotion of the floating operands."""
    if _POLICY != "auto":
        dtype = _POLICY
    else:
        dtype = None
        for t in tensors:
            if t is None or not t.is_floating_point():
                continue
            dtype = t.dtype if dtype is None else torch.promote_types(dtype, t.dtype)
        if dtype is None:
            dtype = torch.float32
    if minimum is not None:
        dtype = torch.promote_types(dtype, minimum)
    return dtype


def align(*tensors, minimum: torch.dtype | None = None):
    """Cast every floating operand to :func:`resolve`'s dtype (dtypes.py:110-126)."""
    dtype = resolve(*tensors, minimum=minimum)
    return tuple(
        t if (t is None or not t.is_floating_point() or t.dtype == dtype) else t.to(dtype)
        for t in tensors
    )


def as_float(*tensors, minimum: torch.dtype | None = None):
    """Like :func:`align` but integer operands are converted too (dtypes.py:129-143)."""
    dtype = resolve(*tensors, minimum=minimum)
    return tuple(t if (t is None or t.dtype == dtype) else t.to(dtype) for t in tensors)


def kernel_dtype(dtype: torch.dtype) -> torch.dtype:
    """The operand dtype a kernel reads for a resolved compute dtype: the MFMA
    kernels take fp32/fp16/bf16; float64 requests run as fp32 operands."""
    return torch.float32 if dtype == torch.float64 else dtype
