"""Which dtype the ops compute in.

The contract is dattri-llm's compute-dtype policy
(``dattri_llm/gradient/ops/dtypes.py:84-143``): under ``"auto"`` an op works in
the promotion of its floating operands' dtypes (bf16 captures stay bf16, a
bf16/fp32 mix becomes fp32, integer operands such as token ids do not count);
a forced dtype overrides that everywhere; ``minimum`` raises the floor for
reductions that need it.  Results come back in that dtype.

On this path the policy has one more consumer: the kernels.  They read bf16,
fp16 or fp32 operands and always accumulate in fp32, so :func:`kernel_dtype`
maps a resolved dtype to the operand dtype a kernel is launched on (float64
requests run on fp32 operands; nothing here computes in float64).
"""

from __future__ import annotations

import contextlib
import functools

import torch

# Names accepted for a forced policy; short forms map to torch's own names.
_SHORT = {"fp32": "float32", "bf16": "bfloat16", "fp16": "float16"}
_FORCEABLE = ("float32", "float64", "bfloat16", "float16")


class _Policy:
    """The process-wide policy: ``forced`` is None under "auto"."""

    forced: torch.dtype | None = None

    @staticmethod
    def parse(spec) -> torch.dtype | None:
        if isinstance(spec, torch.dtype):
            return spec
        if spec == "auto":
            return None
        name = _SHORT.get(spec, spec) if isinstance(spec, str) else None
        if name in _FORCEABLE:
            return getattr(torch, name)
        accepted = sorted(set(_FORCEABLE) | set(_SHORT))
        raise ValueError(f"compute dtype policy must be 'auto', a torch.dtype, or one of {accepted}; got {spec!r}")

    def public(self):
        return "auto" if self.forced is None else self.forced


_policy = _Policy()


def set_compute_dtype(policy):
    """Set the process-wide compute dtype ("auto", a torch.dtype or a dtype
    name); returns the policy it replaces, in the same form."""
    previous = _policy.public()
    _policy.forced = _Policy.parse(policy)
    return previous


def get_compute_dtype():
    """"auto" or the forced torch.dtype."""
    return _policy.public()


@contextlib.contextmanager
def compute_dtype(policy):
    """The policy for the duration of a ``with`` block."""
    previous = set_compute_dtype(policy)
    try:
        yield
    finally:
        set_compute_dtype(previous)


def _floating(tensors):
    return [t.dtype for t in tensors if t is not None and t.is_floating_point()]


def resolve(*tensors, minimum: torch.dtype | None = None) -> torch.dtype:
    """The compute dtype for these operands: the forced one, else the promotion
    of the floating operands (fp32 when there are none), raised to ``minimum``."""
    if _policy.forced is not None:
        dtype = _policy.forced
    else:
        floating = _floating(tensors)
        dtype = functools.reduce(torch.promote_types, floating) if floating else torch.float32
    return dtype if minimum is None else torch.promote_types(dtype, minimum)


def align(*tensors, minimum: torch.dtype | None = None):
    """The operands with every floating one cast to :func:`resolve`'s dtype;
    integer tensors and None pass through, as do tensors already in it."""
    target = resolve(*tensors, minimum=minimum)
    return tuple(t.to(target) if t is not None and t.is_floating_point() and t.dtype != target else t
                 for t in tensors)


def as_float(*tensors, minimum: torch.dtype | None = None):
    """:func:`align` that converts integer operands too (for ops that need a
    floating input, such as a projection of token ids)."""
    target = resolve(*tensors, minimum=minimum)
    return tuple(t.to(target) if t is not None and t.dtype != target else t for t in tensors)


def kernel_dtype(dtype: torch.dtype) -> torch.dtype:
    """The operand dtype a kernel reads for a resolved compute dtype: bf16,
    fp16 and fp32 as they are, float64 as fp32 (fp32 accumulation either way)."""
    return torch.float32 if dtype == torch.float64 else dtype
