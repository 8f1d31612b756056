"""Shared test setup: import paths, the ``gpu`` marker, seeded inputs."""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "dattri-llm_amd")
for _p in (PKG_ROOT, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def rel_err(got, ref) -> float:
    """Normwise relative error max|got - ref| / max|ref| (entrywise relative
    error is ill-posed for near-zero scores)."""
    import numpy as np

    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = float(np.abs(ref).max()) if ref.size else 1.0
    return float(np.abs(got - ref).max() / (denom if denom > 0 else 1.0)) if ref.size else 0.0


# The spec bar: normwise relative error for bf16/fp16 inputs with fp32
# accumulation, and for fp32 inputs.
SPEC_BAR = {"bfloat16": 1e-2, "float16": 1e-2, "float32": 1e-3, "float64": 1e-3}
# What fp32 accumulation against the float64 oracle on identical (already
# rounded) inputs actually leaves, with margin; a result rounded to a 2-byte
# dtype adds half an ulp of its own entries (the unit roundoff: 2^-8 for bf16's
# 8-bit significand, 2^-11 for fp16's 11).
TIGHT_FP32 = 1e-5
HALF_ULP = {"bfloat16": 2.0**-8, "float16": 2.0**-11}


def roundings(n: int, dtype: str = "bfloat16") -> float:
    """Tight bound for a result that passes through ``n`` roundings to a 2-byte
    dtype on the way (an intermediate dense gradient stored in bf16, a bf16
    output): each perturbs an entry by at most half an ulp."""
    return TIGHT_FP32 + n * HALF_ULP[dtype]


def stable_seed(case) -> int:
    """A seed from a test case's parameters that is the same in every process
    (``hash`` of a tuple holding strings is salted per process)."""
    import zlib

    return zlib.crc32(repr(case).encode()) % 1000


def _dtype_name(dtype) -> str:
    return str(dtype).replace("torch.", "")


def assert_parity(got, ref, in_dtype, *, out_dtype=None, tight=None, label=""):
    """Assert both bars on a GPU result against its oracle.

    ``got`` is a tensor (its dtype is the output dtype unless ``out_dtype`` is
    given) or an array of fp32 results; ``in_dtype`` is the dtype of the
    inputs the kernels read (picks the spec bar).  The tight bound is
    ``tight`` or TIGHT_FP32 plus the output rounding.  With DA_PARITY_LOG set,
    the tight bound is logged to that file instead of asserted (the spec bar
    still holds), to measure the errors the kernels leave."""
    import numpy as np

    if hasattr(got, "detach"):
        out_dtype = out_dtype or got.dtype
        got = got.detach().double().cpu().numpy()
    if hasattr(ref, "detach"):
        ref = ref.detach().double().cpu().numpy()
    out_name = _dtype_name(out_dtype) if out_dtype is not None else "float32"
    err = rel_err(np.asarray(got), np.asarray(ref))
    spec = SPEC_BAR[_dtype_name(in_dtype)]
    bound = tight if tight is not None else TIGHT_FP32 + HALF_ULP.get(out_name, 0.0)
    assert err <= spec, f"{label} normwise error {err:.3e} above the {spec:g} bar"
    log = os.environ.get("DA_PARITY_LOG")
    if log:
        import json

        with open(log, "a") as f:
            f.write(json.dumps({"test": os.environ.get("PYTEST_CURRENT_TEST", ""), "label": label,
                                "err": err, "bound": bound, "out": out_name}) + "\n")
        return err
    assert err <= bound, f"{label} normwise error {err:.3e} above the tight bound {bound:.1e}"
    return err


def _bf16_keys(bits):
    """Monotone integer keys of bf16 bit patterns (int16 view): adjacent
    representable values differ by 1, and +0 and -0 share key 0."""
    import numpy as np

    b = np.asarray(bits, dtype=np.int32) & 0xFFFF
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def assert_bf16_rounded(got, ref, *, max_ulps=1, max_frac=2e-3, label=""):
    """Assert that the bf16 tensor ``got`` is the float64 ``ref`` rounded to
    bf16, up to what fp32 accumulation in another order can leave: at most
    ``max_frac`` of the entries off round-to-nearest-even(ref) at all, and none
    more than ``max_ulps`` bf16 ulps off it unless its absolute error is
    within TIGHT_FP32 of max|ref| (an entry summed down to near zero by
    cancellation carries fp32's absolute error over a tiny ulp).  A systematic
    relative error of a fraction of an ulp (a dropped term, a wrong scale)
    moves a large share of the entries across a rounding boundary and fails
    the first test; fp32 accumulation moves only entries within ~1e-6 of one."""
    import numpy as np
    import torch

    assert got.dtype == torch.bfloat16, got.dtype
    ref = np.asarray(ref, dtype=np.float64)
    want = torch.from_numpy(ref.astype(np.float32)).to(torch.bfloat16)
    got = got.detach().cpu().reshape(want.shape).contiguous()
    dist = np.abs(_bf16_keys(got.view(torch.int16).numpy()) - _bf16_keys(want.view(torch.int16).numpy()))
    frac = float(np.count_nonzero(dist)) / max(dist.size, 1)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    abs_err = np.abs(got.double().numpy() - ref)
    far = (dist > max_ulps) & (abs_err > TIGHT_FP32 * scale)
    worst = int(dist[far].max()) if far.any() else 0
    assert not far.any(), f"{label}: {int(far.sum())} entries up to {worst} bf16 ulps from the rounded oracle"
    assert frac <= max_frac, f"{label}: {frac:.2e} of entries off the rounded oracle (limit {max_frac:g})"
    return frac
