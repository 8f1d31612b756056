"""Factorized-vs-materialized routing, re-calibrated to measured MI355X rates.

The reference routes on flop counts alone (``dattri_llm/gradient/ops/dot.py:728-753``):
materialize iff ``kappa * B1*B2*S^2*(D+K) >= (B1+B2)*S*D*K + B1*B2*D*K``.  On
MI355X the two routes run on kernels with very different efficiencies -- the
ghost route is one MFMA-bound kernel, the materialized route is an MFMA-bound
dW kernel plus an HBM-bound score GEMM that streams every dense row -- so the
time model prices each term at the rate its kernel actually achieves:

    t_F = 2*B1*B2*S1*S2*(K+D) / R_ghost                               + 1 launch
    t_M = 2*(B1*S1 + B2*S2)*D*K / R_mat
          + 2*(B1+B2)*D*K*e / R_stream (dW written once and read once)  + 3 launches

with ``e`` the element size, and each extent rounded up to the kernel's tile
(ghost: 256 x 128 tokens; dW: 256 x 256 outputs, 32-token stages).  The rates come from :func:`calibrate` (timed
kernels on the current GPU) or the committed MI355X measurement.

``set_routing_policy("calibrated")`` makes ``maybe_use_materialized_gram`` use
this model; the default ``"flops"`` keeps the reference's rule bit-for-bit
(its known-answer tests pin it).  Both routes are exact, so the policy changes
speed, never scores.
"""

from __future__ import annotations

import json
import os
from dataclasses import asdict, dataclass

# The packed (segmented) ghost kernel over fully live rows runs at about this
# share of the dense engine's rate (measured at K = D = 4096, bf16: 895-910
# against 1121-1139 TFLOP/s at T = 256 and 512), with no padding but the last
# tile's.  The factorized route packs a pair whose dense 256 x 128-token tiles
# hold a smaller share of live row pairs than this (every T up to about 200
# tokens on both sides, and single-token rows).
PACKED_RELATIVE_RATE = 0.8


def ghost_tile_share(s1: int, s2: int) -> float:
    """Share of the dense ghost engine's tile work (256 side-1 x 128 side-2
    tokens per sample pair) that falls on real token pairs."""
    if s1 <= 0 or s2 <= 0:
        return 1.0
    return (s1 / (-(-s1 // 256) * 256)) * (s2 / (-(-s2 // 128) * 128))


_POLICIES = ("flops", "calibrated")
_policy = "flops"
_model = None
RATES_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mi355x_rates.json")


def set_routing_policy(policy: str) -> str:
    """Select ``"flops"`` (the reference rule) or ``"calibrated"``; returns the previous one."""
    global _policy  # noqa: PLW0603
    if policy not in _POLICIES:
        raise ValueError(f"routing policy must be one of {_POLICIES}, got {policy!r}")
    previous, _policy = _policy, policy
    return previous


def get_routing_policy() -> str:
    return _policy


@dataclass(frozen=True)
class CostModel:
    """Measured rates of the three kernels of the two routes."""

    ghost_tflops: float
    materialize_tflops: float
    stream_gbs: float
    launch_us: float = 8.0
    elem_bytes: int = 2
    source: str = ""

    # The kernels run whole tiles: the ghost tile is 256 (side-1 tokens) x 128
    # (side-2 tokens), the dW tile 256 x 256 outputs over 32-token stages.  The
    # rates are measured on whole tiles, so each term is priced on the padded
    # work its kernel actually does.
    @staticmethod
    def _up(n, m):
        return -(-n // m) * m

    def time_factorized(self, b1, b2, s1, s2, k, d) -> float:
        # the dense tiles' padded work, or the packed kernel's at its lower rate
        dense = 2.0 * b1 * b2 * self._up(s1, 256) * self._up(s2, 128) * (k + d)
        packed = 2.0 * b1 * b2 * s1 * s2 * (k + d) / PACKED_RELATIVE_RATE
        return min(dense, packed) / (self.ghost_tflops * 1e12) + self.launch_us * 1e-6

    def time_materialized(self, b1, b2, s1, s2, k, d) -> float:
        tiles = self._up(d, 256) * self._up(k, 256)
        flops = 2.0 * (b1 * self._up(s1, 32) + b2 * self._up(s2, 32)) * tiles
        stream = 2.0 * (b1 + b2) * d * k * self.elem_bytes
        return (flops / (self.materialize_tflops * 1e12) + stream / (self.stream_gbs * 1e9)
                + 3 * self.launch_us * 1e-6)

    def prefers_materialized(self, b1, b2, s1, s2, k, d, kappa: float = 1.0) -> bool:
        return kappa * self.time_factorized(b1, b2, s1, s2, k, d) >= self.time_materialized(b1, b2, s1, s2, k, d)

    def save(self, path: str = RATES_FILE) -> None:
        with open(path, "w") as f:
            json.dump(asdict(self), f, indent=2)
            f.write("\n")


def calibrated_model() -> CostModel:
    """The active calibrated model (loaded from the committed rates file)."""
    global _model  # noqa: PLW0603
    if _model is None:
        with open(RATES_FILE) as f:
            _model = CostModel(**json.load(f))
    return _model


def use_model(model: CostModel) -> None:
    """Install a freshly calibrated model for this process."""
    global _model  # noqa: PLW0603
    _model = model


def calibrate(device=None, repeats: int = 3) -> CostModel:
    """Time the three kernels on the current GPU at the shapes the routes run
    at and return the rates (TFLOP/s for the MFMA kernels, GB/s for the score
    stream):

    * ghost: 32 x 16 sample pairs of a d = 4096 linear at T = 512 (a slice of
      the 256 x 64 ghost workload);
    * dW: 8 samples x 2048 tokens of a 4096 -> 14336 linear (the Llama-3-8B
      block's gate projection);
    * score stream: 8 train x 64 query rows of the same layer's dense
      gradients (58.7 M weights, k-blocked as the dW kernel writes them).
    """
    import torch

    from dattri_llm_amd import kernels

    dev = torch.device(device or "cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16

    def rnd(*shape):
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32).to(bf)

    def timed(fn):
        fn()
        torch.cuda.synchronize(dev)
        best = float("inf")
        for _ in range(repeats):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize(dev)
            best = min(best, s.elapsed_time(e) * 1e-3)
        return best

    b1, b2, t, k = 32, 16, 512, 4096
    a1, g1 = rnd(b1, t, k), rnd(b1, t, k)
    a2, g2 = rnd(b2, t, k), rnd(b2, t, k)
    t_ghost = timed(lambda: kernels.ghost_gram(a1, g1, a2, g2))
    ghost = 2.0 * b1 * b2 * t * t * 2 * k / t_ghost / 1e12
    del a1, g1, a2, g2
    bm, tm, km, dm = 8, 2048, 4096, 14336
    a, g = rnd(bm, tm, km), rnd(bm, tm, dm)
    t_mat = timed(lambda: kernels.materialize_linear(a, g, blocked=True))
    mat = 2.0 * bm * tm * km * dm / t_mat / 1e12
    m1 = kernels.materialize_linear(a, g, blocked=True)
    del a, g
    m2 = rnd(km * dm // 64, 64, 64).permute(1, 0, 2)  # k-blocked (64, W/64, 64) view
    t_score = timed(lambda: kernels.score_gemm([(m1, m2)]))
    stream = (8 + 64) * km * dm * 2 / t_score / 1e9
    name = torch.cuda.get_device_name(dev)
    return CostModel(round(ghost, 1), round(mat, 1), round(stream, 1),
                     source=f"calibrate(repeats={repeats}) on {name}: ghost 32x16 pairs T=512 d=4096; "
                            f"dW 8 x 2048 tokens 4096->14336; score 8x64 rows of the k-blocked 4096x14336 layer")
