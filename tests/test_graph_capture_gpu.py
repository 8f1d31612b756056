"""The scoring entry point inside a captured HIP graph.

``ops.layerwise_cross_dot`` over a block of linear (factorized, with and
without a bias column, dense on one side) and RMSNorm layers is captured on a
side stream after one eager call with the same tensors.  The eager call
probes the query side's live rows (the only host read on the path) and the
probe is cached per tensor, so the captured call makes no host round trip.
Every replay is checked bit for bit against the eager result, with eager work
and synchronizations between the replays; a second eager call after the
replays still matches (the graph left no state behind).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _block(device, dtype, seed):
    from dattri_llm_amd.gradient import Factorized, Gradient, ops

    gen = torch.Generator().manual_seed(seed)

    def r(*shape):
        return torch.randn(*shape, generator=gen).to(dtype).to(device)

    def pair(bt, tt, bq, tq):
        tr = {"lin": Factorized(r(bt, tt, 48), r(bt, tt, 32), module_kwargs={"has_bias": True}),
              "lin2": Factorized(r(bt, tt, 64), r(bt, tt, 16)),
              "norm": Factorized(r(bt, tt, 32), r(bt, tt, 32))}
        te = {"lin": Factorized(r(bq, tq, 48), r(bq, tq, 32), module_kwargs={"has_bias": True}),
              "lin2": ops.materialize(Factorized(r(bq, tq, 64), r(bq, tq, 16)), "nn.Linear"),
              "norm": Factorized(r(bq, tq, 32), r(bq, tq, 32))}
        lts = {"lin": "nn.Linear", "lin2": "nn.Linear", "norm": "nn.RMSNorm"}

        def grad(d):
            reps = {n: ("materialized" if isinstance(v, torch.Tensor) else "factorized") for n, v in d.items()}
            idx = {n: ("batch" if isinstance(v, torch.Tensor) else "batch_token") for n, v in d.items()}
            return Gradient(reps, d, lts, idx)

        return grad(tr), grad(te)

    return pair(5, 40, 3, 24)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layerwise_cross_dot_replays_equal_eager(device, dtype):
    from dattri_llm_amd.gradient import ops

    print(f"graph capture of layerwise_cross_dot dtype={dtype}", flush=True)
    train, test = _block(device, dtype, 11)
    eager = ops.layerwise_cross_dot(train, test)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):  # a warm-up on the capture stream, as torch's graph API expects
        warm = ops.layerwise_cross_dot(train, test)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(warm, eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = ops.layerwise_cross_dot(train, test)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}"
        assert torch.equal(ops.layerwise_cross_dot(train, test), eager)  # eager work between replays
        torch.cuda.synchronize()
    del graph
    assert torch.equal(ops.layerwise_cross_dot(train, test), eager)
