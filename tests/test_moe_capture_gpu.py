"""Routed expert captures to exact per-sample gradients on the MI355X (the
reference's TestDuplicateRows, tests/gradient/test_moe.py:479-495 and
tests/gradient/test_fused_experts.py:243-269).

A small top-2 MoE block gathers each expert's rows as the reference's
fused_experts.py:210-237 does (slot-major, ascending token), so an expert sees
an (n_e, d) matrix.  The rows are located in the block input with
locate_rows (the drop-in for RoutedTokenTracker._match), scattered back to
(B, T, d) by RowLayout.regroup, and materialize_factors of the regrouped
capture must equal each sample's expert gradient from its own backward pass
in float64 -- also when samples repeat rows (a duplicated sample, a shared
prefix), where only the k-th-occurrence rule places them right.  The routing
is fixed from the float64 router so both passes route alike."""

from __future__ import annotations

import copy

import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu

B, T, D, E, K = 3, 7, 16, 4, 2


class TinyMoE(nn.Module):
    def __init__(self):
        super().__init__()
        self.router = nn.Linear(D, E, bias=False)
        self.experts = nn.ModuleList(nn.Linear(D, D) for _ in range(E))

    def route(self, x):
        probs = torch.softmax(self.router(x.reshape(-1, D)).double(), dim=-1)
        w, idx = torch.topk(probs, K, dim=-1)
        return w, idx

    def forward(self, x, w, idx):
        b, t, _ = x.shape
        flat = x.reshape(b * t, D)
        out = torch.zeros_like(flat)
        mask = torch.nn.functional.one_hot(idx, E).permute(2, 1, 0)  # (E, K, B*T)
        for e in range(E):
            slot, tok = torch.where(mask[e])
            y = self.experts[e](flat[tok]) * w[tok, slot, None].to(flat.dtype)
            out = out.index_add(0, tok, y)
        return out.reshape(b, t, D)


@pytest.mark.parametrize("kind", ["distinct", "repeated-sample", "shared-prefix"])
def test_expert_gradients_stay_exact(device, kind):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.routing import locate_rows

    torch.manual_seed(0)
    model64 = TinyMoE().double()
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, D, generator=gen, dtype=torch.float64)
    if kind == "repeated-sample":
        x[1] = x[0]
    elif kind == "shared-prefix":
        x[2, :4] = x[1, :4]
    wout = torch.randn(B, T, D, generator=gen, dtype=torch.float64)
    with torch.no_grad():
        w, idx = model64.route(x)
    print(f"moe capture {kind}", flush=True)

    # each sample alone, float64 on the CPU
    truth = {e: [] for e in range(E)}
    for i in range(B):
        model64.zero_grad()
        sl = slice(i * T, (i + 1) * T)
        (model64(x[i:i + 1], w[sl], idx[sl]) * wout[i:i + 1]).sum().backward()
        for e, ex in enumerate(model64.experts):
            gw = ex.weight.grad if ex.weight.grad is not None else torch.zeros_like(ex.weight)
            gb = ex.bias.grad if ex.bias.grad is not None else torch.zeros_like(ex.bias)
            truth[e].append(torch.cat([gw, gb.unsqueeze(-1)], -1).flatten())

    # the batched fp32 pass on the GPU, expert captures by hooks
    model = copy.deepcopy(model64).float().to(device)
    caps = {}

    def keep(e):
        def hook(_mod, inputs, out):
            caps[e] = {"a": inputs[0].detach()}
            out.register_hook(lambda grad: caps[e].__setitem__("g", grad.detach()))
        return hook

    handles = [ex.register_forward_hook(keep(e)) for e, ex in enumerate(model.experts)]
    xd = x.float().to(device)
    (model(xd, w.to(device), idx.to(device)) * wout.float().to(device)).sum().backward()
    for h in handles:
        h.remove()

    flat = xd.reshape(B * T, D)
    for e in range(E):
        a_rows, g_rows = caps[e]["a"], caps[e]["g"]
        layout = locate_rows(a_rows, flat, B, T)
        assert layout is not None, (kind, e)
        a, g = layout.regroup(a_rows), layout.regroup(g_rows)
        got = ops.materialize_factors(a, g, "nn.Linear", module_kwargs={"has_bias": True})
        want = torch.stack(truth[e])
        torch.testing.assert_close(got.double().cpu(), want, rtol=1e-4, atol=1e-5 * max(1.0, want.abs().max().item()),
                                   msg=lambda m: f"[{kind}] expert {e}: {m}")
