"""Parity of the MoE routed layer at the Mixtral shapes: 8 experts, top-2,
d 4096, fused gate_up 4096 -> 28672 and down 14336 -> 4096, 16 train x 256
tokens against 16 queries x 256 tokens, routed by the real router (softmax
top-2 of N(0, 1) logits).  The grouped ghost kernel runs every expert of both
linears in one launch; the float64 oracle sums the reference's per-expert
ghost products (its compact form, pinned against the dense-with-zeros regroup
in the CPU tests)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from conftest import assert_parity

pytestmark = pytest.mark.gpu

N_EXP, TOP_K, B, T = 8, 2, 16, 256
LAYERS = [("gate_up", 4096, 28672), ("down", 14336, 4096)]


def _rnd(gen, shape, scale, device):
    x = torch.empty(*shape, device=device)
    x.normal_(0.0, scale, generator=gen)
    return x.to(torch.bfloat16)


def _side(gen, device):
    """Router logits and per-expert captures (routed order) of one side."""
    from dattri_llm_amd.gradient import ops

    logits = torch.empty(B * T, N_EXP, device=device).normal_(0.0, 1.0, generator=gen)
    _w, idx = ops.moe.router_topk(logits, TOP_K)
    rows = ops.moe.expert_rows(idx, N_EXP)
    caps = []
    for _slot, tok in rows:
        r = tok.numel()
        caps.append({n: (_rnd(gen, (r, din), din**-0.5, device), _rnd(gen, (r, dout), dout**-0.5, device))
                     for n, din, dout in LAYERS})
    return logits, idx, rows, caps


def test_mixtral_layer_full_width(device):
    from dattri_llm_amd.gradient import ops

    print("mixtral moe layer 16x256 vs 16x256, 8 experts top-2, gate_up 4096->28672, down 14336->4096",
          flush=True)
    gen = torch.Generator(device=device).manual_seed(5)
    sides = [_side(gen, device) for _ in range(2)]
    for logits, idx, _rows, _caps in sides:  # the router is bit-exact against torch.topk
        _tv, ti = torch.topk(torch.softmax(logits.cpu().float(), dim=-1), TOP_K, dim=-1)
        assert torch.equal(idx.cpu(), ti)
    segs = [ops.moe.route_segments(idx, N_EXP, B, T) for _l, idx, _r, _c in sides]
    per_layer = [([(*sides[0][3][e][n], *sides[1][3][e][n]) for e in range(N_EXP)], False) for n, _i, _o in LAYERS]
    got = ops.moe.moe_layers_cross_gram(per_layer, segs[0], segs[1])
    torch.cuda.synchronize()
    want = np.zeros((B, B))
    for e in range(N_EXP):
        tok1, tok2 = (sides[s][2][e][1].cpu().numpy() for s in range(2))
        for n, _i, _o in LAYERS:
            a1, g1 = (x.double().cpu().numpy() for x in sides[0][3][e][n])
            a2, g2 = (x.double().cpu().numpy() for x in sides[1][3][e][n])
            want += oracle.moe_segment_ghost_compact(a1, g1, tok1, a2, g2, tok2, B, B, T, T)
    assert_parity(got, want, torch.bfloat16, label="grouped ghost, full width")


def _zero_filled(rows, caps, device):
    """The reference's capture of routed experts: each expert's routed rows
    scattered back to zero-filled (B, T, d) factors at their own positions
    (hooks/routing.py:71-86), one linear layer per (expert, expert linear)."""
    from dattri_llm_amd.gradient import Factorized, Gradient

    data = {}
    for e, (_slot, tok) in enumerate(rows):
        for n, din, dout in LAYERS:
            a = torch.zeros(B * T, din, dtype=torch.bfloat16, device=device)
            g = torch.zeros(B * T, dout, dtype=torch.bfloat16, device=device)
            a[tok], g[tok] = caps[e][n]
            data[f"experts.{e}.{n}"] = Factorized(a.view(B, T, din), g.view(B, T, dout), module_kwargs={"has_bias": False})
    return Gradient(dict.fromkeys(data, "factorized"), data, dict.fromkeys(data, "nn.Linear"),
                    dict.fromkeys(data, "batch_token"))


def test_zero_filled_experts_take_the_packed_route(device):
    """Dense-with-zeros expert captures through the drop-in ops at the Mixtral
    widths: the gradient-carrying rows are found on the device, every expert
    of both linears runs in ONE grouped launch (no dense ghost launch over the
    zero rows), and the scores equal the oracle's segment sums."""
    from dattri_llm_amd import kernels
    from dattri_llm_amd.gradient import ops

    print("mixtral zero-filled experts through layerwise_cross_dot / cross_gram", flush=True)
    gen = torch.Generator(device=device).manual_seed(6)
    sides = [_side(gen, device) for _ in range(2)]
    train, test = (_zero_filled(sides[s][2], sides[s][3], device) for s in range(2))
    want = np.zeros((B, B))
    one = None
    for e in range(N_EXP):
        tok1, tok2 = (sides[s][2][e][1].cpu().numpy() for s in range(2))
        for n, _i, _o in LAYERS:
            a1, g1 = (x.double().cpu().numpy() for x in sides[0][3][e][n])
            a2, g2 = (x.double().cpu().numpy() for x in sides[1][3][e][n])
            part = oracle.moe_segment_ghost_compact(a1, g1, tok1, a2, g2, tok2, B, B, T, T)
            want += part
            if e == 0 and n == "gate_up":
                one = part
    with kernels.launch_events() as log:
        got = ops.layerwise_cross_dot(train, test, mode="factorized")
    torch.cuda.synchronize()
    assert len(log.get("ghost_gram_grouped", [])) == 1 and "ghost_gram" not in log
    assert_parity(got, want, torch.bfloat16, label="16 zero-filled expert layers")
    f1, f2 = train.data["experts.0.gate_up"], test.data["experts.0.gate_up"]
    single = ops.cross_gram(f1.activation, f1.pre_activation_grad, f2.activation, f2.pre_activation_grad,
                            "nn.Linear", mode="factorized")
    assert_parity(single, one, torch.bfloat16, label="one expert through cross_gram")
