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
