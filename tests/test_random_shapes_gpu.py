"""Seeded random shapes for the main kernels against float64 products of the
same inputs on the device: widths at every 16-byte multiple, ragged token
counts, sliced and k-blocked score operands, narrow dW sides, both norm kinds
and projection widths.  Inputs are exact in their dtype and every kernel
accumulates in fp32, so the bound is a few fp32 roundings of the result's
scale (measured worst: 3.6e-6)."""

from __future__ import annotations

import random

import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = 5e-5
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _vec(dt):
    return 16 // torch.tensor([], dtype=dt).element_size()


def _rnd(device, *shape, dt):
    return torch.randn(*shape, device=device).to(dt)


def _rel(got, ref):
    return float((got.double() - ref).abs().max() / (ref.abs().max() + 1e-30))


def _cases(seed, n=24):
    rng = random.Random(seed)
    return [(rng, rng.choice(DTYPES)) for _ in range(n)]


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_score_gemm_random_layers(device, seed):
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed):
        v = _vec(dt)
        b1, b2 = rng.randint(1, 150), rng.randint(1, 150)
        pairs, info = [], []
        ref = torch.zeros(b1, b2, dtype=torch.float64, device=device)
        for _ in range(rng.randint(1, 4)):
            w = v * rng.randint(1, 2000)
            form = rng.choice(["plain", "slice", "blocked"] if w % 64 == 0 else ["plain", "slice"])
            m1, m2 = _rnd(device, b1, w, dt=dt), _rnd(device, b2, w, dt=dt)
            ref += m1.double() @ m2.double().T
            if form == "slice":
                pad = v * rng.randint(1, 64)
                big1 = torch.zeros(b1, w + pad, dtype=dt, device=device)
                big2 = torch.zeros(b2, w + pad, dtype=dt, device=device)
                big1[:, :w], big2[:, :w] = m1, m2
                m1, m2 = big1[:, :w], big2[:, :w]
            elif form == "blocked":
                x1 = kernels.blocked_storage(b1, w, dt, device)
                x1.copy_(m1.view(b1, -1, 64))
                x2 = kernels.blocked_storage(b2, w, dt, device)
                x2.copy_(m2.view(b2, -1, 64))
                m1, m2 = x1, x2
            pairs.append((m1, m2))
            info.append((w, form))
        print(f"score_gemm seed={seed} {dt} {b1}x{b2} {info}", flush=True)
        assert _rel(kernels.score_gemm(pairs), ref) <= TOL, (dt, b1, b2, info)


@pytest.mark.parametrize("seed", [21, 22, 23])
def test_materialize_random_shapes(device, seed):
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed):
        v = _vec(dt)
        b, t = rng.randint(1, 6), rng.randint(1, 500)
        k = v * (rng.randint(1, 8) if rng.random() < 0.25 else rng.randint(1, 120))
        d = v * rng.randint(1, 120)
        bias = rng.random() < 0.3
        a, g = _rnd(device, b, t, k, dt=dt), _rnd(device, b, t, d, dt=dt)
        print(f"materialize seed={seed} {dt} B={b} T={t} K={k} D={d} bias={bias}", flush=True)
        got = kernels.materialize_linear(a, g, bias=bias, out_dtype=torch.float32).reshape(b, -1)
        a64 = a.double()
        if bias:
            a64 = torch.cat([a64, torch.ones(b, t, 1, dtype=torch.float64, device=device)], -1)
        ref = torch.bmm(g.double().transpose(1, 2).contiguous(), a64).reshape(b, -1)
        assert _rel(got, ref) <= TOL, (dt, b, t, k, d, bias)


@pytest.mark.parametrize("seed", [31, 32, 33])
def test_ghost_gram_random_shapes(device, seed):
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed):
        v = _vec(dt)
        b1, b2, s1, s2 = rng.randint(1, 10), rng.randint(1, 10), rng.randint(1, 300), rng.randint(1, 300)
        k, d = v * rng.randint(1, 64), v * rng.randint(1, 64)
        bias = rng.random() < 0.3
        a1, g1 = _rnd(device, b1, s1, k, dt=dt), _rnd(device, b1, s1, d, dt=dt)
        a2, g2 = _rnd(device, b2, s2, k, dt=dt), _rnd(device, b2, s2, d, dt=dt)
        print(f"ghost seed={seed} {dt} {b1}x{b2} S={s1}/{s2} K={k} D={d} bias={bias}", flush=True)

        def dw(a, g):
            a = a.double()
            if bias:
                a = torch.cat([a, torch.ones(*a.shape[:2], 1, dtype=torch.float64, device=device)], -1)
            return torch.bmm(g.double().transpose(1, 2).contiguous(), a).reshape(a.shape[0], -1)

        ref = dw(a1, g1) @ dw(a2, g2).T
        assert _rel(kernels.ghost_gram(a1, g1, a2, g2, bias=bias), ref) <= TOL, (dt, b1, b2, s1, s2, k, d)


@pytest.mark.parametrize("seed", [41, 42, 43])
def test_norm_weight_grad_random_shapes(device, seed):
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed):
        v = _vec(dt)
        b, t, d = rng.randint(1, 8), rng.randint(1, 900), v * rng.randint(1, 600)
        kind, eps = rng.choice([0, 1]), rng.choice([1e-5, 1e-6])
        bias = kind == 1 and rng.random() < 0.5
        x, g = _rnd(device, b, t, d, dt=dt), _rnd(device, b, t, d, dt=dt)
        print(f"norm seed={seed} {dt} B={b} T={t} d={d} kind={kind} bias={bias}", flush=True)
        got = kernels.norm_weight_grad(x, g, kind=kind, eps=eps, bias=bias, out_dtype=torch.float32)
        x64, g64 = x.double(), g.double()
        if kind == 0:
            xh = x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + eps)
        else:
            mu = x64.mean(-1, keepdim=True)
            xh = (x64 - mu) / torch.sqrt(((x64 - mu) ** 2).mean(-1, keepdim=True) + eps)
        ref = (xh * g64).sum(1)
        if bias:
            ref = torch.cat([ref, g64.sum(1)], -1)
        assert _rel(got, ref) <= TOL, (dt, b, t, d, kind, eps, bias)


@pytest.mark.parametrize("seed", [51, 52, 53])
def test_project_outer_random_shapes(device, seed):
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed):
        v = _vec(dt)
        b, t = rng.randint(1, 40), rng.randint(1, 400)
        k, d = v * rng.randint(1, 400), v * rng.randint(1, 400)
        ka, kg = rng.choice([8, 16, 32, 64]), rng.choice([8, 16, 32, 64])
        a, g = _rnd(device, b, t, k, dt=dt), _rnd(device, b, t, d, dt=dt)
        pin, pout = _rnd(device, ka, k, dt=dt), _rnd(device, kg, d, dt=dt)
        print(f"project seed={seed} {dt} B={b} T={t} K={k} D={d} ka={ka} kg={kg}", flush=True)
        got = kernels.project_outer(a, g, pin, pout, out_dtype=torch.float32).reshape(b, -1)
        ap, gp = a.double() @ pin.double().T, g.double() @ pout.double().T
        ref = torch.bmm(gp.transpose(1, 2).contiguous(), ap).reshape(b, -1)
        assert _rel(got, ref) <= TOL, (dt, b, t, k, d, ka, kg)


@pytest.mark.parametrize("seed", [61, 62, 63])
def test_ghost_per_token_random_shapes(device, seed):
    """K[i, t, j] = sum_s (a1_it . a2_js + bias)(g1_it . g2_js), widths at any
    element count (the wrapper pads rows to whole 16-byte chunks)."""
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed, 12):
        b1, b2, t1, t2 = rng.randint(1, 6), rng.randint(1, 6), rng.randint(1, 300), rng.randint(1, 300)
        k, d = rng.randint(1, 300), rng.randint(1, 300)
        bias = rng.random() < 0.3
        a1, g1 = _rnd(device, b1, t1, k, dt=dt), _rnd(device, b1, t1, d, dt=dt)
        a2, g2 = _rnd(device, b2, t2, k, dt=dt), _rnd(device, b2, t2, d, dt=dt)
        print(f"per-token seed={seed} {dt} {b1}x{b2} T={t1}/{t2} K={k} D={d} bias={bias}", flush=True)
        got = kernels.ghost_gram_per_token(a1, g1, a2, g2, bias=bias)
        ka = a1.double().reshape(b1 * t1, k) @ a2.double().reshape(b2 * t2, k).T
        kg = g1.double().reshape(b1 * t1, d) @ g2.double().reshape(b2 * t2, d).T
        ref = ((ka + float(bias)) * kg).reshape(b1, t1, b2, t2).sum(-1)
        assert got.shape == (b1, t1, b2)
        assert _rel(got, ref) <= TOL, (dt, b1, b2, t1, t2, k, d, bias)


def _segments(rng, device, batch, rows):
    """Random non-decreasing per-sample offsets over at most ``rows`` packed
    rows (int32, B+1 entries) and, half the time, a random row index into
    ``rows`` physical rows."""
    cuts = sorted(rng.randint(0, rows) for _ in range(batch - 1))
    end = rng.randint(cuts[-1] if cuts else 0, rows)
    seg = torch.tensor([0, *cuts, end], dtype=torch.int32, device=device)
    idx = None
    if rng.random() < 0.5:
        idx = torch.tensor(rng.sample(range(rows), rows), dtype=torch.int32, device=device)
    return seg, idx


@pytest.mark.parametrize("seed", [71, 72, 73])
def test_grouped_ghost_random_segments(device, seed):
    """Segment-summed ghost products over groups of different widths (the
    experts of several routed layers), ragged and empty samples, with and
    without a row index."""
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed, 6):
        v = _vec(dt)
        b1, b2 = rng.randint(1, 12), rng.randint(1, 12)
        bias = rng.random() < 0.3
        groups1, groups2, info = [], [], []
        ref = torch.zeros(b1, b2, dtype=torch.float64, device=device)
        for _ in range(rng.randint(1, 6)):
            k, d = v * rng.randint(1, 40), v * rng.randint(1, 40)
            sides = []
            for b in (b1, b2):
                rows = rng.randint(1, 400)
                a, g = _rnd(device, rows, k, dt=dt), _rnd(device, rows, d, dt=dt)
                seg, idx = _segments(rng, device, b, rows)
                sides.append((a, g, seg, idx))
            dws = []
            for a, g, seg, idx in sides:
                s = seg.tolist()
                order = idx.long() if idx is not None else torch.arange(a.shape[0], device=device)
                per = []
                for i in range(len(s) - 1):
                    r = order[s[i]:s[i + 1]]
                    ar = a[r].double()
                    if bias:
                        ar = torch.cat([ar, torch.ones(ar.shape[0], 1, dtype=torch.float64, device=device)], -1)
                    per.append((g[r].double().T @ ar).reshape(-1))
                dws.append(torch.stack(per))
            ref += dws[0] @ dws[1].T
            groups1.append(sides[0])
            groups2.append(sides[1])
            info.append((k, d))
        print(f"grouped seed={seed} {dt} {b1}x{b2} groups {info} bias={bias}", flush=True)
        got = kernels.ghost_gram_grouped(groups1, groups2, bias=bias)
        assert _rel(got, ref) <= TOL, (dt, b1, b2, info, bias)


@pytest.mark.parametrize("seed", [81, 82, 83])
def test_route_segments_random_routings(device, seed):
    """da_moe_route's per-expert segments against a torch CPU restatement of
    the reference's enumeration: expert e's routed rows in slot-major, token
    ascending order (torch.where over the one-hot mask permuted to (E, k, N)),
    then grouped by sample, stably; random top-k sets over 1-256 experts."""
    from dattri_llm_amd.gradient import ops

    rng = random.Random(seed)
    for _ in range(10):
        n_exp = rng.choice([1, 2, 5, 8, 16, 60, 128, 256])
        k = rng.randint(1, min(8, n_exp))
        batch, tokens = rng.randint(1, min(64, 8192 // n_exp)), rng.randint(1, 128)  # E * B <= 8192 bins
        n = batch * tokens
        gen = torch.Generator().manual_seed(rng.randrange(1 << 30))
        idx = torch.rand(n, n_exp, generator=gen).argsort(-1)[:, :k].contiguous()  # k distinct experts per token
        print(f"route seed={seed} E={n_exp} k={k} B={batch} T={tokens}", flush=True)
        got = ops.moe.route_segments(idx.to(device), n_exp, batch, tokens)
        assert len(got) == n_exp
        tok_all = torch.arange(n).unsqueeze(1).expand(n, k)
        slot_all = torch.arange(k).unsqueeze(0).expand(n, k)
        for e in range(n_exp):
            hit = idx == e
            p = (slot_all[hit] * n + tok_all[hit]).sort().values  # slot-major, token ascending
            sample = (p % n) // tokens
            seg = torch.zeros(batch + 1, dtype=torch.int64)
            seg[1:] = torch.bincount(sample, minlength=batch).cumsum(0)
            rows = torch.sort(sample, stable=True).indices
            seg_g, rows_g = got[e]
            assert torch.equal(seg_g.cpu().to(torch.int64), seg), (e, n_exp, k, batch, tokens)
            assert torch.equal(rows_g.cpu().to(torch.int64), rows), (e, n_exp, k, batch, tokens)


@pytest.mark.parametrize("seed", [91, 92])
def test_row_dots_random_layers(device, seed):
    """Per-row squared norms and dots summed over layers (row-major, sliced and
    k-blocked layers mixed)."""
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed, 12):
        v = _vec(dt)
        b = rng.randint(1, 96)
        layers, ref, info = [], torch.zeros(b, dtype=torch.float64, device=device), []
        for _ in range(rng.randint(1, 5)):
            w = v * rng.randint(1, 3000)
            m1 = _rnd(device, b, w, dt=dt)
            m2 = _rnd(device, b, w, dt=dt) if rng.random() < 0.5 else None
            ref += (m1.double() * (m2 if m2 is not None else m1).double()).sum(-1)
            if w % 64 == 0 and rng.random() < 0.4:
                x = kernels.blocked_storage(b, w, dt, device)
                x.copy_(m1.view(b, -1, 64))
                m1 = x
                if m2 is not None:
                    y = kernels.blocked_storage(b, w, dt, device)
                    y.copy_(m2.view(b, -1, 64))
                    m2 = y
            layers.append((m1, m2))
            info.append((w, m2 is None))
        print(f"row_dots seed={seed} {dt} B={b} {info}", flush=True)
        assert _rel(kernels.row_dots(layers), ref) <= TOL, (dt, b, info)


@pytest.mark.parametrize("seed", [101, 102])
def test_embedding_cross_gram_random_ids(device, seed):
    """sum over (t, s) with tok1[i,t] == tok2[j,s] of g1[i,t] . g2[j,s], ids
    drawn from small and large vocabularies (many and few matches), with
    negative (padding) ids that match nothing."""
    from dattri_llm_amd import kernels

    for rng, dt in _cases(seed, 8):
        b1, b2, t1, t2 = rng.randint(1, 8), rng.randint(1, 8), rng.randint(1, 200), rng.randint(1, 200)
        vocab, d = rng.choice([5, 50, 1000, 128256]), _vec(dt) * rng.randint(1, 100)
        gen = torch.Generator().manual_seed(rng.randrange(1 << 30))
        tok1 = torch.randint(-1, vocab, (b1, t1), generator=gen)
        tok2 = torch.randint(-1, vocab, (b2, t2), generator=gen)
        g1, g2 = _rnd(device, b1, t1, d, dt=dt), _rnd(device, b2, t2, d, dt=dt)
        print(f"embedding seed={seed} {dt} {b1}x{b2} T={t1}/{t2} V={vocab} d={d}", flush=True)
        got = kernels.embedding_cross_gram(tok1.to(device), g1, tok2.to(device), g2)
        match = (tok1.reshape(-1, 1) == tok2.reshape(1, -1)) & (tok1.reshape(-1, 1) >= 0)
        dots = g1.double().reshape(b1 * t1, d) @ g2.double().reshape(b2 * t2, d).T
        ref = (dots * match.to(device)).reshape(b1, t1, b2, t2).sum((1, 3))
        assert _rel(got, ref) <= TOL, (dt, b1, b2, t1, t2, vocab, d)
