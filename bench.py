#!/usr/bin/env python
"""Pair-score throughput of the gradient-scoring path on one MI355X.

Default workload (the headline metric): a Llama-3-8B-shaped decoder block
(d 4096, 32 q / 8 kv heads -> q/k/v/o 4096->4096/1024/1024/4096, SwiGLU FFN
14336, two RMSNorm(4096)), bf16, with the factors its 7 linears and 2 norms
capture for 8 train sequences x 2048 tokens and 64 query sequences x 512
tokens.  A step is one train block through the drop-in scoring path, as
dattri-llm's attribute loop runs it: TracInAttributor.attribute_sources ->
score_sources -> inner_product -> ops.layerwise_cross_dot.  The reference's
cost rule routes every layer of this block to the materialized form, so the
kernels a step launches are

    RMSNorm per-sample weight grads  (norm kernel, x2)
    per-sample dW of the 7 linears   (materialize kernel, x7)
    a share of one multi-layer score GEMM (score kernel: 9 layers; sixteen
    train blocks share one pass over the queries, 128 x 64 per launch)

and the block's (8, 64) scores are copied to pinned host memory.  Inputs are
synthetic (seeded on the device) and already resident in HBM; the query block
is routed to dense once (route_test_rep), before the timed region, and
reported as ``query_prep_ms``.  The same step issued as raw kernel calls is
timed beside it (``kernels_only_ms``, ``boundary_overhead``).

Prints ONE JSON line.  Other workloads (not the headline):
``--workload ghost``   the fused ghost cross-gram, 256 train x 64 query, T=512, d 4096;
``--workload per_token`` the per-token cross-gram on the same shapes, (256, 512, 64) out;
``--workload project`` projected (k=64) capture of the Llama-7B MLP, 512 + 128 samples;
``--workload moe``     a Mixtral-shaped MoE layer on the segmented ghost route;
``--workload kfac``    the K-FAC covariance fit of the Llama-8B block's 7 linears over one train block;
``--workload capture`` the LoGRA capture fused into autograd on a Llama-7B MLP (128 x 128 tokens);
``--workload store``   attribute from an on-disk (memmap) gradient store through pinned H2D;
``--workload copy``    a 2 GiB device copy, the reference point for byte counters.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "dattri-llm_amd"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "train×query pair-scores/sec (Llama-8B-shaped block, bf16); MFMA util % of peak"
PEAK_BF16_TFLOPS = 2500.0
# C4: train blocks scored per pass over the dense query block (score_sources' train_blocks_per_pass).
# The 64 query rows are read once per 16 blocks: 128 train rows, two 64 x 64 tiles of the score ring
# whose workgroups stream the query rows in step on the same XCDs. Score per block: 0.76-0.79 ms
# against 1.01-1.10 with 8 blocks per pass (+3-5% pair-scores/s on the same box). 24 blocks need
# more dense rows than the default cache budget holds beside the queries.
PASS = 16
PEAK_HBM_GBS = 8000.0

D_MODEL, D_KV, D_FFN = 4096, 1024, 14336
# (layer, activation factor, d_in, d_out)
LINEARS = [
    ("q_proj", "attn_in", D_MODEL, D_MODEL),
    ("k_proj", "attn_in", D_MODEL, D_KV),
    ("v_proj", "attn_in", D_MODEL, D_KV),
    ("o_proj", "o_in", D_MODEL, D_MODEL),
    ("gate_proj", "mlp_in", D_MODEL, D_FFN),
    ("up_proj", "mlp_in", D_MODEL, D_FFN),
    ("down_proj", "down_in", D_FFN, D_MODEL),
]
NORMS = [("input_layernorm", D_MODEL), ("post_attention_layernorm", D_MODEL)]
ACT_WIDTH = {"attn_in": D_MODEL, "o_in": D_MODEL, "mlp_in": D_MODEL, "down_in": D_FFN}
RMS_EPS = 1e-5


def _randn(shape, gen, dtype, scale=1.0):
    import torch

    x = torch.empty(shape, dtype=torch.float32, device="cuda")
    x.normal_(0.0, scale, generator=gen)
    return x.to(dtype)


def make_block(batch: int, tokens: int, seed: int):
    """Synthetic captures of one block: shared activation factors per input,
    one output-gradient factor per layer, norm inputs and gradients."""
    import torch

    gen = torch.Generator(device="cuda").manual_seed(seed)
    bf = torch.bfloat16
    acts = {k: _randn((batch, tokens, w), gen, bf) for k, w in ACT_WIDTH.items()}
    grads = {n: _randn((batch, tokens, dout), gen, bf, dout**-0.5) for n, _a, _i, dout in LINEARS}
    norms = {n: (_randn((batch, tokens, d), gen, bf), _randn((batch, tokens, d), gen, bf, d**-0.5))
             for n, d in NORMS}
    return acts, grads, norms


def dense_block(acts, grads, norms, timers=None):
    """Per-sample dense gradients of every layer (the materialized route)."""
    import torch

    from dattri_llm_amd import kernels

    out = {}
    for name, d in NORMS:
        x, g = norms[name]
        ev = _ev(timers, "norm_weight_grad")
        out[name] = kernels.norm_weight_grad(x, g, kind=0, eps=RMS_EPS, out_dtype=torch.bfloat16)
        _ev_end(ev)
    for name, act, _din, _dout in LINEARS:
        ev = _ev(timers, f"materialize:{name}")
        out[name] = kernels.materialize_linear(acts[act], grads[name], blocked=True)
        _ev_end(ev)
    return out


def dense_group(blocks):
    """``dense_block`` of several train blocks (``(acts, grads, norms)`` each)
    stacked along the batch: each linear layer's blocks written into row
    slices of one k-blocked buffer (the layout one score pass reads for all of
    them)."""
    import torch

    from dattri_llm_amd import kernels

    out = {}
    for name, _d in NORMS:
        out[name] = torch.cat([kernels.norm_weight_grad(*norms[name], kind=0, eps=RMS_EPS, out_dtype=torch.bfloat16)
                               for _a, _g, norms in blocks])
    for name, act, din, dout in LINEARS:
        b = blocks[0][0][act].shape[0]
        buf = kernels.blocked_storage(len(blocks) * b, din * dout, torch.bfloat16, blocks[0][0][act].device)
        for i, (acts, grads, _n) in enumerate(blocks):
            kernels.materialize_linear(acts[act], grads[name], blocked=True, out=buf[i * b:(i + 1) * b])
        out[name] = buf
    return out


def _ev(timers, key):
    if timers is None:
        return None
    import torch

    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    timers.setdefault(key, []).append((s, e))
    return e


def _ev_end(e):
    if e is not None:
        e.record()


def _mean_ms(timers, key):
    pairs = timers.get(key, [])
    return sum(s.elapsed_time(e) for s, e in pairs) / max(len(pairs), 1)


TRAFFIC_PROFILE = os.path.join(REPO, "profiles", "llama8b_block_hbm_traffic.md")
GHOST_TRAFFIC = os.path.join(REPO, "profiles", "ghost_c2_hbm_traffic.md")
PROJECT_TRAFFIC = os.path.join(REPO, "profiles", "project_llama7b_mlp_hbm_traffic.md")
MOE_TRAFFIC = os.path.join(REPO, "profiles", "moe_mixtral_layer_hbm_traffic.md")
KFAC_TRAFFIC = os.path.join(REPO, "profiles", "kfac_llama8b_block_hbm_traffic.md")
CAPTURE_TRAFFIC = os.path.join(REPO, "profiles", "capture_llama7b_mlp_hbm_traffic.md")
STORE_TRAFFIC = os.path.join(REPO, "profiles", "store_attribute_hbm_traffic.md")


def profiled_traffic(kernel: str, path: str = TRAFFIC_PROFILE):
    """HBM bytes per launch of ``kernel`` from the committed counter summary
    (FETCH_SIZE / WRITE_SIZE runs scaled by the copy calibration), or None."""
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_per_launch" and parts[1] == kernel:
                    return float(parts[2])
    except OSError:
        pass
    return None


def vendor_gemm_ref(seconds: float = 1.0):
    """Sustained throughput of the vendor library's square bf16 GEMM
    (torch.matmul -> hipBLASLt, 8192^3) on this GPU, run after the timed region.
    Under dense bf16 MFMA load on random data the chip lowers its clock to stay
    within its power limit, so this is the attainable MFMA reference that an
    MFMA-bound kernel's fraction of the spec-sheet peak should be read against."""
    import torch

    n = 8192
    gen = torch.Generator(device="cuda").manual_seed(7)
    a = _randn((n, n), gen, torch.bfloat16)
    b = _randn((n, n), gen, torch.bfloat16)
    c = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
    for _ in range(10):
        torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    reps = max(10, int(seconds / max((time.perf_counter() - t0) / 10, 1e-6)))
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        torch.matmul(a, b, out=c)
    e.record()
    torch.cuda.synchronize()
    tf = 2.0 * n**3 * reps / (s.elapsed_time(e) * 1e9)
    del a, b, c
    return {"ref": f"torch.matmul bf16 {n}x{n}x{n} (hipBLASLt), sustained {reps} launches",
            "tflops": round(tf, 1), "frac_of_peak": round(tf / PEAK_BF16_TFLOPS, 4)}


def cpu_info():
    cores = len(os.sched_getaffinity(0))
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, model


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        info = [p for p in threadpool_info() if p.get("user_api") == "blas"]
        if info:
            return int(info[0]["num_threads"])
    except Exception:  # noqa: BLE001
        pass
    return int(os.environ.get("OMP_NUM_THREADS", "1"))


# ---------------------------------------------------------------------------
# Llama block (headline)
# ---------------------------------------------------------------------------


def block_gradient(acts, grads, norms):
    """The block's captures as the reference's hooks hold them: a Gradient of
    raw factorized layers (module kwargs kept, preprocessing left to the ops)."""
    from dattri_llm_amd.gradient import Factorized, Gradient

    data, types = {}, {}
    for name, act, _din, _dout in LINEARS:
        data[name] = Factorized(acts[act], grads[name], module_kwargs={"has_bias": False})
        types[name] = "nn.Linear"
    for name, d in NORMS:
        x, g = norms[name]
        data[name] = Factorized(x, g, module_kwargs={"has_bias": False, "eps": RMS_EPS, "normalized_shape": (d,)})
        types[name] = "nn.RMSNorm"
    return Gradient(dict.fromkeys(data, "factorized"), data, types, dict.fromkeys(data, "batch_token"))


def bench_block(args):
    """One step = one train block through the drop-in scoring path, as the
    reference's attribute loop runs it: TracInAttributor.attribute_sources over
    a source of train blocks (score_sources -> inner_product ->
    ops.layerwise_cross_dot, the cost rule routing every layer, the block's
    scores copied to pinned host memory).  The query block is routed once
    (route_test_rep), before the timed region.  The same step issued as raw
    kernel calls is timed beside it (kernels_only_ms)."""
    import torch

    from dattri_llm_amd import kernels
    from dattri_llm_amd.attribution import TracInAttributor

    n_train, t_train, n_query, t_query = 8, 2048, 64, 512
    # PASS distinct train blocks, cycled: the blocks of one group are
    # different tensors, as a real source's are
    train_facs = [make_block(n_train, t_train, seed=10 + i) for i in range(PASS)]
    query_fac = make_block(n_query, t_query, seed=1)
    trains = [block_gradient(*fac) for fac in train_facs]
    attr = TracInAttributor(train_batch_size=n_train, device="cuda")
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    routed = attr.route_test_rep(block_gradient(*query_fac))
    torch.cuda.synchronize()
    query_prep_ms = (time.perf_counter() - t0) * 1e3
    routes = {n: ("dense" if isinstance(v, torch.Tensor) else "factorized") for n, v in routed.data.items()}
    train_ids = [f"train{i}" for i in range(n_train)]
    test_source = [(0, routed, [f"query{j}" for j in range(n_query)])]

    def attribute(k, per_pass=PASS):
        return attr.attribute_sources(((step, trains[step % PASS], train_ids) for step in range(k)), test_source,
                                      train_blocks_per_pass=per_pass)

    # Setup: reserve one full group's dense buffers in the caching allocator (allocated and
    # released here), so that no multi-GB device allocation falls inside a timed region, whatever
    # the warmup's group size (a 5-step warmup builds a group of 5).
    reserve = [kernels.blocked_storage(PASS * n_train, din * dout, torch.bfloat16, "cuda")
               for _n, _a, din, dout in LINEARS]
    del reserve
    attribute(args.warmup)
    torch.cuda.synchronize()
    with kernels.launch_events() as log:
        t0 = time.perf_counter()
        score = attribute(args.steps)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
    assert score.scores.shape == (n_train * args.steps, n_query)
    # the same steps with the reference's schedule, one query pass per train block
    attribute(args.warmup, per_pass=1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    attribute(args.steps, per_pass=1)
    torch.cuda.synchronize()
    ms_one = (time.perf_counter() - t0) * 1e3 / args.steps

    def event_ms(name):
        launches = log.get(name, [])
        return sum(s.elapsed_time(e) for s, e in launches) / args.steps, round(len(launches) / args.steps, 4)

    # The same steps as raw kernel calls (no boundary), grouped alike: per group of
    # PASS train blocks, dW of the 7 linears and 2 norm grads per block, one score GEMM.
    q_dense = {n: routed.data[n] for n in routed.data}
    raw_scores = torch.empty(PASS * n_train, n_query, dtype=torch.float32, device="cuda")

    names = list(trains[0].data)  # the order layerwise_cross_dot sums the layers in

    def raw_steps(k):
        for first in range(0, k, PASS):
            nb = min(PASS, k - first)
            tr = dense_group([train_facs[(first + i) % PASS] for i in range(nb)])
            kernels.score_gemm([(tr[n], q_dense[n]) for n in names], out=raw_scores[:nb * n_train])
            del tr  # before the next group is built, as score_sources does
        return nb

    raw_steps(args.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    last = raw_steps(args.steps)
    torch.cuda.synchronize()
    raw_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # the drop-in scores are the raw ones rounded to the compute dtype (bf16); compare the last group
    rows = last * n_train
    same = bool(torch.equal(score.scores[-rows:], raw_scores[:rows].to(torch.bfloat16).float().cpu()))

    # Algorithmic work.
    dk = {n: din * dout for n, _a, din, dout in LINEARS}
    width = sum(dk.values()) + sum(d for _, d in NORMS)
    mat_flops = sum(2.0 * n_train * t_train * v for v in dk.values())
    # one score launch reads a group's train blocks (PASS, the last group of the timed steps
    # possibly fewer) and the queries once
    score_bytes_launch = (PASS * n_train + n_query) * width * 2.0
    groups = [min(PASS, args.steps - f) for f in range(0, args.steps, PASS)]
    score_bytes = sum((nb * n_train + n_query) * width * 2.0 for nb in groups) / args.steps  # per step
    norm_bytes = 2.0 * n_train * t_train * D_MODEL * 2
    t_mat, n_mat = event_ms("materialize_linear")
    t_score, n_score = event_ms("score_gemm")
    t_norm, n_norm = event_ms("norm_weight_grad")
    kern = {
        "materialize_linear": {"ms_per_step": round(t_mat, 4), "launches_per_step": n_mat,
                               "tflops": round(mat_flops / t_mat / 1e9, 1)},
        "score_gemm": {"ms_per_step": round(t_score, 4), "launches_per_step": n_score,
                       "gbs": round(score_bytes / t_score / 1e6, 1)},
        "norm_weight_grad": {"ms_per_step": round(t_norm, 4), "launches_per_step": n_norm,
                             "gbs": round(2 * norm_bytes / t_norm / 1e6, 1)},
    }
    dw_mfma_util = mat_flops / (t_mat * 1e9) / PEAK_BF16_TFLOPS
    # the whole step's matrix work (dW of the 7 linears and the score GEMM)
    # over the step's wall time: the MFMA utilisation of the step
    step_flops = mat_flops + 2.0 * n_train * n_query * width
    step_mfma_util = step_flops / (ms * 1e9) / PEAK_BF16_TFLOPS

    # Dominant kernel: the one taking most of the step (summed over its launches).
    # Its roofline is the step's algorithmic work over the summed event time,
    # i.e. per-launch work over the average launch duration.
    totals = {"materialize_tiles_tr8": t_mat, "score_ring64": t_score, "norm_grad_ring": t_norm}
    big = max(totals, key=totals.get)
    if big == "score_ring64":
        gbs = score_bytes / t_score / 1e6
        roof = {"bound": "hbm", "kernel": big, "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                "work_per_launch": f"{score_bytes_launch:.4g} B ({PASS * n_train + n_query} rows x {width} weights x 2 B)",
                "launches_per_step": n_score}
    elif big == "materialize_tiles_tr8":
        tf = mat_flops / (t_mat * 1e9)
        roof = {"bound": "mfma", "kernel": big, "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None,
                "work_per_launch": f"{mat_flops / max(n_mat, 1):.4g} flop average over the 7 linears "
                                   "(2 x 8 samples x 2048 tokens x d_in x d_out each)",
                "launches_per_step": n_mat}
    else:
        gbs = 2 * norm_bytes / t_norm / 1e6
        roof = {"bound": "hbm", "kernel": big, "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "launches_per_step": n_norm}
    roof["step_share"] = round(totals[big] / ms, 3)
    roof["traffic"] = profiled_traffic(big)
    if roof["traffic"] is not None:
        roof["traffic_source"] = os.path.relpath(TRAFFIC_PROFILE, REPO)

    pairs = n_train * n_query
    result = {
        "metric": METRIC,
        "value": round(pairs / (ms / 1e3), 1),
        "unit": "pair-scores/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b-block: 8 train x 2048 tok vs 64 query x 512 tok, 7 linears + 2 RMSNorm, "
                        "TracInAttributor.attribute_sources (cost-rule routing per layer; 16 train blocks "
                        "per pass over the dense queries)",
            "train_block": [n_train, t_train],
            "train_blocks_per_query_pass": PASS,
            "query_block": [n_query, t_query],
            "score_width_per_sample": width,
            "routes": routes,
        },
        "mfma_util": round(step_mfma_util, 4),
        "mfma_util_basis": f"{step_flops:.4g} flop per step (dW + score GEMM) / step time / 2.5 PF/s bf16 peak",
        "dw_mfma_util": round(dw_mfma_util, 4),
        "one_block_per_pass": {"value": round(n_train * n_query / (ms_one / 1e3), 1), "ms_per_step": round(ms_one, 4),
                               "schedule": "train_blocks_per_pass=1 (the reference's loop: one query pass per "
                                           "train block)"},
        "query_prep_ms": round(query_prep_ms, 2),
        "kernels_only_ms": round(raw_ms, 4),
        "boundary_overhead": round(ms / raw_ms - 1.0, 4),
        "dropin_equals_kernels": same,
        "roofline": roof,
        "kernels": kern,
    }
    if args.cpu_baseline:
        last = train_facs[(args.steps - 1) % PASS]
        result["cpu_baseline"], result["parity"] = cpu_baseline_block(last, query_fac, score.scores[-n_train:])
    return result


def cpu_baseline_block(train_fac, query_fac, gpu_scores):
    """The oracle (numpy fp32) on a bounded sample of the same step, from the
    same bf16 inputs: the whole 8-sample train block (T=2048, all 9 layers)
    materialized and scored, one GEMM per layer like the reference's loop,
    against the first 16 of the 64 queries; the score part is scaled to 64
    queries (it streams the query matrix, so its time is linear in the query
    count).  The same sample gives the parity of the bench's own scores."""
    import numpy as np

    import oracle

    nq = 16

    def host(fac, rows=None):
        acts, grads, norms = fac
        sel = (lambda x: x) if rows is None else (lambda x: x[:rows])
        return ({k: sel(v).float().cpu().numpy() for k, v in acts.items()},
                {k: sel(v).float().cpu().numpy() for k, v in grads.items()},
                {k: (sel(x).float().cpu().numpy(), sel(g).float().cpu().numpy()) for k, (x, g) in norms.items()})

    def dense(acts, grads, norms):
        out = {}
        for n, _d in NORMS:
            out[n] = oracle.norm_weight_grad(norms[n][0], norms[n][1], "nn.RMSNorm", RMS_EPS)
        for n, a, _i, _o in LINEARS:
            out[n] = oracle.materialize_linear(acts[a], grads[n])
        return out

    q_dense = dense(*host(query_fac, nq))
    tr = host(train_fac)
    names = list(q_dense)
    n_train_total = tr[0]["attn_in"].shape[0]
    n_query_total = query_fac[0]["attn_in"].shape[0]
    best_mat = best_score = float("inf")
    want = None
    for _ in range(2):
        t0 = time.perf_counter()
        tr_dense = dense(*tr)
        best_mat = min(best_mat, time.perf_counter() - t0)
        t0 = time.perf_counter()
        want = oracle.score_gemm([tr_dense[n] for n in names], [q_dense[n] for n in names])
        best_score = min(best_score, time.perf_counter() - t0)
        del tr_dense
    step_s = best_mat + (n_query_total / nq) * best_score
    cores, model = cpu_info()
    got = gpu_scores[:, :nq].double().numpy()
    err = float(np.abs(got - want).max() / np.abs(want).max())
    baseline = {
        "value": round(n_train_total * n_query_total / step_s, 3),
        "unit": "pair-scores/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": f"numpy fp32 oracle on the bench's own bf16 inputs: the 8-sample train block (T=2048, "
                  f"7 linears + 2 RMSNorm) materialized ({best_mat:.2f} s) and scored vs 16 dense queries "
                  f"({best_score:.2f} s), best of 2; score time scaled x{n_query_total // nq} to 64 queries -> "
                  f"step {step_s:.2f} s; host {model}, {cores} cores visible",
    }
    parity = {"normwise_rel_err": err, "bar": 1e-2, "ok": err <= 1e-2,
              "sample": f"the last timed step's 8 x {nq} scores (bf16 results) against the fp32 oracle"}
    return baseline, parity


# ---------------------------------------------------------------------------
# ghost cross-gram (factorized route)
# ---------------------------------------------------------------------------


def bench_ghost(args):
    import torch

    from dattri_llm_amd import kernels

    n1, n2, t, d = 256, 64, 512, 4096
    gen = torch.Generator(device="cuda").manual_seed(0)
    bf = torch.bfloat16
    a1 = _randn((n1, t, d), gen, bf, d**-0.5)
    g1 = _randn((n1, t, d), gen, bf, d**-0.5)
    a2 = _randn((n2, t, d), gen, bf, d**-0.5)
    g2 = _randn((n2, t, d), gen, bf, d**-0.5)
    out = torch.empty(n1, n2, dtype=torch.float32, device="cuda")
    for _ in range(args.warmup):
        kernels.ghost_gram(a1, g1, a2, g2, out=out)
    torch.cuda.synchronize()
    timers: dict = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ev = _ev(timers, "ghost")
        kernels.ghost_gram(a1, g1, a2, g2, out=out)
        _ev_end(ev)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    flops = 2.0 * n1 * n2 * t * t * (d + d)
    t_k = _mean_ms(timers, "ghost")
    tflops = flops / t_k / 1e9
    result = {
        "metric": "ghost cross-gram pair-scores/sec (256x64 pairs, T=512, d=4096, bf16)",
        "value": round(n1 * n2 / (ms / 1e3), 1),
        "unit": "pair-scores/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "ghost cross-gram 256 train x 64 query, T=512, d_in=d_out=4096"},
        "roofline": {"bound": "mfma", "kernel": "ghost_gram_tiles_v3", "achieved": round(tflops, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic("ghost_gram_tiles_v3", GHOST_TRAFFIC),
                     "traffic_source": os.path.relpath(GHOST_TRAFFIC, REPO),
                     "work_per_launch": f"{flops:.4g} flop = 2 x 256 x 64 pairs x 512^2 x (4096 + 4096)"},
    }
    if args.cpu_baseline:
        import numpy as np

        import oracle

        rng = np.random.default_rng(0)
        s = [rng.standard_normal((n, t, d), dtype=np.float32) for n in (8, 8, 4, 4)]
        t0 = time.perf_counter()
        oracle.cross_gram_factorized(s[0], s[1], s[2], s[3])
        dt = time.perf_counter() - t0
        cores, model = cpu_info()
        result["cpu_baseline"] = {"value": round(32 / dt, 3), "unit": "pair-scores/s",
                                  "cores": blas_threads(), "kind": "port",
                                  "sample": f"numpy fp32 oracle, 8 train x 4 query at T=512, d=4096 "
                                            f"({dt:.2f} s); host {model}, {cores} cores visible"}
    return result


def bench_per_token(args):
    """Per-token cross-gram on the C2 shapes: every train token position of 256
    samples x 512 tokens against 64 whole query samples (T=512, d=4096): the
    ghost flops with a per-row epilogue, (256, 512, 64) fp32 out."""
    import torch

    from dattri_llm_amd import kernels

    n1, n2, t, d = 256, 64, 512, 4096
    gen = torch.Generator(device="cuda").manual_seed(0)
    bf = torch.bfloat16
    a1, g1 = _randn((n1, t, d), gen, bf, d**-0.5), _randn((n1, t, d), gen, bf, d**-0.5)
    a2, g2 = _randn((n2, t, d), gen, bf, d**-0.5), _randn((n2, t, d), gen, bf, d**-0.5)
    out = torch.empty(n1, t, n2, dtype=torch.float32, device="cuda")
    for _ in range(args.warmup):
        kernels.ghost_gram_per_token(a1, g1, a2, g2, out=out)
    torch.cuda.synchronize()
    timers: dict = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ev = _ev(timers, "per_token")
        kernels.ghost_gram_per_token(a1, g1, a2, g2, out=out)
        _ev_end(ev)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    flops = 2.0 * n1 * n2 * t * t * (d + d)
    t_k = _mean_ms(timers, "per_token")
    tflops = flops / t_k / 1e9
    result = {
        "metric": "per-token train x query scores/sec (256 x 512 train tokens x 64 queries, T=512, d=4096, bf16)",
        "value": round(n1 * t * n2 / (ms / 1e3), 1),
        "unit": "token-scores/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "per-token cross-gram 256 train x 512 tok vs 64 query x 512 tok, d_in=d_out=4096"},
        "roofline": {"bound": "mfma", "kernel": "ghost_per_token_v3", "achieved": round(tflops, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "work_per_launch": f"{flops:.4g} flop = 2 x 256 x 64 pairs x 512^2 x (4096 + 4096)"},
    }
    if args.cpu_baseline:
        import numpy as np

        import oracle

        rng = np.random.default_rng(0)
        s = [rng.standard_normal((n, t, d), dtype=np.float32) for n in (4, 4, 2, 2)]
        t0 = time.perf_counter()
        oracle.cross_gram_per_token(s[0], s[1], s[2], s[3])
        dt = time.perf_counter() - t0
        cores, model = cpu_info()
        result["cpu_baseline"] = {"value": round(4 * t * 2 / dt, 1), "unit": "token-scores/s",
                                  "cores": blas_threads(), "kind": "port",
                                  "sample": f"numpy fp32 oracle, 4 train x 512 tokens x 2 query at d=4096 "
                                            f"({dt:.2f} s); host {model}, {cores} cores visible"}
    return result


# ---------------------------------------------------------------------------
# projected capture (LoGRA route): fused project + outer product, then score
# ---------------------------------------------------------------------------

PROJ_LAYERS = [("gate_proj", 4096, 11008), ("up_proj", 4096, 11008), ("down_proj", 11008, 4096)]


def bench_project(args):
    """Llama-7B MLP projected capture: 512 train + 128 query samples at T=128,
    k=64 on both sides; one step projects and outer-sums every sample of the 3
    MLP linears (fused kernel) and scores the 512 x 128 projected gradients."""
    import torch

    from dattri_llm_amd import kernels
    from dattri_llm_amd.gradient.ops.projection import gaussian_matrix

    n_train, n_query, t, k = 512, 128, 128, 64
    n = n_train + n_query
    gen = torch.Generator(device="cuda").manual_seed(0)
    bf = torch.bfloat16
    acts = {"mlp_in": _randn((n, t, 4096), gen, bf, 4096**-0.5), "down_in": _randn((n, t, 11008), gen, bf, 11008**-0.5)}
    grads = {name: _randn((n, t, dout), gen, bf, dout**-0.5) for name, _i, dout in PROJ_LAYERS}
    mats = {}
    for li, (name, din, dout) in enumerate(PROJ_LAYERS):
        pin = gaussian_matrix(din, k, 2 * li + 1).t().contiguous().to("cuda", bf)
        pout = gaussian_matrix(dout, k, 2 * li).t().contiguous().to("cuda", bf)
        mats[name] = (pin, pout)
    act_of = {"gate_proj": "mlp_in", "up_proj": "mlp_in", "down_proj": "down_in"}
    scores = torch.empty(n_train, n_query, dtype=torch.float32, device="cuda")

    def step(timers=None):
        feats = {}
        for name, _i, _o in PROJ_LAYERS:
            ev = _ev(timers, "project_outer")
            feats[name] = kernels.project_outer(acts[act_of[name]], grads[name], *mats[name])
            _ev_end(ev)
        ev = _ev(timers, "score_gemm")
        kernels.score_gemm([(f[:n_train], f[n_train:]) for f in feats.values()], out=scores)
        _ev_end(ev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timers: dict = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(timers)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    layer_bytes = {name: n * t * (din + dout) * 2.0 for name, din, dout in PROJ_LAYERS}
    t_proj = _mean_ms(timers, "project_outer")
    t_score = _mean_ms(timers, "score_gemm")
    gbs = sum(layer_bytes.values()) / 3 / t_proj / 1e6
    result = {
        "metric": "train x query pair-scores/sec (Llama-7B MLP, projected k=64 capture, bf16)",
        "value": round(n_train * n_query / (ms / 1e3), 1),
        "unit": "pair-scores/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "llama-7b MLP projected capture: 512 train + 128 query, T=128, "
                               "gate/up 4096->11008, down 11008->4096, k=64"},
        "roofline": {"bound": "hbm", "kernel": "da_project_outer (project_pieces + outer_from_pieces)",
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("da_project_outer", PROJECT_TRAFFIC),
                     "traffic_source": os.path.relpath(PROJECT_TRAFFIC, REPO),
                     "work_per_launch": "640 samples x 128 tokens x (d_in + d_out) x 2 B = 2.47e9 B",
                     "launches_per_step": 3, "step_share": round(3 * t_proj / ms, 3)},
        "kernels": {"project_outer": {"ms": round(t_proj, 4), "gbs": round(gbs, 1)},
                    "score_gemm": {"ms": round(t_score, 4)}},
    }
    if args.cpu_baseline:
        import numpy as np

        import oracle

        rng = np.random.default_rng(0)
        f32 = np.float32
        nb = 16
        feats_cpu, dt = [], 0.0
        for li, (name, din, dout) in enumerate(PROJ_LAYERS):
            a = rng.standard_normal((nb, t, din), dtype=f32)
            g = rng.standard_normal((nb, t, dout), dtype=f32)
            pin = gaussian_matrix(din, k, 2 * li + 1).numpy()
            pout = gaussian_matrix(dout, k, 2 * li).numpy()
            t0 = time.perf_counter()
            feats_cpu.append(oracle.project_outer(a, g, pin, pout))
            dt += time.perf_counter() - t0
        per_sample = dt / nb
        step_s = per_sample * n
        cores, model = cpu_info()
        result["cpu_baseline"] = {
            "value": round(n_train * n_query / step_s, 3), "unit": "pair-scores/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"numpy fp32 oracle: projected capture of 16 samples on the 3 layers ({dt:.2f} s), "
                      f"scaled to 640 samples (score GEMM of 512x128x12288 omitted: < 1% of the step); "
                      f"host {model}, {cores} cores visible"}
    return result


# ---------------------------------------------------------------------------
# MoE: router top-k, expert segments, segmented ghost products
# ---------------------------------------------------------------------------


def bench_moe(args):
    """Mixtral-shaped MoE layer: 8 experts, top-2, d 4096, d_ff 14336 (fused
    gate_up 4096->28672, down 14336->4096); 16 train x 256 tokens vs 16 query
    x 256 tokens.  One step: router top-k and expert segments of both sides,
    then the segment-summed ghost products of both expert linears."""
    import torch

    from dattri_llm_amd.gradient import ops

    n_exp, top_k, b, t = 8, 2, 16, 256
    layers = [("gate_up", 4096, 28672), ("down", 14336, 4096)]
    gen = torch.Generator(device="cuda").manual_seed(0)
    bf = torch.bfloat16
    logits = [_randn((b * t, n_exp), gen, torch.float32) for _ in range(2)]
    # Captures in routed order, one set per side, sized from the routing.
    routing = [ops.moe.expert_rows(ops.moe.router_topk(lg, top_k)[1], n_exp) for lg in logits]
    caps = []
    for side in routing:
        per_exp = []
        for _slot, tok in side:
            r = tok.numel()
            per_exp.append({name: (_randn((r, din), gen, bf, din**-0.5), _randn((r, dout), gen, bf, dout**-0.5))
                            for name, din, dout in layers})
        caps.append(per_exp)
    rows = [[tok.numel() for _s, tok in side] for side in routing]
    scores = torch.zeros(b, b, dtype=torch.float32, device="cuda")

    def step(timers=None):
        ev = _ev(timers, "route")
        segs = []
        for lg, r in zip(logits, rows):  # router top-k, then every expert's per-sample segments in one launch
            segs.append(ops.moe.route_segments(ops.moe.router_topk(lg, top_k)[1], n_exp, b, t, rows_per_expert=r))
        _ev_end(ev)
        ev = _ev(timers, "ghost")  # one grouped launch: every expert of both linears
        per_layer = [([(*caps[0][e][name], *caps[1][e][name]) for e in range(n_exp)], False)
                     for name, _i, _o in layers]
        ops.moe.moe_layers_cross_gram(per_layer, segs[0], segs[1], out=scores)
        _ev_end(ev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timers: dict = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(timers)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    flops = sum(2.0 * rows[0][e] * rows[1][e] * (din + dout) for e in range(n_exp) for _n, din, dout in layers)
    t_ghost = _mean_ms(timers, "ghost")
    tf = flops / t_ghost / 1e9
    result = {
        "metric": "train x query pair-scores/sec (Mixtral-shaped MoE layer, top-2 of 8, bf16)",
        "value": round(b * b / (ms / 1e3), 1),
        "unit": "pair-scores/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "mixtral moe layer: 16 train x 256 tok vs 16 query x 256 tok, 8 experts top-2, "
                               "gate_up 4096->28672, down 14336->4096, grouped packed ghost route",
                   "rows_per_expert": rows},
        "roofline": {"bound": "mfma", "kernel": "ghost_grouped_tiles_v3", "achieved": round(tf, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic("ghost_grouped_tiles_v3", MOE_TRAFFIC),
                     "traffic_source": os.path.relpath(MOE_TRAFFIC, REPO),
                     "work_per_step": f"{flops:.4g} flop = sum over experts and both linears "
                                                       "of 2 x rows1 x rows2 x (d_in + d_out)",
                     "launches_per_step": 1, "step_share": round(t_ghost / ms, 3)},
        "kernels": {"route_ms": round(_mean_ms(timers, "route"), 4), "ghost_ms": round(t_ghost, 4)},
    }
    if args.cpu_baseline:
        import numpy as np

        import oracle

        # The reference's CPU path on the whole step (all 16 train x 16 query samples): per expert
        # and linear, the routed rows regrouped to zero-filled (B, T, d) factors, then the dense
        # ghost product.
        ns = b
        sample = []
        for e in range(n_exp):
            toks = [routing[side][e][1] for side in range(2)]
            keep = [(tk < ns * t).cpu() for tk in toks]
            for li, (name, _i, _o) in enumerate(layers):
                fac = [tuple(x[k.to(x.device)].float().cpu().numpy() for x in caps[side][e][name])
                       for side, k in zip(range(2), keep)]
                sample.append((fac, [tk.cpu()[k].numpy() for tk, k in zip(toks, keep)]))
        t0 = time.perf_counter()
        total = np.zeros((ns, ns))
        for ((a1, g1), (a2, g2)), (tk1, tk2) in sample:
            total += oracle.moe_segment_ghost(a1, g1, tk1, a2, g2, tk2, ns, ns, t, t)
        dt = time.perf_counter() - t0
        cores, model = cpu_info()
        result["cpu_baseline"] = {"value": round(ns * ns / dt, 3), "unit": "pair-scores/s", "cores": blas_threads(),
                                  "kind": "port",
                                  "sample": f"numpy float64 oracle (the reference's zero-filled regroup + dense ghost "
                                            f"product) over all 8 experts and both linears for {ns} train x {ns} "
                                            f"query samples ({dt:.2f} s); host {model}, {cores} cores visible"}
    return result


# ---------------------------------------------------------------------------
# projected capture fused into autograd (gradient/capture.py)
# ---------------------------------------------------------------------------


def bench_capture(args):
    """LoGRA capture (k = 64, materialized) of a Llama-7B SwiGLU MLP (gate/up
    4096 -> 11008, down 11008 -> 4096, bf16) inside autograd, one micro-batch of
    128 samples x 128 tokens per step: forward + backward with FusedCapture
    (the capture is the layers' backward: input gradient + one fused
    project-and-outer-sum launch, no weight-gradient GEMM).  Beside it, on the
    same inputs: the plain forward + backward (weight gradients, no capture) and
    the hook-based capture of the reference's design (forward hook keeps the
    activation, backward hook projects both factors and contracts them, weight
    gradients still formed)."""
    import torch
    from torch import nn

    from dattri_llm_amd.gradient import FusedCapture, ops

    b, t, d, f, k = 128, 128, 4096, 11008, 64
    torch.manual_seed(0)

    class Mlp(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate = nn.Linear(d, f, bias=False)
            self.up = nn.Linear(d, f, bias=False)
            self.down = nn.Linear(f, d, bias=False)

        def forward(self, x):
            return self.down(nn.functional.silu(self.gate(x)) * self.up(x))

    model = Mlp().to(device="cuda", dtype=torch.bfloat16)
    for p_ in model.parameters():
        p_.data.mul_(0.05)
    gen = torch.Generator(device="cuda").manual_seed(1)
    x = _randn((b, t, d), gen, torch.bfloat16)
    w = _randn((b, t, d), gen, torch.bfloat16, d**-0.5)

    def loss():
        return (model(x).float() * w.float()).sum()

    cap = FusedCapture(model, proj_dim=k, capture_style="materialized")
    proj = ops.DattriProjector()
    seen: dict = {}  # the last step's (input, grad_output) per layer, to time the capture launches alone
    for name, slot in cap.slots.items():
        inner = slot.capture

        def keep(xa, ga, _inner=inner, _n=name):
            seen[_n] = (xa, ga, _inner)
            _inner(xa, ga)

        slot.capture = keep

    def fused():
        cap.clear()
        with cap:
            loss().backward()
        return cap.gradient()

    def plain():
        model.zero_grad(set_to_none=True)
        loss().backward()

    stash, out = {}, {}

    def hooked():
        model.zero_grad(set_to_none=True)
        hs = []
        for name, m in (("gate", model.gate), ("up", model.up), ("down", model.down)):
            hs.append(m.register_forward_hook(lambda _m, inp, _o, n=name: stash.__setitem__(n, inp[0].detach())))

            def bw(_m, _gi, go, n=name):
                a_p, g_p = ops.project_factors(stash.pop(n), go[0].detach(), "nn.Linear", proj,
                                               {"has_bias": False}, proj_dim=k)
                out[n] = ops.materialize_factors(a_p, g_p, "nn.Linear")

            hs.append(m.register_full_backward_hook(bw))
        loss().backward()
        for h in hs:
            h.remove()

    def run(fn, steps, warm):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    ms_plain = run(plain, args.steps, args.warmup)
    ms_hook = run(hooked, args.steps, args.warmup)
    ms = run(fused, args.steps, args.warmup)
    cap.clear()
    # The capture kernel (da_project_outer) back to back on the last step's
    # tensors with the session's resolved matrices: GPU time per launch (inside
    # backward, events around a launch would also hold the host work between).
    from dattri_llm_amd import kernels

    launches = []
    for xa, ga, _inner in seen.values():
        p_in = cap.projector.resolve(xa.shape[-1], proj_dim=k, proj_seed=cap.proj_seed + 1,
                                     device=xa.device, dtype=xa.dtype)
        p_out = cap.projector.resolve(ga.shape[-1], proj_dim=k, proj_seed=cap.proj_seed,
                                      device=ga.device, dtype=ga.dtype)
        launches.append((xa, ga, p_in.transposed, p_out.transposed))

    def capture_kernels():
        for xa, ga, pi, po in launches:
            kernels.project_outer(xa, ga, pi, po)

    reps = 10
    for _ in range(2):
        capture_kernels()
    torch.cuda.synchronize()
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_ev.record()
    for _ in range(reps):
        capture_kernels()
    e_ev.record()
    torch.cuda.synchronize()
    t_cap = s_ev.elapsed_time(e_ev) / (reps * len(launches))  # per layer launch
    layer_bytes = {"gate": b * t * (d + f) * 2.0, "up": b * t * (d + f) * 2.0, "down": b * t * (f + d) * 2.0}
    cap_bytes = sum(layer_bytes.values()) / 3  # average per capture launch
    gbs = cap_bytes / t_cap / 1e6
    result = {
        "metric": "captured samples/sec, LoGRA k=64 capture inside autograd (Llama-7B SwiGLU MLP, bf16)",
        "value": round(b / (ms / 1e3), 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "llama-7b mlp (gate/up 4096->11008, down 11008->4096, SwiGLU) forward + backward, "
                               "128 samples x 128 tokens, FusedCapture proj_dim 64 materialized"},
        "roofline": {"bound": "hbm", "kernel": "da_project_outer (the capture launch of each layer's backward)",
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("da_project_outer", CAPTURE_TRAFFIC),
                     "traffic_source": os.path.relpath(CAPTURE_TRAFFIC, REPO),
                     "work_per_launch": f"{cap_bytes:.4g} B average = B x T x (d_in + d_out) x 2 B per layer",
                     "launches_per_step": 3},
        "kernels": {"fused_step_ms": round(ms, 4), "plain_backward_step_ms": round(ms_plain, 4),
                    "hook_capture_step_ms": round(ms_hook, 4), "capture_ms_per_layer": round(t_cap, 4)},
    }
    if args.cpu_baseline:
        import copy

        import oracle
        from dattri_llm_amd.gradient.ops.projection import gaussian_matrix

        # The reference's capture on the CPU for the whole step (all 128 samples): fp32 forward +
        # backward with hooks keeping each layer's (input, output gradient), then the oracle's
        # projected outer product per layer.
        nb = b
        cpu_model = copy.deepcopy(model).float().cpu()
        xs, ws = x[:nb].float().cpu(), w[:nb].float().cpu()
        kept: dict = {}
        hooks = []
        shapes = {"gate": (d, f), "up": (d, f), "down": (f, d)}
        for name in shapes:
            mod = getattr(cpu_model, name)
            hooks.append(mod.register_forward_hook(lambda _m, i, _o, n=name: kept.__setitem__(n, [i[0].detach()])))
            hooks.append(mod.register_full_backward_hook(lambda _m, _gi, go, n=name: kept[n].append(go[0].detach())))
        mats = {n: (gaussian_matrix(din, k, 2 * li + 1).numpy(), gaussian_matrix(dout, k, 2 * li).numpy())
                for li, (n, (din, dout)) in enumerate(shapes.items())}
        t0 = time.perf_counter()
        (cpu_model(xs) * ws).sum().backward()
        feats = [oracle.project_outer(av.numpy(), gv.numpy(), *mats[n]) for n, (av, gv) in kept.items()]
        dt = time.perf_counter() - t0
        for h in hooks:
            h.remove()
        assert all(fe.shape == (nb, k * k) for fe in feats)
        cores, model_name = cpu_info()
        result["cpu_baseline"] = {"value": round(nb / dt, 3), "unit": "samples/s", "cores": blas_threads(),
                                  "kind": "port",
                                  "sample": f"torch fp32 forward + backward on the CPU with hook capture and the "
                                            f"numpy oracle's projected outer product, all {nb} samples of the step "
                                            f"({dt:.2f} s); host {model_name}, {cores} cores visible"}
    return result


# ---------------------------------------------------------------------------
# attribute from an on-disk store (gradient/store.py)
# ---------------------------------------------------------------------------


def bench_store(args):
    """Store-then-attribute: LoGRA-projected (k = 64, materialized) gradients of
    3 layers, bf16, for 32768 train samples in 64 files of 512 (the memmap
    store format), scored against 128 cached queries.  One step reads the whole
    train store through PinnedBlockSource (private map -> pinned host buffer ->
    copy-stream H2D overlapped with scoring) and scores it with
    TracInAttributor in train batches of 4096.  The store is written to a temporary directory first (it
    sits in the page cache, so the read side is host memory -> GPU); beside it
    the same scoring from device-resident blocks."""
    import shutil
    import tempfile

    import torch

    from dattri_llm_amd.attribution import TracInAttributor
    from dattri_llm_amd.gradient.gradient import Gradient, GradientRecord
    from dattri_llm_amd.gradient.store import GradientStore, PinnedBlockSource, records_to_block

    layers, width, files, per_file, n_query = ("gate", "up", "down"), 64 * 64, 64, 512, 128
    gen = torch.Generator().manual_seed(0)

    def block(n, tag, i):
        g = Gradient({l: "materialized" for l in layers},
                     {l: (torch.randn(n, width, generator=gen) / 64).bfloat16() for l in layers},
                     {l: "nn.Linear" for l in layers})
        return GradientRecord(0, [f"{tag}{i}-{j}" for j in range(n)], g)

    root = tempfile.mkdtemp(prefix="dattri_store_")
    try:
        train = GradientStore(os.path.join(root, "train"))
        for i in range(files):
            train.save_bulk([block(per_file, "tr", i)])
        test = GradientStore(os.path.join(root, "test"))
        test.save_bulk([block(n_query, "q", 0)])
        dev = torch.device("cuda")

        def resident(store):
            out = []
            for f, by_step in store.iter_steps(store.available_steps()):
                recs = store.load_records(f)
                for step, idxs in by_step.items():
                    b, h = records_to_block(recs, idxs)
                    out.append((step, b.to(dev), h))
            return out

        test_mem = resident(test)
        train_mem = resident(train)
        attr = TracInAttributor(train_batch_size=8 * per_file, device=dev)

        def from_store():
            src = PinnedBlockSource(train, device=dev)
            attr.attribute_sources(src, test_mem)
            return src.h2d_bytes

        def from_memory():
            attr.attribute_sources(train_mem, test_mem)

        def run(fn, steps, warm):
            for _ in range(warm):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                out = fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / steps, out

        ms, h2d = run(from_store, args.steps, args.warmup)
        ms_mem, _ = run(from_memory, args.steps, args.warmup)
        # The score launch itself on one train batch (8 files, 4096 rows) against the queries.
        from dattri_llm_amd import kernels

        batch = {l: torch.cat([b.data[l] for _s, b, _h in train_mem[:8]]) for l in layers}
        out = torch.empty(8 * per_file, n_query, dtype=torch.float32, device=dev)
        pairs = [(batch[l], test_mem[0][1].data[l]) for l in layers]
        for _ in range(3):
            kernels.score_gemm(pairs, out=out)
        reps = 20
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record()
        for _ in range(reps):
            kernels.score_gemm(pairs, out=out)
        e_ev.record()
        torch.cuda.synchronize()
        t_score = s_ev.elapsed_time(e_ev) / reps
        cpu = None
        if args.cpu_baseline:
            import numpy as np

            import oracle

            # The reference's CPU path over the whole store: each memmap group read back
            # (load_records), its blocks assembled, then the numpy oracle's layer-summed scores
            # against the 128 queries.
            q_recs = test.load_records(test.iter_steps(test.available_steps())[0][0])
            q_block, _ = records_to_block(q_recs, list(range(len(q_recs))))
            q_np = [q_block.data[l].float().numpy() for l in layers]
            t0 = time.perf_counter()
            rows = 0
            for f, by_step in train.iter_steps(train.available_steps()):
                recs = train.load_records(f)
                for _step, idxs in by_step.items():
                    blk, _h = records_to_block(recs, idxs)
                    oracle.score_gemm([blk.data[l].float().numpy() for l in layers], q_np)
                    rows += blk.batch_size
            dt = time.perf_counter() - t0
            cores, model_name = cpu_info()
            cpu = {"value": round(rows / dt, 1), "unit": "train-samples/s", "cores": blas_threads(), "kind": "port",
                   "sample": f"the whole store ({rows} train rows, {dt:.2f} s): memmap groups read back, blocks "
                             f"assembled, numpy oracle scores against the 128 queries; host {model_name}, "
                             f"{cores} cores visible"}
    finally:
        shutil.rmtree(root, ignore_errors=True)
    n_train = files * per_file
    launch_bytes = (8 * per_file + n_query) * len(layers) * width * 2.0
    gbs = launch_bytes / t_score / 1e6
    return {
        "metric": "train samples scored/sec from an on-disk gradient store (LoGRA k=64, 3 layers, bf16)",
        "value": round(n_train / (ms / 1e3), 1),
        "unit": "train-samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "attribute from a memmap store: 32768 train x 128 query, 3 layers x 4096 "
                               "(64x64 LoGRA blocks) bf16, 64 files of 512; store in the page cache"},
        "roofline": {"bound": "hbm", "kernel": "da_score_gemm (score_ring64 + reduce), one 4096-row train batch",
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic("score_ring64", STORE_TRAFFIC),
                     "traffic_source": os.path.relpath(STORE_TRAFFIC, REPO),
                     "work_per_launch": f"{launch_bytes:.4g} B = (4096 + 128) x 3 x 4096 x 2 B",
                     "launch_ms": round(t_score, 4), "launches_per_step": files // 8},
        "pipeline": {"h2d_bytes_per_step": h2d, "h2d_gbs": round(h2d / ms / 1e6, 1),
                     "resident_ms_per_step": round(ms_mem, 4)},
        **({"cpu_baseline": cpu} if cpu else {}),
    }


# ---------------------------------------------------------------------------
# K-FAC covariance fit (gradient/ops/kronecker.py, streaming accumulators)
# ---------------------------------------------------------------------------


def bench_kfac(args):
    """K-FAC fit pass over one Llama-8B-block train block (8 x 2048 tokens):
    the A = a^T a and G = g^T g covariance sums of the 7 linears
    (``LayerKroneckerAccumulator.update``), each a symmetric token-axis
    contraction (``da_row_gram``: the 256 x 256 tiles on or above the
    diagonal, then the mirror) over the block's 16384 rows.  The work counted
    is the distinct entries, 2 x rows x p(p+1)/2 flop per factor of width p."""
    import torch

    from dattri_llm_amd.gradient import ops

    n_train, t_train = 8, 2048
    acts, grads, _norms = make_block(n_train, t_train, seed=0)
    torch.cuda.synchronize()

    def step(timers=None):
        accs = {}
        for name, act, _din, _dout in LINEARS:
            ev = _ev(timers, "kfac")
            acc = ops.LayerKroneckerAccumulator()
            acc.update(acts[act], grads[name], "nn.Linear")
            accs[name] = acc
            _ev_end(ev)
        return accs

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timers: dict = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(timers)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    rows = n_train * t_train
    flops = sum(1.0 * rows * (din * (din + 1) + dout * (dout + 1)) for _n, _a, din, dout in LINEARS)
    t_k = _mean_ms(timers, "kfac") * len(LINEARS)
    tf = flops / t_k / 1e9
    result = {
        "metric": "K-FAC covariance fit token rows/sec (Llama-8B-shaped block, 7 linears, bf16)",
        "value": round(rows / (ms / 1e3), 1),
        "unit": "token-rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "k-fac covariances (a^T a, g^T g, fp32 out) of the llama3-8b block's 7 linears "
                               "over one 8 x 2048-token train block"},
        "roofline": {"bound": "mfma",
                     "kernel": "materialize_tiles_tr (symmetric row Gram of 16384 rows) + mirror_lower",
                     "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                     "traffic": profiled_traffic("materialize_tiles_tr", KFAC_TRAFFIC),
                     "traffic_source": os.path.relpath(KFAC_TRAFFIC, REPO),
                     "work_per_step": f"{flops:.4g} flop = sum over the 7 linears of 16384 x (d_in (d_in + 1) "
                                      "+ d_out (d_out + 1)), the distinct entries of A and G",
                     "step_share": round(t_k / ms, 3)},
    }
    if args.cpu_baseline:
        import numpy as np

        import oracle

        rng = np.random.default_rng(0)
        n = 2048  # one sequence of q_proj's factors
        a = rng.standard_normal((1, n, D_MODEL), dtype=np.float32)
        g = rng.standard_normal((1, n, D_MODEL), dtype=np.float32)
        t0 = time.perf_counter()
        oracle.kfac_factors(a, g)
        dt = time.perf_counter() - t0
        cores, model = cpu_info()
        result["cpu_baseline"] = {"value": round(n / dt, 1), "unit": "token-rows/s (q_proj only)",
                                  "cores": blas_threads(), "kind": "port",
                                  "sample": f"numpy float64 oracle kfac_factors on 2048 rows of q_proj "
                                            f"(4096 x 4096 both sides, {dt:.2f} s); host {model}, "
                                            f"{cores} cores visible"}
    return result


# ---------------------------------------------------------------------------
# plain device copy: the reference point for HBM byte counters
# ---------------------------------------------------------------------------


def bench_copy(args):
    """A 2 GiB device-to-device copy (torch's copy kernel): its achieved
    bandwidth, and under a counter profiler the FETCH_SIZE / WRITE_SIZE
    readings that correspond to exactly 2 GiB read and 2 GiB written."""
    import torch

    nbytes = 2 << 30
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    timers: dict = {}
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ev = _ev(timers, "copy")
        dst.copy_(src)
        _ev_end(ev)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    t_k = _mean_ms(timers, "copy")
    gbs = 2 * nbytes / t_k / 1e6
    return {"metric": "device copy bandwidth (2 GiB read + 2 GiB written)", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "device copy 2 GiB"},
            "roofline": {"bound": "hbm", "kernel": "copy", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    # 32 timed steps after 8 warmup: whole groups of the block workload's 16 train blocks per query pass
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", choices=["block", "ghost", "per_token", "project", "moe", "kfac", "capture",
                                           "store", "copy"],
                    default="block")
    ap.add_argument("--no-cpu-baseline", dest="cpu_baseline", action="store_false")
    ap.add_argument("--no-gemm-ref", dest="gemm_ref", action="store_false",
                    help="skip the vendor-GEMM reference added to MFMA-bound lines")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the scoring path would shard train rows, one slice per GPU). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    runs = {"block": bench_block, "ghost": bench_ghost, "per_token": bench_per_token, "project": bench_project,
            "moe": bench_moe, "kfac": bench_kfac, "capture": bench_capture, "store": bench_store,
            "copy": bench_copy}
    result = runs[args.workload](args)
    roof = result.get("roofline") or {}
    if args.gemm_ref and roof.get("bound") == "mfma":
        roof["attainable"] = vendor_gemm_ref()
        roof["frac_of_attainable"] = round(roof["achieved"] / roof["attainable"]["tflops"], 4)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
