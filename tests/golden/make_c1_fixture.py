"""Write tests/golden/c1_scores.json: the C1 32 x 8 TracIn score matrix from
per-sample autograd gradients of the tiny decoder (tests/c1_model.py) --
the ground truth the oracle and the GPU path are both checked against.

    python tests/golden/make_c1_fixture.py
"""

from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import torch  # noqa: E402

from c1_model import c1_inputs, per_sample_grads  # noqa: E402


def main():
    torch.set_num_threads(8)
    model, train, query = c1_inputs(0)
    g_tr = per_sample_grads(model, train).double()
    g_q = per_sample_grads(model, query).double()
    scores = (g_tr @ g_q.T).tolist()
    out = {
        "description": "C1: 2-layer decoder (d128, 4 heads, FFN 512 GELU, LayerNorm, vocab 1024, seq 64), "
                       "seed 0, fp32; TracIn scores over all 13 linear layers (weights + biases) from "
                       "per-sample autograd gradients; rows = 32 train, cols = 8 query",
        "train_ids_checksum": int(train.sum()),
        "query_ids_checksum": int(query.sum()),
        "scores": scores,
    }
    with open(os.path.join(HERE, "c1_scores.json"), "w") as f:
        json.dump(out, f)
    print("wrote c1_scores.json", torch.tensor(scores).abs().max().item())


if __name__ == "__main__":
    main()
