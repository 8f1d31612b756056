"""CPU oracle for the gradient-scoring path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of TRAIS-Lab/dattri-llm 0.1.0's ops on this path, each
function citing the reference file:line it follows.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the reference results are compared with / the timed CPU
baseline.  The product package
(``dattri_llm_amd``) never imports it and has no CPU fallback.

Every function computes in the dtype of its inputs (float64 for parity
checks, float32 for the CPU-baseline timing); bf16 inputs are first widened by
the caller, i.e. the oracle is "the reference run with compute dtype float32
(or float64) on bf16-rounded inputs".

Pinning (how each function is checked independently of its own formula) is
listed in ``oracle/ops.py``'s header and enforced by ``tests/test_oracle.py``.
"""

from oracle.ops import *  # noqa: F401,F403
