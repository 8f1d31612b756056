"""The MoE router's selection order (csrc/topk_select.h, the code the
da_moe_topk kernel runs) built for the host and checked against torch.topk on
the CPU, and the oracle's restatement checked the same way.  Rows are drawn
from a few distinct logit values so that ties are the rule, with NaN, +inf and
all -inf rows mixed in; both ATen branches (partial sort for k * 64 <= n,
nth_element otherwise) are covered."""

from __future__ import annotations

import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

import oracle
from conftest import PKG_ROOT, REPO

SHAPES = [(e, k) for e in (1, 2, 3, 5, 8, 9, 16, 33, 64, 65, 128, 130, 256) for k in (1, 2, 3, 4, 8, 16) if k <= e]


def _tied_logits(rows, e, seed):
    r = np.random.default_rng(seed)
    x = r.integers(0, 1 + seed % 4, size=(rows, e)).astype(np.float32)
    x[::7, r.integers(0, e)] = np.nan
    x[3::9, r.integers(0, e)] = np.inf
    x[5::11, :] = -np.inf
    x[6::13, :] = 0.0  # all-equal rows (zero hidden states)
    return x


def _torch_topk(x, k):
    probs = torch.softmax(torch.from_numpy(x).float(), dim=-1)
    vals, idx = torch.topk(probs, k, dim=-1)
    return probs.numpy(), idx.numpy(), (vals / vals.sum(-1, keepdim=True)).numpy()


@pytest.fixture(scope="module")
def host_select(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("topk") / "libtopk_select_host.so"
    src = os.path.join(REPO, "tests", "topk_select_host.cpp")
    subprocess.run([gxx, "-O2", "-std=c++17", "-shared", "-fPIC", f"-I{os.path.join(PKG_ROOT, 'csrc')}",
                    src, "-o", str(out)], check=True)
    lib = ctypes.CDLL(str(out))
    lib.topk_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.topk_rows.restype = None
    return lib


@pytest.mark.parametrize("e,k", SHAPES)
def test_kernel_selection_matches_torch_topk(host_select, e, k):
    x = _tied_logits(60, e, seed=e * 31 + k)
    probs, want, _ = _torch_topk(x, k)
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    got = np.zeros((x.shape[0], k), dtype=np.int64)
    host_select.topk_rows(probs.ctypes.data, x.shape[0], e, k, got.ctypes.data)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("e,k", SHAPES)
def test_oracle_router_matches_torch_topk(e, k):
    x = _tied_logits(40, e, seed=e * 17 + k)
    _probs, want_idx, want_w = _torch_topk(x, k)
    w, idx = oracle.moe_router_topk(x, k)
    assert np.array_equal(idx, want_idx)
    np.testing.assert_allclose(w, want_w, rtol=1e-6, equal_nan=True)


def test_ties_are_not_index_order():
    """The reason for restating the library's selection: torch.topk's CPU tie
    order is neither index order nor stable (all-equal rows of 8 experts come
    back as [6, 5]; a three-way tie at {1, 2, 4} with k = 3 as [1, 4, 2])."""
    _p, idx, _w = _torch_topk(np.zeros((1, 8), np.float32), 2)
    assert idx.tolist() == [[6, 5]]
    x = np.array([[1, 4, 4, 0, 4, -1, 0.5, 0.2]], np.float32)
    _p, idx, _w = _torch_topk(x, 3)
    assert idx.tolist() == [[1, 4, 2]]
    assert oracle.moe_router_topk(x, 3)[1].tolist() == [[1, 4, 2]]
