"""Host logic of the K-FAC / EK-FAC attributors on the CPU: option validation
(the reference's attribution/algorithm/kronecker.py:555-597, :1472-1484), the
re-iterable train source requirement (:301-308), the no-eligible-layer error
(:335-347) and the test-side transform guard (:610-613).  None of these paths
launches a kernel."""

from __future__ import annotations

import pytest
import torch

from dattri_llm_amd.attribution import EKFACAttributor, KFACAttributor
from dattri_llm_amd.gradient import Factorized, Gradient


class Source:
    def __init__(self, blocks, reusable=True):
        self.blocks, self.reusable = blocks, reusable

    def __iter__(self):
        return iter(self.blocks)


def _norm_only_block():
    x = torch.randn(2, 3, 4)
    data = {"ln": Factorized(x, x.clone())}
    return Gradient({"ln": "factorized"}, data, {"ln": "nn.RMSNorm"}, {"ln": "batch_token"})


@pytest.mark.parametrize("kwargs, match", [
    ({"damping": -1.0}, "damping must be non-negative"),
    ({"non_kfac_strategy": "fim"}, "non_kfac_strategy must be"),
    ({"direct_fim_max_params": 0}, "direct_fim_max_params must be positive"),
])
def test_options_are_validated(kwargs, match):
    with pytest.raises(ValueError, match=match):
        KFACAttributor(device="cpu").set_options(**kwargs)


def test_ekfac_mode_is_validated():
    assert EKFACAttributor(device="cpu", mode="approx").mode == "approx"
    with pytest.raises(ValueError, match="mode must be one of"):
        EKFACAttributor(device="cpu", mode="fast")


def test_train_source_must_be_reusable():
    src = Source([(0, _norm_only_block(), ["a", "b"])], reusable=False)
    with pytest.raises(ValueError, match="re-iterable train source"):
        KFACAttributor(device="cpu").attribute_sources(src, src)


@pytest.mark.parametrize("cls", [KFACAttributor, EKFACAttributor])
def test_no_eligible_layer_raises(cls):
    src = Source([(0, _norm_only_block(), ["a", "b"])])
    with pytest.raises(ValueError, match="non_kfac_strategy='direct'"):
        cls(device="cpu").attribute_sources(src, src)


def test_transform_needs_a_fit():
    with pytest.raises(RuntimeError, match="prepare_scoring"):
        KFACAttributor(device="cpu").transform_test_rep(_norm_only_block())
