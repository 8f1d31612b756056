"""Gradient data model and ops (the reference's ``dattri_llm.gradient`` surface on this path)."""

from dattri_llm_amd.gradient import ops
from dattri_llm_amd.gradient.gradient import Factorized, Gradient, GradientRecord
from dattri_llm_amd.gradient.capture import FusedCapture

__all__ = ["Factorized", "FusedCapture", "Gradient", "GradientRecord", "ops"]
