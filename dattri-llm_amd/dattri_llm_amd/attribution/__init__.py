"""Attribution on the MI355X scoring path: scores, the scoring loop, TracIn/GradCos, K-FAC/EK-FAC."""

from dattri_llm_amd.attribution.base import InnerProductAttributor
from dattri_llm_amd.attribution.kronecker import EKFACAttributor, KFACAttributor, KroneckerAttributor
from dattri_llm_amd.attribution.score import AttributionScore
from dattri_llm_amd.attribution.tracin import TracInAttributor
from dattri_llm_amd.attribution.utils import finalize_factors, rebatch_blocks, score_sources

__all__ = ["AttributionScore", "EKFACAttributor", "InnerProductAttributor", "KFACAttributor",
           "KroneckerAttributor", "TracInAttributor", "finalize_factors", "rebatch_blocks", "score_sources"]
