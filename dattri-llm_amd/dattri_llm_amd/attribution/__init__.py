"""Attribution on the MI355X scoring path: scores, the scoring loop, TracIn/GradCos."""

from dattri_llm_amd.attribution.score import AttributionScore
from dattri_llm_amd.attribution.tracin import TracInAttributor
from dattri_llm_amd.attribution.utils import finalize_factors, rebatch_blocks, score_sources

__all__ = ["AttributionScore", "TracInAttributor", "finalize_factors", "rebatch_blocks", "score_sources"]
