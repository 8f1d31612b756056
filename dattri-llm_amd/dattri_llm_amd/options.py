"""``Literal`` aliases for the enumerated string options on the scoring path.

Same names and values as the reference's ``dattri_llm/options.py:18-54``;
every option is still validated where it is consumed.
"""

from __future__ import annotations

from typing import Literal

CaptureStyle = Literal["factorized", "materialized", "auto"]
RoutingMode = Literal["factorized", "materialized", "auto"]
DotReduce = Literal["sum", "none"]
ProjectionStyle = Literal["logra", "dense", "mask"]
AttributionGranularity = Literal["instance", "token"]
ScoreTrajectory = Literal["aware", "agnostic"]
