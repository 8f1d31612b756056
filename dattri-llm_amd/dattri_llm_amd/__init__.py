"""dattri_llm_amd -- MI355X (gfx950) implementation of dattri-llm's gradient-scoring path.

Mirrors the reference's public names on this path (``gradient.ops``,
``Gradient``/``Factorized``, ``AttributionScore``) over hand-written HIP
kernels reached through a C ABI (``include/dattri_amd.h``).
"""

__version__ = "0.1.0"
