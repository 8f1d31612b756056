"""Small host-side utilities (cache budgets)."""

from dattri_llm_amd.utils.cache import CacheBudget, TensorCache

__all__ = ["CacheBudget", "TensorCache"]
