"""Byte budgets and an in-memory tensor cache for the scoring loop.

Mirrors the parts of ``dattri_llm/utils/cache.py`` the scoring path uses:
``CacheBudget`` (:89-131, a fraction of free device memory, re-read on every
query) and the memory residency of ``TensorCache`` (:132, ``get`` / ``put`` /
``get_or_compute`` under a budget, usable as a context manager).  Disk and
tiered residency belong to the on-disk store, which this build does not
provide.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Callable

import torch

DEFAULT_CACHE_FRACTION = 0.35


def available_host_bytes() -> int:
    try:
        with open("/proc/meminfo", encoding="utf-8") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except (OSError, ValueError, IndexError):
        pass
    return 16 * 2**30


class CacheBudget:
    """Byte budget a cache may occupy on a device (``None`` = host)."""

    def __init__(self, device=None, *, fraction: float = DEFAULT_CACHE_FRACTION,
                 limit_bytes: int | None = None) -> None:
        self._device = torch.device(device) if device is not None else None
        self._fraction = fraction
        self._limit = limit_bytes

    @property
    def device(self):
        return self._device

    def total(self) -> int:
        """Bytes the cache may hold in total, right now."""
        if self._limit is not None:
            return self._limit
        if self._device is not None and self._device.type == "cuda":
            free, _total = torch.cuda.mem_get_info(self._device)
            return int(free * self._fraction)
        return int(available_host_bytes() * self._fraction)

    def fits(self, nbytes: int, held: int = 0) -> bool:
        """Whether *nbytes* more may be cached given *held* bytes already are."""
        return held + nbytes <= self.total()


def _nbytes(value) -> int:
    if isinstance(value, torch.Tensor):
        return value.numel() * value.element_size()
    if isinstance(value, (tuple, list)):
        return sum(_nbytes(v) for v in value)
    return 0


class TensorCache:
    """An in-memory, budget-bounded key -> tensor cache (LRU eviction)."""

    def __init__(self, residency: str = "memory", *, budget: CacheBudget | None = None) -> None:
        if residency != "memory":
            raise NotImplementedError("only memory residency is provided on this path")
        self._budget = budget
        self._items: OrderedDict = OrderedDict()
        self._held = 0

    def get(self, key):
        value = self._items.get(key)
        if value is not None:
            self._items.move_to_end(key)
        return value

    def put(self, key, value) -> bool:
        size = _nbytes(value)
        if key in self._items:
            self._held -= _nbytes(self._items.pop(key))
        if self._budget is not None:
            if not self._budget.fits(size, 0):  # could never fit: keep what is cached
                return False
            while self._items and not self._budget.fits(size, self._held):
                _k, old = self._items.popitem(last=False)
                self._held -= _nbytes(old)
            if not self._budget.fits(size, self._held):
                return False
        self._items[key] = value
        self._held += size
        return True

    def get_or_compute(self, key, fn: Callable):
        value = self.get(key)
        if value is None:
            value = fn()
            self.put(key, value)
        return value

    def clear(self) -> None:
        self._items.clear()
        self._held = 0

    def __contains__(self, key) -> bool:
        return key in self._items

    def __len__(self) -> int:
        return len(self._items)

    def __enter__(self):
        return self

    def __exit__(self, *_exc) -> bool:
        self.clear()
        return False
