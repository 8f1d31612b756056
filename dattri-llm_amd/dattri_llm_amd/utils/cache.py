"""Byte budgets and an in-memory tensor cache for the scoring loop.

Mirrors the parts of ``dattri_llm/utils/cache.py`` the scoring path uses:
``CacheBudget`` (:89-131, a fraction of free device memory, re-read on every
query) and the memory residency of ``TensorCache`` (:132, ``get`` / ``put`` /
``get_or_compute`` under a budget, usable as a context manager).  Disk and
tiered residency belong to the on-disk store, which this build does not
provide.
"""

from __future__ import annotations

import os
import re
from collections import OrderedDict
from typing import Callable

import torch

DEFAULT_CACHE_FRACTION = 0.35

_MEM_AVAILABLE = re.compile(r"^MemAvailable:\s+(\d+)\s+kB", re.MULTILINE)


def host_free_bytes() -> int:
    """Host memory a new allocation can take now: the kernel's MemAvailable
    estimate (free plus reclaimable page cache), else the free physical pages."""
    try:
        with open("/proc/meminfo", encoding="ascii") as f:
            found = _MEM_AVAILABLE.search(f.read())
        if found:
            return int(found.group(1)) << 10
    except OSError:
        pass
    return os.sysconf("SC_AVPHYS_PAGES") * os.sysconf("SC_PAGE_SIZE")


def device_free_bytes(device) -> int:
    """Free bytes on ``device`` now (``None`` or a CPU device: the host)."""
    if device is not None and device.type == "cuda":
        return int(torch.cuda.mem_get_info(device)[0])
    return host_free_bytes()


class CacheBudget:
    """How many bytes a cache may hold on one device (``None``: the host).

    A budget is a rule evaluated on demand, not a reservation: either the
    fixed ``limit_bytes``, or ``fraction`` of what is free on the device at
    the moment of asking, so a cache shrinks its claims as the rest of the
    run allocates (the reference's ``utils/cache.py:89-131`` contract).
    """

    __slots__ = ("device", "fraction", "limit_bytes")

    def __init__(self, device=None, *, fraction: float = DEFAULT_CACHE_FRACTION,
                 limit_bytes: int | None = None) -> None:
        self.device = None if device is None else torch.device(device)
        self.fraction = fraction
        self.limit_bytes = limit_bytes

    def total(self) -> int:
        """The budget's size in bytes, evaluated now."""
        if self.limit_bytes is None:
            return int(self.fraction * device_free_bytes(self.device))
        return int(self.limit_bytes)

    def room(self, held: int = 0) -> int:
        """Bytes that may still be added on top of ``held`` (never negative)."""
        return max(self.total() - held, 0)

    def fits(self, nbytes: int, held: int = 0) -> bool:
        """True when ``nbytes`` more fit on top of ``held``."""
        return nbytes <= self.room(held)


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
