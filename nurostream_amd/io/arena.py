"""Byte budget shared by every in-flight block (neurostream/io/arena.py:26-86).

Same contract as the reference: `acquire(nbytes, timeout)` blocks until the
bytes fit, raises `BudgetExceeded` for a request larger than the whole budget
and `TimeoutError` when a timed wait starves; `release` never goes below zero;
`stats.peak_bytes` records the high-water mark. Here the budget bounds the
device staging bytes of blocks copied from host RAM and not yet consumed.
"""
from __future__ import annotations

import threading
import time
from dataclasses import dataclass


class BudgetExceeded(RuntimeError):
    """A single request is larger than the entire budget."""


@dataclass
class ArenaStats:
    peak_bytes: int = 0
    total_acquired: int = 0
    n_waits: int = 0
    wait_seconds: float = 0.0


class Arena:
    """Counting semaphore over bytes with blocking acquire."""

    def __init__(self, budget_bytes: int) -> None:
        if budget_bytes <= 0:
            raise ValueError("budget must be positive")
        self.budget = int(budget_bytes)
        self._used = 0
        self._cv = threading.Condition()
        self.stats = ArenaStats()

    @property
    def used(self) -> int:
        return self._used

    @property
    def available(self) -> int:
        return self.budget - self._used

    def acquire(self, nbytes: int, timeout: float | None = None) -> None:
        if nbytes > self.budget:
            raise BudgetExceeded(
                f"request of {nbytes / 1e6:.1f}MB exceeds the whole {self.budget / 1e6:.1f}MB "
                "budget; raise the budget or lower block_rows")
        with self._cv:
            if self._used + nbytes > self.budget:
                self.stats.n_waits += 1
                t0 = time.perf_counter()
                ok = self._cv.wait_for(lambda: self._used + nbytes <= self.budget, timeout)
                self.stats.wait_seconds += time.perf_counter() - t0
                if not ok:
                    raise TimeoutError(f"arena starved waiting for {nbytes / 1e6:.1f}MB")
            self._used += nbytes
            self.stats.total_acquired += nbytes
            if self._used > self.stats.peak_bytes:
                self.stats.peak_bytes = self._used

    def release(self, nbytes: int) -> None:
        with self._cv:
            self._used = max(0, self._used - nbytes)
            self._cv.notify_all()

    def reset(self) -> None:
        with self._cv:
            self._used = 0
            self.stats = ArenaStats()
            self._cv.notify_all()

    def summary(self) -> str:
        return (f"peak {self.stats.peak_bytes / 1e6:.1f}MB / budget {self.budget / 1e6:.1f}MB | "
                f"waits {self.stats.n_waits} ({self.stats.wait_seconds:.2f}s)")
