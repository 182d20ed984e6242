"""Byte budget for blocks in flight (the contract of neurostream/io/arena.py:14-86).

The streaming seam holds a lease on every block it has queued and not yet
consumed; the arena caps the bytes of all such leases. The interface is the
reference's -- `Arena(budget_bytes)` with `budget`, `used`, `available`,
`acquire(nbytes, timeout=None)`, `release(nbytes)`, `reset()`, `stats`
(`ArenaStats`) and `summary()`; `BudgetExceeded` for a request the budget can
never hold, `TimeoutError` for a timed wait that runs out -- but the
bookkeeping here is a first-come-first-served queue: a request that has to
wait is granted before any later request, so a stream of small leases cannot
starve a large one (the reference wakes every waiter and lets them race).
A zero timeout is a try-acquire.
"""
from __future__ import annotations

import threading
import time
from collections import deque
from dataclasses import dataclass


class BudgetExceeded(RuntimeError):
    """One request asks for more bytes than the whole budget."""


@dataclass
class ArenaStats:
    peak_bytes: int = 0        # most bytes leased at once
    total_acquired: int = 0    # bytes granted over the arena's life (since reset)
    n_waits: int = 0           # requests that could not be granted on arrival
    wait_seconds: float = 0.0  # time those requests spent queued


class Arena:
    """Leases of bytes against a fixed budget, granted in arrival order."""

    def __init__(self, budget_bytes: int) -> None:
        budget = int(budget_bytes)
        if budget <= 0:
            raise ValueError(f"arena budget must be a positive byte count, got {budget_bytes}")
        self.budget = budget
        self._held = 0
        self._mutex = threading.Lock()
        self._queue: deque[list] = deque()  # waiting requests: [nbytes, event, granted]
        self.stats = ArenaStats()

    @property
    def used(self) -> int:
        return self._held

    @property
    def available(self) -> int:
        return self.budget - self._held

    def _grant(self, nbytes: int) -> None:
        self._held += nbytes
        st = self.stats
        st.total_acquired += nbytes
        st.peak_bytes = max(st.peak_bytes, self._held)

    def _serve_queue(self) -> None:
        """Grant queued requests from the front while they fit (mutex held)."""
        while self._queue and self._held + self._queue[0][0] <= self.budget:
            req = self._queue.popleft()
            self._grant(req[0])
            req[2] = True
            req[1].set()

    def acquire(self, nbytes: int, timeout: float | None = None) -> None:
        """Lease `nbytes`, waiting (up to `timeout` seconds; None = no limit)
        behind earlier requests until they fit."""
        nbytes = int(nbytes)
        if nbytes > self.budget:
            raise BudgetExceeded(
                f"a {nbytes:,}-byte block can never fit a {self.budget:,}-byte arena: use smaller "
                "blocks (block_rows) or a larger budget")
        with self._mutex:
            if not self._queue and self._held + nbytes <= self.budget:
                self._grant(nbytes)
                return
            req = [nbytes, threading.Event(), False]
            self._queue.append(req)
            self.stats.n_waits += 1
        t0 = time.perf_counter()
        req[1].wait(timeout)
        with self._mutex:
            self.stats.wait_seconds += time.perf_counter() - t0
            if req[2]:
                return
            self._queue.remove(req)
            self._serve_queue()  # requests queued behind this one may fit now
        raise TimeoutError(f"no {nbytes:,} bytes of the arena came free within {timeout} s "
                           f"({self._held:,} of {self.budget:,} leased)")

    def release(self, nbytes: int) -> None:
        """Return a lease; the count never drops below zero."""
        with self._mutex:
            self._held = max(0, self._held - int(nbytes))
            self._serve_queue()

    def reset(self) -> None:
        """Forget every lease and the statistics; waiting requests are granted
        in order as far as the emptied budget allows."""
        with self._mutex:
            self._held = 0
            self.stats = ArenaStats()
            self._serve_queue()

    def summary(self) -> str:
        st = self.stats
        return (f"arena: peak {st.peak_bytes / 2**20:.1f} MiB of {self.budget / 2**20:.1f} MiB, "
                f"{st.total_acquired / 2**20:.1f} MiB leased in total, {st.n_waits} waits "
                f"({st.wait_seconds:.3f} s)")
