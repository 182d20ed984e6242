"""Disk reader (the io/reader.py seam) over the native worker pool.

`DiskReader` keeps the reference's AsyncReader surface (io/reader.py:72-155):
`submit(offset, nbytes)` returns a future, `wait(fut)` resolves it while
counting prefetch hits and stall time, `read` is the blocking form, and
`close` shuts the pool. `IOStats` has the reference's fields and properties
(io/reader.py:31-69).

The reads themselves run in libnsx (`nsx_reader_*`): worker threads issue
positional reads, O_DIRECT where the file system allows it, into staging
buffers. On a GPU reader, `submit` reads straight into a new device tensor:
each chunk is copied out of pinned staging on the reader's copy stream by
the worker that read it, and `wait` orders the caller's stream after those
copies without blocking the host beyond the read itself.
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass
from pathlib import Path

import torch

from .. import _native as N

# io/reader.py:21-27: eight workers was the reference drive's best queue depth
DEFAULT_WORKERS = 8
SLOT_BYTES = 8 << 20  # one staging buffer; larger reads are split across buffers and workers


@dataclass
class IOStats:
    """Reader counters (the fields of io/reader.py:31-69). The native reader
    reports requests, bytes, summed read time and the span of its reads;
    stalls and prefetch hits are counted where futures are waited on."""
    requests: int = 0
    bytes_read: int = 0
    read_seconds: float = 0.0   # summed over workers, so overlapping reads count more than once
    stall_seconds: float = 0.0  # time the compute thread blocked on a future
    prefetch_hits: int = 0      # waits that found their read already done
    prefetch_misses: int = 0    # waits that had to block
    first_read: float = 0.0     # CLOCK_MONOTONIC seconds
    last_read: float = 0.0

    @property
    def wall_seconds(self) -> float:
        """Span from the first read's start to the latest read's end."""
        return self.last_read - self.first_read if self.last_read > self.first_read else 0.0

    @property
    def throughput_gbps(self) -> float:
        """Bytes over the reads' wall-clock span, in GB/s (summed per-worker
        time would understate a pool of concurrent readers)."""
        span = self.wall_seconds
        return self.bytes_read / span / 1e9 if span > 0 else 0.0

    @property
    def prefetch_rate(self) -> float:
        waits = self.prefetch_hits + self.prefetch_misses
        return self.prefetch_hits / waits if waits else 0.0

    def summary(self) -> str:
        return (f"reads: {self.requests} ({self.bytes_read / 2**30:.2f} GiB) at {self.throughput_gbps:.2f} GB/s "
                f"over {self.wall_seconds:.2f} s, {self.stall_seconds:.3f} s stalled, "
                f"{100 * self.prefetch_rate:.1f}% of waits already done")


class ReadFuture:
    """One submitted read: its ticket and destination tensor."""

    __slots__ = ("reader", "ticket", "tensor", "retired", "cancelled", "__weakref__")

    def __init__(self, reader: "DiskReader", ticket: int, tensor: torch.Tensor) -> None:
        self.reader = reader
        self.ticket = ticket
        self.tensor = tensor
        self.retired = False
        self.cancelled = False

    def done(self) -> bool:
        return self.retired or self.reader._poll(self.ticket)

    def result(self) -> torch.Tensor:
        return self.reader._retire(self)

    def cancel(self) -> bool:
        """A read cannot be taken back once queued: wait for it, then drop it
        (the destination must outlive the copy into it). False, as for a
        running concurrent.futures.Future."""
        if not self.retired:
            try:
                self.reader._retire(self)
            except (OSError, EOFError, RuntimeError):
                pass
        self.cancelled = True
        return False

    def __del__(self) -> None:  # never free a destination a copy may still write
        if not self.retired and self.reader is not None and self.reader._handle is not None:
            try:
                self.reader._retire(self)
            except Exception:
                pass


class DiskReader:
    """Thread-pool positional reader of one file (io/reader.py:72-155).

    device: where `submit` puts bytes (a CUDA device: device tensors; None or
    "cpu": host tensors). direct: try O_DIRECT. n_workers may be 0 (a reader
    that never reads; waits time out).
    """

    def __init__(self, path: str | Path, n_workers: int = DEFAULT_WORKERS, device=None, direct: bool = True,
                 slot_bytes: int = SLOT_BYTES, n_slots: int | None = None) -> None:
        self.path = Path(path)
        self.n_workers = int(n_workers)
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        self._lib = N.load()
        self._handle = None
        cuda = self.device.type == "cuda"
        if cuda and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self._copy_stream = torch.cuda.Stream(self.device) if cuda else None
        n_slots = n_slots if n_slots is not None else max(4, 2 * self.n_workers)
        h = C.c_void_p()
        flags = N.READ_DIRECT if direct else 0
        if cuda:
            with torch.cuda.device(self.device):
                rc = self._lib.nsx_reader_open(str(self.path).encode(), self.n_workers, flags, n_slots, slot_bytes,
                                               self.device.index, self._copy_stream.cuda_stream, C.byref(h))
        else:
            rc = self._lib.nsx_reader_open(str(self.path).encode(), self.n_workers, flags, n_slots, slot_bytes,
                                           -1, None, C.byref(h))
        N.check(rc, "open")
        self._handle = h
        self._stall = 0.0
        self._hits = 0
        self._misses = 0

    # -- native plumbing ---------------------------------------------------

    def _stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream if self.device.type == "cuda" else None

    def _submit(self, offset: int, nbytes: int, dst: torch.Tensor) -> ReadFuture:
        if self._handle is None:
            raise RuntimeError("reader is closed")
        on_dev = dst.is_cuda
        t = C.c_uint64()
        N.check(self._lib.nsx_reader_submit(self._handle, int(offset), int(nbytes), dst.data_ptr() if nbytes else None,
                                            int(on_dev), self._stream() if on_dev else None, C.byref(t)),
                f"read of {nbytes} bytes at {offset}")
        if on_dev:
            dst.record_stream(self._copy_stream)  # the copy stream writes it
        return ReadFuture(self, t.value, dst)

    def _poll(self, ticket: int) -> bool:
        return self._handle is not None and self._lib.nsx_reader_poll(self._handle, ticket) == 1

    def _retire(self, fut: ReadFuture, timeout: float | None = None) -> torch.Tensor:
        if fut.retired:
            return fut.tensor
        on_dev = fut.tensor.is_cuda
        us = -1 if timeout is None else int(timeout * 1e6)
        rc = self._lib.nsx_reader_wait(self._handle, fut.ticket, us, self._stream() if on_dev else None)
        if rc != N.ETIMEDOUT:
            fut.retired = True
        N.check(rc, f"{self.path.name}")
        if on_dev:
            fut.tensor.record_stream(torch.cuda.current_stream(self.device))
        return fut.tensor

    # -- the AsyncReader surface --------------------------------------------

    def submit(self, offset: int, nbytes: int) -> ReadFuture:
        """Queue a read into a new tensor on this reader's device. Returns immediately."""
        dst = torch.empty(int(nbytes), dtype=torch.uint8, device=self.device)
        return self._submit(offset, nbytes, dst)

    def submit_many(self, spans: list[tuple[int, int]]) -> list[ReadFuture]:
        return [self.submit(off, n) for off, n in spans]

    def read(self, offset: int, nbytes: int) -> torch.Tensor:
        """Blocking read into a host tensor (pinned on a GPU reader)."""
        pin = self.device.type == "cuda"
        dst = torch.empty(int(nbytes), dtype=torch.uint8, pin_memory=pin)
        return self._retire(self._submit(offset, nbytes, dst))

    def wait(self, fut: ReadFuture, timeout: float | None = None) -> torch.Tensor:
        """Resolve a future, charging blocked time to stall_seconds (io/reader.py:127-139)."""
        if fut.done():
            self._hits += 1
            return self._retire(fut)
        t0 = time.perf_counter()
        try:
            return self._retire(fut, timeout)
        finally:
            self._stall += time.perf_counter() - t0
            self._misses += 1

    @property
    def stats(self) -> IOStats:
        st = IOStats(stall_seconds=self._stall, prefetch_hits=self._hits, prefetch_misses=self._misses)
        if self._handle is not None:
            c = N.ReaderStatsC()
            N.check(self._lib.nsx_reader_get_stats(self._handle, C.byref(c)), "stats")
            self._last = c
        c = getattr(self, "_last", None)
        if c is not None:
            st.requests, st.bytes_read, st.read_seconds = c.requests, c.bytes_read, c.read_seconds
            st.first_read, st.last_read = c.first_read, c.last_read
        return st

    @property
    def direct(self) -> bool:
        """True while reads bypass the page cache."""
        c = N.ReaderStatsC()
        N.check(self._lib.nsx_reader_get_stats(self._handle, C.byref(c)), "stats")
        return bool(c.direct)

    def close(self) -> None:
        if self._handle is None:
            return
        _ = self.stats  # keep the final counters
        h, self._handle = self._handle, None
        N.check(self._lib.nsx_reader_close(h), "close")

    def __enter__(self) -> "DiskReader":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
