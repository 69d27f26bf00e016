"""Pinned host staging for codec payloads: a reusable pool of pinned buffers and a
device-to-host copy stream per GPU.

Behaviour of the reference connector's pinned staging (`_stage_cpu`,
src/unchain_kv/vllm_connector.py:3406-3458, pool `_acquire_pinned_stage_buffer`
:3970-4040): payload copies leave the forward stream, run on a dedicated copy
stream that first waits for the work queued so far, land in pinned buffers that
are reused once released and their copy has finished, and the pool can be capped
in buffers or bytes (UNCHAIN_KV_HOST_MIRROR_LAYERS / _BYTES); when the cap leaves
no buffer the caller copies synchronously instead.

Here buffers are plain pinned byte tensors sized in 2 MiB steps, handed out
smallest-fit; a released buffer returns to the pool at once and is reused only
after its last copy's event has completed. Each lease has a number, so a late
release of an earlier lease (a view's finaliser after an explicit release) leaves
the buffer's current lease alone.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass

GRANULE = 2 << 20


@dataclass(eq=False)
class PinnedSlot:
    tensor: object            # pinned uint8 CPU tensor
    event: object = None      # last copy into or out of it (torch.cuda.Event)
    leased: bool = False
    lease: int = 0            # number of the current (or last) lease

    @property
    def capacity(self) -> int:
        return int(self.tensor.numel())

    def view(self, nbytes: int):
        return self.tensor[:nbytes]


class PinnedPool:
    """Pinned host buffers reused across layers (thread-safe)."""

    def __init__(self, cap_bytes: int = 0, cap_buffers: int = 0) -> None:
        self.cap_bytes = max(0, int(cap_bytes))
        self.cap_buffers = max(0, int(cap_buffers))
        self._slots: list[PinnedSlot] = []
        self._lock = threading.Lock()
        self.allocations = 0

    @staticmethod
    def _idle(slot: PinnedSlot) -> bool:
        return not slot.leased and (slot.event is None or slot.event.query())

    @property
    def committed_bytes(self) -> int:
        return sum(s.capacity for s in self._slots)

    def acquire(self, nbytes: int, torch) -> PinnedSlot | None:
        """A leased buffer of at least nbytes, or None when the caps leave none."""
        nbytes = max(1, int(nbytes))
        with self._lock:
            fits = [s for s in self._slots if s.capacity >= nbytes and self._idle(s)]
            if fits:
                slot = min(fits, key=lambda s: s.capacity)
                slot.leased = True
                slot.lease += 1
                return slot
            size = -(-nbytes // GRANULE) * GRANULE
            if self.cap_bytes and size > self.cap_bytes:
                # no eviction could make room: keep the idle buffers for later layers
                return None

            def over() -> bool:
                return ((self.cap_buffers and len(self._slots) >= self.cap_buffers)
                        or (self.cap_bytes and self.committed_bytes + size > self.cap_bytes))

            while over():
                idle = [s for s in self._slots if self._idle(s)]
                if not idle:
                    return None
                self._slots.remove(max(idle, key=lambda s: s.capacity))
            slot = PinnedSlot(torch.empty(size, dtype=torch.uint8, pin_memory=True), leased=True,
                              lease=1)
            self._slots.append(slot)
            self.allocations += 1
            return slot

    def release(self, slot: PinnedSlot, lease: int | None = None) -> None:
        """Ends the slot's lease (only lease number ``lease``, when given)."""
        with self._lock:
            if lease is None or slot.lease == lease:
                slot.leased = False


class CopyStreams:
    """One device-to-host copy stream per GPU, at the default priority."""

    def __init__(self) -> None:
        self._streams: dict[int, object] = {}
        self._lock = threading.Lock()

    def get(self, device, torch):
        index = device.index if device.index is not None else torch.cuda.current_device()
        with self._lock:
            stream = self._streams.get(index)
            if stream is None:
                stream = self._streams[index] = torch.cuda.Stream(device=index)
            return stream


class HostCopier:
    """Copies payload bytes into a staging buffer, large totals split over a few
    threads (numpy releases the GIL for large contiguous copies: one Llama-3-8B
    layer's 100 MB of payloads took ~4 ms on one thread)."""

    PARALLEL_BYTES = 8 << 20
    PIECE = 4 << 20

    def __init__(self, threads: int = 8) -> None:
        self.threads = max(1, threads)
        self._pool = None
        self._lock = threading.Lock()

    def _executor(self):
        with self._lock:
            if self._pool is None:
                from concurrent.futures import ThreadPoolExecutor

                self._pool = ThreadPoolExecutor(self.threads, thread_name_prefix="ukv-stage")
            return self._pool

    def copy(self, dst, pieces) -> None:
        """dst: writable uint8 numpy array; pieces: (offset in dst, bytes-like)."""
        self.copy_streamed(dst, pieces, None)

    def copy_streamed(self, dst, pieces, on_ready, end: int | None = None,
                      window: int = 16 << 20) -> None:
        """copy() that also calls ``on_ready(lo, hi)`` on the calling thread each
        time a further prefix of ``dst`` holds its bytes: ascending, contiguous
        ranges of at least ``window`` bytes from 0, the last one ending at ``end``
        (default: the end of the last piece; bytes between pieces are whatever
        ``dst`` held). A device copy of each range can then run while later pieces
        are still being copied. ``pieces`` must be in ascending offset order."""
        import numpy as np

        if end is None:
            end = max((at + len(src) for at, src in pieces), default=0)
        total = sum(len(src) for _, src in pieces)
        if total < self.PARALLEL_BYTES or self.threads == 1:
            view = memoryview(dst)
            for at, src in pieces:
                view[at:at + len(src)] = src
            if on_ready is not None and end > 0:
                on_ready(0, end)
            return
        jobs = []
        for at, src in pieces:
            arr = np.frombuffer(src, dtype=np.uint8)
            for lo in range(0, arr.size, self.PIECE):
                hi = min(lo + self.PIECE, arr.size)
                jobs.append((at + lo, arr[lo:hi]))
        if any(jobs[k + 1][0] < jobs[k][0] for k in range(len(jobs) - 1)):
            raise ValueError("pieces must be in ascending offset order")

        def run(job):
            at, arr = job
            np.copyto(dst[at:at + arr.size], arr)

        from concurrent.futures import wait

        pool = self._executor()
        futures = [pool.submit(run, job) for job in jobs]
        issued = 0
        try:
            for (at, arr), fut in zip(jobs, futures):
                fut.result()  # in order: every earlier job has finished too
                done = at + arr.size
                if on_ready is not None and done - issued >= window:
                    on_ready(issued, done)
                    issued = done
            if on_ready is not None and end > issued:
                on_ready(issued, end)
        except BaseException:
            # no copy may still write into dst once the caller sees the error (it
            # may hand dst back to a pool): cancel the queued jobs, wait for the rest
            for fut in futures:
                fut.cancel()
            wait(futures)
            raise

