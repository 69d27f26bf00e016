"""Host staging copies of the connector's restore (staging.HostCopier): the
threaded path places every payload's bytes exactly where the single-threaded
path does, for byte strings, numpy-backed memoryviews and odd sizes."""

import numpy as np

from unchainkv_amd.staging import HostCopier


def _pieces(rng, sizes, gap=37):
    pieces, at = [], 0
    for k, n in enumerate(sizes):
        data = rng.integers(0, 256, n, dtype=np.uint8)
        src = data.tobytes() if k % 2 else memoryview(data)
        pieces.append((at, src))
        at += n + gap
    return pieces, at


def test_threaded_copy_matches_serial():
    rng = np.random.default_rng(3)
    sizes = [9 << 20, 1, (5 << 20) + 3, 4 << 20, 12345]
    pieces, end = _pieces(rng, sizes)
    serial = np.zeros(end, np.uint8)
    HostCopier(threads=1).copy(serial, pieces)
    threaded = np.full(end, 7, np.uint8)
    HostCopier(threads=4).copy(threaded, pieces)
    for at, src in pieces:
        assert bytes(serial[at:at + len(src)]) == bytes(src)
    # gaps untouched by either path
    mask = np.ones(end, bool)
    for at, src in pieces:
        mask[at:at + len(src)] = False
    assert (serial[mask] == 0).all() and (threaded[mask] == 7).all()
    assert np.array_equal(serial[~mask], threaded[~mask])


def test_small_totals_stay_on_the_calling_thread():
    rng = np.random.default_rng(4)
    pieces, end = _pieces(rng, [100, 2000, 3])
    copier = HostCopier(threads=4)
    dst = np.zeros(end, np.uint8)
    copier.copy(dst, pieces)
    assert copier._pool is None
    for at, src in pieces:
        assert bytes(dst[at:at + len(src)]) == bytes(src)


def test_streamed_copy_reports_each_finished_prefix_in_order():
    """copy_streamed hands out ascending, contiguous ranges from 0 to the end, each
    at least the window long except the last, and every byte of a range is in
    place when the range is reported (what lets the connector start a range's
    host-to-device copy while later payloads are still being copied)."""
    rng = np.random.default_rng(5)
    sizes = [9 << 20, 1, (5 << 20) + 3, 4 << 20, 12345, 7 << 20]
    pieces, end = _pieces(rng, sizes)
    expected = np.full(end, 9, np.uint8)
    for at, src in pieces:
        expected[at:at + len(src)] = np.frombuffer(src, np.uint8)
    dst = np.full(end, 9, np.uint8)
    ranges = []

    def on_ready(lo, hi):
        assert np.array_equal(dst[lo:hi], expected[lo:hi]), (lo, hi)
        ranges.append((lo, hi))

    HostCopier(threads=4).copy_streamed(dst, pieces, on_ready, end=end, window=6 << 20)
    assert ranges[0][0] == 0 and ranges[-1][1] == end
    assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
    assert all(hi - lo >= 6 << 20 for lo, hi in ranges[:-1])
    assert len(ranges) > 2
    assert np.array_equal(dst, expected)


def test_streamed_copy_of_a_small_total_reports_one_range():
    rng = np.random.default_rng(6)
    pieces, end = _pieces(rng, [100, 2000])
    got = []
    dst = np.zeros(end, np.uint8)
    HostCopier(threads=4).copy_streamed(dst, pieces, lambda lo, hi: got.append((lo, hi)))
    assert got == [(0, pieces[-1][0] + 2000)]


class _FakeTensor:
    def __init__(self, n):
        self.n = n

    def numel(self):
        return self.n


class _FakeTorch:
    uint8 = "uint8"

    def __init__(self):
        self.allocated = 0

    def empty(self, n, dtype=None, pin_memory=False):
        self.allocated += 1
        return _FakeTensor(n)


def test_pinned_pool_keeps_idle_slots_when_a_request_exceeds_the_cap():
    from unchainkv_amd.staging import GRANULE, PinnedPool

    torch = _FakeTorch()
    pool = PinnedPool(cap_bytes=8 * GRANULE)
    a = pool.acquire(3 * GRANULE, torch)
    b = pool.acquire(3 * GRANULE, torch)
    pool.release(a)
    pool.release(b)
    assert len(pool._slots) == 2
    assert pool.acquire(9 * GRANULE, torch) is None     # larger than the cap itself
    assert len(pool._slots) == 2 and torch.allocated == 2
    # a request that fits after evicting one idle slot still gets one
    c = pool.acquire(5 * GRANULE, torch)
    assert c is not None and c.capacity == 5 * GRANULE
    assert pool.committed_bytes <= 8 * GRANULE


def test_streamed_copy_error_leaves_no_copy_running():
    """When the range callback raises (as an upload may), copy_streamed re-raises
    only after every copy job has finished or been cancelled: nothing writes into
    the destination once the caller sees the error and returns it to a pool."""
    import threading
    import time

    import pytest

    rng = np.random.default_rng(8)
    pieces, end = _pieces(rng, [4 << 20] * 12)
    dst = np.zeros(end, np.uint8)
    copier = HostCopier(threads=2)
    running = []
    lock = threading.Lock()
    original = np.copyto

    def slow_copy(out, src):
        with lock:
            running.append(1)
        time.sleep(0.01)
        original(out, src)
        with lock:
            running.pop()

    def fail(lo, hi):
        raise RuntimeError("upload failed")

    np.copyto = slow_copy
    try:
        with pytest.raises(RuntimeError, match="upload failed"):
            copier.copy_streamed(dst, pieces, fail, window=4 << 20)
        assert not running
        snapshot = dst.copy()
        time.sleep(0.05)
        assert np.array_equal(dst, snapshot)
    finally:
        np.copyto = original
