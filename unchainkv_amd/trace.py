"""JSONL trace events of the codec path.

Same row shape as the reference's writer (src/unchain_kv/trace.py:11-24):
``{"event": name, "t": perf_counter(), **fields}``, one JSON object per line,
appended under a lock; a writer without a path records nothing.
``RecordingTrace`` keeps rows in memory (for tests and for callers that forward
events elsewhere).
"""

from __future__ import annotations

import json
import threading
import time
from pathlib import Path


class TraceWriter:
    def __init__(self, path: Path | str | None) -> None:
        self.path = Path(path) if path else None
        if self.path is not None:
            self.path.parent.mkdir(parents=True, exist_ok=True)
        self._lock = threading.Lock()

    def event(self, name: str, **fields: object) -> None:
        if self.path is None:
            return
        row = {"event": name, "t": time.perf_counter(), **fields}
        with self._lock:
            with self.path.open("a", encoding="utf-8") as handle:
                handle.write(json.dumps(row, sort_keys=True) + "\n")


class RecordingTrace:
    def __init__(self) -> None:
        self.rows: list[tuple[str, dict]] = []
        self._lock = threading.Lock()

    def event(self, name: str, **fields: object) -> None:
        with self._lock:
            self.rows.append((name, dict(fields)))

    def names(self) -> list[str]:
        with self._lock:
            return [name for name, _ in self.rows]
