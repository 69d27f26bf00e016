"""Per-layer Top-16 overflow backoff of the connector's codec policy.

Observable behaviour follows the reference connector's Top-16 backoff
(src/unchain_kv/vllm_connector.py:2906-3021): after an overflowed Top-16 payload
a layer skips Top-16 for a window of payloads, then lets exactly one probe payload
try it; a probe that overflows again doubles the window (up to a cap), a probe that
fits reopens the layer. Every decision carries the layer's epoch, and a result
whose epoch is no longer current is ignored (a late ``ready`` of an older payload
cannot undo a newer decision). A layer whose encoder declines is closed for good.
The trace event names and fields are the reference's.

The state of one layer is a small record; a layer never seen is open with epoch 0.

    open ──overflow──▶ cooling(window) ──window payloads skipped──▶ due
     ▲                                                              │ admit
     └──────────── probe fits ◀──── probing ◀───────────────────────┘
                   probe overflows: cooling(min(2 * window, cap))
"""

from __future__ import annotations

import threading
from dataclasses import dataclass


@dataclass
class _Gate:
    epoch: int = 0
    window: int = 0            # 0: no backoff in force
    skips_left: int = 0        # payloads still to skip before the next probe
    probing: bool = False
    closed: bool = False

    @property
    def open(self) -> bool:
        return self.window == 0


class Top16Backoff:
    """Admission of Top-16 attempts per layer (thread-safe). ``emit(name,
    **fields)`` receives the trace events."""

    def __init__(self, max_window: int, emit) -> None:
        self.max_window = max(1, int(max_window))
        self._emit = emit
        self._gates: dict[int, _Gate] = {}
        self._lock = threading.Lock()

    def _gate(self, layer: int) -> _Gate:
        gate = self._gates.get(layer)
        if gate is None:
            gate = self._gates[layer] = _Gate()
        return gate

    # -- queries (tests and traces) --------------------------------------
    def window(self, layer: int) -> int:
        with self._lock:
            gate = self._gates.get(layer)
            return gate.window if gate else 0

    def skips_left(self, layer: int) -> int | None:
        """Payloads still skipped before a probe; None when no backoff is in force."""
        with self._lock:
            gate = self._gates.get(layer)
            return None if gate is None or gate.open else gate.skips_left

    def epoch(self, layer: int) -> int:
        with self._lock:
            gate = self._gates.get(layer)
            return gate.epoch if gate else 0

    def closed(self, layer: int) -> bool:
        with self._lock:
            gate = self._gates.get(layer)
            return bool(gate and gate.closed)

    def close(self, layer: int) -> None:
        """Close a layer without an attempt (no event, epoch unchanged)."""
        with self._lock:
            self._gate(layer).closed = True

    # -- decisions --------------------------------------------------------
    def admit(self, layer: int) -> tuple[bool, int, bool]:
        """(try Top-16, epoch, is probe) for the next payload of ``layer``."""
        with self._lock:
            gate = self._gate(layer)
            if gate.closed:
                return False, gate.epoch, False
            if gate.open:
                return True, gate.epoch, False
            if gate.skips_left:
                gate.skips_left -= 1
                note = ("splitzip_top16_cooldown_skip",
                        {"layer": layer, "remaining": gate.skips_left, "window": gate.window})
                decision = (False, gate.epoch, False)
            elif gate.probing:
                note = ("splitzip_top16_probe_wait_skip", {"layer": layer})
                decision = (False, gate.epoch, False)
            else:
                gate.epoch += 1
                gate.probing = True
                note = ("splitzip_top16_probe", {"layer": layer, "window": gate.window})
                decision = (True, gate.epoch, True)
        self._emit(note[0], **note[1])
        return decision

    def settle(self, layer: int, epoch: int, probe: bool, overflow: bool) -> None:
        """Outcome of an attempt admitted at ``epoch``."""
        if layer < 0 or epoch < 0:
            return
        with self._lock:
            gate = self._gate(layer)
            if gate.epoch != epoch:
                note = ("splitzip_top16_stale_result", {"layer": layer})
            elif overflow:
                # a probe that overflows backs off twice as long; any other
                # overflow restarts the backoff at one payload
                grown = min(max(1, 2 * gate.window), self.max_window) if probe else 1
                gate.window = gate.skips_left = grown
                gate.probing = False
                gate.epoch += 1
                note = ("splitzip_top16_overflow",
                        {"layer": layer, "window": grown, "probe": probe})
            elif probe:
                gate.window = gate.skips_left = 0
                gate.probing = False
                gate.epoch += 1
                note = ("splitzip_top16_probe_success", {"layer": layer})
            else:
                return
        self._emit(note[0], **note[1])

    def disable(self, layer: int, epoch: int) -> None:
        """The encoder declined the layer: no more Top-16 for it."""
        if layer < 0 or epoch < 0:
            return
        with self._lock:
            gate = self._gate(layer)
            current = gate.epoch == epoch
            if current:
                gate.closed = True
                gate.window = gate.skips_left = 0
                gate.probing = False
                gate.epoch += 1
        self._emit("splitzip_top16_unavailable" if current else "splitzip_top16_stale_result",
                   layer=layer)

    def cancel(self, layer: int, epoch: int, probe: bool) -> None:
        """A probe's encode raised: let the next payload probe instead."""
        if not probe:
            return
        with self._lock:
            gate = self._gates.get(layer)
            if gate is None or gate.epoch != epoch:
                return
            gate.probing = False
        self._emit("splitzip_top16_probe_error", layer=layer)
