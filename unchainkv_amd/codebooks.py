"""Top-16 exponent codebooks: exponent statistics and the fit rule.

Rule (scripts/extract_llama_top16_codebooks.py:39-42 of the reference): per layer
and K/V plane, the exponents seen at least once are ranked by count, most
frequent first, ties to the smaller exponent; the first 16 form the plane's
codebook (code 0 = most frequent). A plane with fewer than 16 distinct exponents
has no codebook.

``summarize_symbol_counts`` produces the ``bf16_exponent_stats`` trace payload
(field names of src/unchain_kv/trace.py:27-58, which the extraction reads back);
``CodebookFitter`` accumulates such trace rows and fits one codebook per layer,
with the result keys of the reference's extraction script.
"""

from __future__ import annotations

import hashlib
import json
import math
from collections.abc import Iterable
from pathlib import Path

import numpy as np

PLANES = ("k", "v")


def _histogram(counts) -> np.ndarray:
    h = np.asarray(list(counts) if not isinstance(counts, np.ndarray) else counts, dtype=np.int64)
    if h.shape != (256,):
        raise ValueError(f"histogram has {h.size} bins, expected 256")
    return h


def rank_exponents(histogram) -> np.ndarray:
    """Exponents with a non-zero count, by (-count, exponent)."""
    h = _histogram(histogram)
    seen = np.flatnonzero(h)
    # lexsort: last key is primary -> count descending, then exponent ascending
    return seen[np.lexsort((seen, -h[seen]))]


def fit_top16(histogram) -> list[int]:
    ranked = rank_exponents(histogram)
    if ranked.size < 16:
        raise ValueError(f"only {ranked.size} observed exponents")
    return [int(e) for e in ranked[:16]]


def fit_layer_codebook(k_histogram, v_histogram) -> bytes:
    """32-byte layer codebook: 16 K exponents then 16 V exponents."""
    return bytes(fit_top16(k_histogram) + fit_top16(v_histogram))


def coverage(histogram, codebook) -> float:
    h = _histogram(histogram)
    total = int(h.sum())
    return float(h[list(codebook)].sum()) / total if total else 0.0


def summarize_symbol_counts(counts: Iterable[int]) -> dict[str, object]:
    """Trace payload of one plane's exponent histogram: word count, the
    histogram, distinct exponents, Shannon entropy in bits, and for the 8 and 16
    most frequent exponents their list, coverage and escape count/rate."""
    h = _histogram(counts)
    words = int(h.sum())
    ranked = rank_exponents(h)
    # summed bin by bin in exponent order, in double precision, so that the trace
    # field is the same float as the reference's (a pairwise numpy sum differs in
    # the last bits)
    entropy = 0.0
    if words:
        for count in h.tolist():
            if count > 0:
                entropy += (count / words) * math.log2(count / words)
        entropy = -entropy
    summary: dict[str, object] = {"words": words, "histogram": h.tolist(),
                                  "unique_exponents": int(ranked.size), "entropy_bits": entropy}
    for size in (8, 16):
        top = ranked[:size]
        escapes = words - int(h[top].sum())
        summary[f"top{size}_exponents"] = top.tolist()
        summary[f"top{size}_coverage"] = (words - escapes) / words if words else 0.0
        summary[f"top{size}_escape_count"] = escapes
        summary[f"top{size}_escape_rate"] = escapes / words if words else 0.0
    return summary


class CodebookFitter:
    """Sums ``bf16_exponent_stats`` histograms per (layer, plane) over trace rows
    and fits the layer codebooks."""

    def __init__(self, layers: Iterable[int]) -> None:
        self.layers = [int(layer) for layer in layers]
        self._sums = np.zeros((len(self.layers), len(PLANES), 256), dtype=np.int64)
        self._slot = {layer: i for i, layer in enumerate(self.layers)}
        self.rows = 0
        self.sources: list[str] = []

    def add_row(self, row: dict) -> bool:
        """Adds one trace row; False when it is not an exponent row of a wanted layer."""
        slot = self._slot.get(int(row.get("layer", -1)))
        if row.get("event") != "bf16_exponent_stats" or slot is None:
            return False
        for p, plane in enumerate(PLANES):
            bins = row[plane]["histogram"]
            if len(bins) != 256:
                raise ValueError(f"layer {self.layers[slot]} {plane} histogram has "
                                 f"{len(bins)} bins")
            self._sums[slot, p] += np.asarray(bins, dtype=np.int64)
        self.rows += 1
        return True

    def add_trace(self, path) -> None:
        with open(path, encoding="utf-8") as handle:
            for line in handle:
                if line.strip():
                    self.add_row(json.loads(line))
        self.sources.append(str(path))

    def histogram(self, layer: int, plane: str) -> np.ndarray:
        return self._sums[self._slot[layer], PLANES.index(plane)].copy()

    def result(self) -> dict[str, object]:
        books = bytearray()
        per_layer = []
        for layer in self.layers:
            entry: dict[str, object] = {"layer": layer}
            for plane in PLANES:
                h = self.histogram(layer, plane)
                try:
                    chosen = fit_top16(h)
                except ValueError as exc:
                    raise ValueError(f"layer {layer} {plane}: {exc}") from None
                entry[plane] = {"words": int(h.sum()), "top16_exponents": chosen,
                                "coverage": coverage(h, chosen)}
                books.extend(chosen)
            per_layer.append(entry)
        return {
            "passed": self.rows >= len(self.layers),
            "trace_rows": self.rows,
            "layers": per_layer,
            "extension_hex": books.hex(),
            "extension_bytes": len(books),
            "extension_sha256": hashlib.sha256(bytes(books)).hexdigest(),
            "source_traces": list(self.sources),
        }


def extract(paths: list[Path], layers: Iterable[int]) -> dict[str, object]:
    """Codebooks of ``layers`` fit on the exponent rows of the given JSONL traces
    (the result of the reference's extract_llama_top16_codebooks.py, for any
    layer range)."""
    fitter = CodebookFitter(layers)
    for path in paths:
        fitter.add_trace(path)
    return fitter.result()
