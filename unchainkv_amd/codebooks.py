"""Top-16 exponent codebooks: histogram statistics and the fit rule.

The fit follows scripts/extract_llama_top16_codebooks.py:15-60 of the reference:
per layer and plane, exponents are ranked by (-count, value) and the first 16 with
a non-zero count form the codebook (code 0 = most frequent); fewer than 16
observed exponents is an error. ``summarize_symbol_counts`` follows
src/unchain_kv/trace.py:27-58 (the ``bf16_exponent_stats`` trace payload that the
extraction script reads). ``extract`` aggregates such trace rows.
"""

from __future__ import annotations

import hashlib
import json
import math
from collections.abc import Iterable
from pathlib import Path


def fit_top16(histogram) -> list[int]:
    histogram = [int(v) for v in histogram]
    if len(histogram) != 256:
        raise ValueError(f"histogram has {len(histogram)} bins, expected 256")
    ranked = sorted(range(256), key=lambda value: (-histogram[value], value))
    selected = [value for value in ranked if histogram[value] > 0][:16]
    if len(selected) != 16:
        raise ValueError(f"only {len(selected)} observed exponents")
    return selected


def fit_layer_codebook(k_histogram, v_histogram) -> bytes:
    """32-byte layer codebook: 16 K exponents then 16 V exponents."""
    return bytes(fit_top16(k_histogram) + fit_top16(v_histogram))


def coverage(histogram, codebook) -> float:
    total = sum(int(v) for v in histogram)
    covered = sum(int(histogram[e]) for e in codebook)
    return covered / total if total else 0.0


def summarize_symbol_counts(counts: Iterable[int]) -> dict[str, object]:
    histogram = [int(v) for v in counts]
    words = sum(histogram)
    ranked = sorted((s for s, c in enumerate(histogram) if c > 0),
                    key=lambda s: (-histogram[s], s))
    entropy = 0.0
    if words:
        entropy = -sum((c / words) * math.log2(c / words) for c in histogram if c > 0)
    result: dict[str, object] = {
        "words": words,
        "histogram": histogram,
        "unique_exponents": len(ranked),
        "entropy_bits": entropy,
    }
    for size in (8, 16):
        top = ranked[:size]
        covered = sum(histogram[s] for s in top)
        result.update({
            f"top{size}_exponents": top,
            f"top{size}_coverage": covered / words if words else 0.0,
            f"top{size}_escape_count": words - covered,
            f"top{size}_escape_rate": (words - covered) / words if words else 0.0,
        })
    return result


def extract(paths: list[Path], layers: Iterable[int]) -> dict[str, object]:
    """Aggregate ``bf16_exponent_stats`` trace rows of the given layers and fit one
    codebook per layer (K then V), as the reference's extraction script does."""
    layers = list(layers)
    counts = {layer: {plane: [0] * 256 for plane in ("k", "v")} for layer in layers}
    rows = 0
    for path in paths:
        for line in Path(path).read_text(encoding="utf-8").splitlines():
            row = json.loads(line)
            layer = int(row.get("layer", -1))
            if row.get("event") != "bf16_exponent_stats" or layer not in counts:
                continue
            rows += 1
            for plane in ("k", "v"):
                histogram = row[plane]["histogram"]
                if len(histogram) != 256:
                    raise ValueError(f"layer {layer} {plane} histogram has {len(histogram)} bins")
                counts[layer][plane] = [a + int(b) for a, b in zip(counts[layer][plane], histogram)]
    books = bytearray()
    per_layer = []
    for layer in layers:
        entry = {"layer": layer}
        for plane in ("k", "v"):
            histogram = counts[layer][plane]
            selected = fit_top16(histogram)
            entry[plane] = {
                "words": sum(histogram),
                "top16_exponents": selected,
                "coverage": coverage(histogram, selected),
            }
            books.extend(selected)
        per_layer.append(entry)
    return {
        "passed": rows >= len(layers),
        "trace_rows": rows,
        "layers": per_layer,
        "extension_hex": books.hex(),
        "extension_bytes": len(books),
        "extension_sha256": hashlib.sha256(books).hexdigest(),
        "source_traces": [str(p) for p in paths],
    }
