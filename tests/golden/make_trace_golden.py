#!/usr/bin/env python3
"""Write reference-produced fixtures for the exponent-statistics trace payload.

Run in the build container only, where the reference checkout is at
/root/reference. ``summarize_symbol_counts`` (src/unchain_kv/trace.py:27-58) turns
one plane's 256-bin exponent histogram into the ``bf16_exponent_stats`` trace
fields (the connector's `_trace_bf16_exponents`, vllm_connector.py:2871-2904);
its exact output (ranking ties, float entropy and rates) is pinned by nothing
but the function itself, so this script imports the reference's trace module
(pure Python: json, math, pathlib, threading, time) and records its output on
seeded histograms. Only the inputs and the outputs it produced are written, as
JSON data, to ``trace_summary_cases.json``.

Histograms: empty; one exponent; four equal counts (entropy 2 bits); ties in
count ranked by exponent; more than 16 exponents with random counts; all 256
exponents; counts of real size (a 16 M-word plane of N(0, 1) bf16 words, K
scaled per channel as in the benchmark's generator) and huge counts.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

REFERENCE = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "trace_summary_cases.json"


def bf16_exponents(values: np.ndarray) -> np.ndarray:
    """Exponent bits of the bf16 rounding (to nearest even) of float32 values."""
    bits = values.astype(np.float32).view(np.uint32)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    return ((rounded >> 7) & 0xFF).astype(np.int64)


def histograms():
    rng = np.random.default_rng(20261202)
    cases = []

    def add(name, hist):
        hist = [int(x) for x in hist]
        assert len(hist) == 256
        cases.append((name, hist))

    add("empty", [0] * 256)
    one = [0] * 256
    one[127] = 12345
    add("one_exponent", one)
    four = [0] * 256
    for e in (7, 9, 11, 13):
        four[e] = 25
    add("four_equal", four)
    ties = [0] * 256
    for e in (200, 3, 150, 90, 17, 250, 64, 128, 1, 2):
        ties[e] = 40                      # ten-way tie at the top
    for e in range(30, 50):
        ties[e] = 7                       # twenty-way tie below it
    ties[255] = 41
    add("ties_ranked_by_exponent", ties)
    for k in (5, 17, 40, 100):
        h = np.zeros(256, np.int64)
        idx = rng.choice(256, k, replace=False)
        h[idx] = rng.integers(1, 1000, k)
        add(f"random_{k}_exponents", h)
    add("all_256", rng.integers(1, 50, 256))
    # real-size plane: K = N(0,1) * logU(0.1, 10) per channel, 16 M words
    words = 1 << 24
    scale = np.exp(rng.uniform(np.log(0.1), np.log(10.0), 1024))
    k = rng.standard_normal(words).astype(np.float32) * np.tile(scale, words // 1024)
    add("k_plane_16m_words", np.bincount(bf16_exponents(k), minlength=256))
    v = (rng.standard_normal(words) * 0.5).astype(np.float32)
    add("v_plane_16m_words", np.bincount(bf16_exponents(v), minlength=256))
    huge = np.zeros(256, np.int64)
    huge[[120, 121, 122, 123, 124]] = [3 << 40, 1 << 40, 1 << 38, 7, 1]
    add("huge_counts", huge)
    return cases


def main() -> None:
    sys.path.insert(0, str(REFERENCE / "src"))
    from unchain_kv.trace import summarize_symbol_counts  # noqa: E402

    rows = []
    for name, hist in histograms():
        rows.append({"name": name, "histogram": hist,
                     "summary": summarize_symbol_counts(hist)})
    OUT.write_text(json.dumps({"source": "src/unchain_kv/trace.py:27-58", "cases": rows},
                              indent=None, sort_keys=True) + "\n")
    print(f"wrote {len(rows)} cases to {OUT.name}")


if __name__ == "__main__":
    main()
