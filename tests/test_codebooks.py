"""Product codebook statistics and fit (unchainkv_amd.codebooks), on the CPU.

Pinned by the reference's extraction known answer
(tests/test_extract_llama_top16_codebooks.py:15-38: histogram 16 - e on exponents
0..15 for layers 28-31 gives bytes(range(16)) per plane, 128 bytes in all), by the
oracle's independent fit, and by closed forms of the summary fields."""

import json
import math

import numpy as np
import pytest

import oracle
from unchainkv_amd import codebooks as cb


def _rows(layers, k_hist, v_hist):
    return [{"event": "bf16_exponent_stats", "layer": layer, "k": {"histogram": k_hist},
             "v": {"histogram": v_hist}} for layer in layers]


def test_extract_known_answer(tmp_path):
    hist = [0] * 256
    for e in range(16):
        hist[e] = 16 - e
    trace = tmp_path / "trace.jsonl"
    trace.write_text("".join(json.dumps(r) + "\n" for r in _rows(range(28, 32), hist, hist)))
    result = cb.extract([trace], range(28, 32))
    assert result["passed"] and result["trace_rows"] == 4
    assert result["extension_bytes"] == 128
    assert result["extension_hex"] == bytes(range(16)).hex() * 8
    assert [entry["layer"] for entry in result["layers"]] == [28, 29, 30, 31]
    assert result["layers"][0]["k"] == {"words": sum(hist), "top16_exponents": list(range(16)),
                                       "coverage": 1.0}
    assert result["source_traces"] == [str(trace)]


def test_extract_sums_rows_and_skips_other_events(tmp_path):
    a = [0] * 256
    b = [0] * 256
    for e in range(20):
        a[100 + e] = 1          # ties: smaller exponent first
        b[100 + e] = 20 - e     # b alone ranks 100, 101, ...
    b[119] = 50                 # ... but in the sum 119 leads
    rows = _rows([3], a, a) + _rows([3], b, b) + [{"event": "other", "layer": 3}] + \
        _rows([4], a, a)
    trace = tmp_path / "t.jsonl"
    trace.write_text("".join(json.dumps(r) + "\n" for r in rows))
    result = cb.extract([trace], [3])
    summed = [x + y for x, y in zip(a, b)]
    assert result["trace_rows"] == 2
    assert bytes.fromhex(result["extension_hex"])[:16] == bytes(oracle.fit_top16_py(summed))
    assert bytes.fromhex(result["extension_hex"])[0] == 119
    with pytest.raises(ValueError):          # layer 5 has no rows, so no codebook
        cb.extract([trace], [3, 4, 5])


def test_fit_matches_oracle_on_random_histograms():
    rng = np.random.default_rng(5)
    for _ in range(200):
        hist = rng.integers(0, 6, 256) * (rng.random(256) < 0.3)
        expect = oracle.fit_top16_py(hist.tolist())
        if expect is None:
            with pytest.raises(ValueError):
                cb.fit_top16(hist)
        else:
            assert cb.fit_top16(hist) == list(expect)


def test_summary_closed_forms():
    hist = [0] * 256
    for e in (7, 9, 11, 13):
        hist[e] = 25
    s = cb.summarize_symbol_counts(hist)
    assert s["words"] == 100 and s["unique_exponents"] == 4
    assert math.isclose(s["entropy_bits"], 2.0)          # uniform over 4 symbols
    assert s["top8_exponents"] == [7, 9, 11, 13] and s["top16_escape_count"] == 0
    hist[200] = 300
    for e in range(20, 40):
        hist[e] = 1
    s = cb.summarize_symbol_counts(hist)
    assert s["top8_exponents"][:5] == [200, 7, 9, 11, 13]
    assert s["top8_exponents"][5:] == [20, 21, 22]
    assert s["top8_escape_count"] == 420 - (300 + 100 + 3)
    assert math.isclose(s["top16_coverage"], (300 + 100 + 11) / 420)
    empty = cb.summarize_symbol_counts([0] * 256)
    assert empty["words"] == 0 and empty["entropy_bits"] == 0.0 and empty["top8_exponents"] == []


def test_fit_rejects_bad_histograms():
    with pytest.raises(ValueError):
        cb.fit_top16([1] * 255)
    with pytest.raises(ValueError):
        cb.fit_layer_codebook([1] * 10 + [0] * 246, [1] * 256)
    assert cb.fit_layer_codebook([1] * 256, [0] * 100 + [1] * 156) == \
        bytes(range(16)) + bytes(range(100, 116))


def test_summary_matches_the_reference_trace_payload(golden_dir):
    """tests/golden/trace_summary_cases.json holds the reference's own
    summarize_symbol_counts (src/unchain_kv/trace.py:27-58) on 12 seeded
    histograms (empty, ties, all 256 exponents, 16 M-word planes, huge counts):
    every field equal, the entropy to the last bit."""
    import json

    cases = json.loads((golden_dir / "trace_summary_cases.json").read_text())["cases"]
    assert len(cases) == 12
    for case in cases:
        ours = json.loads(json.dumps(cb.summarize_symbol_counts(case["histogram"]),
                                     sort_keys=True))
        assert ours == case["summary"], case["name"]
        assert ours["entropy_bits"].hex() == case["summary"]["entropy_bits"].hex(), case["name"]
