"""The oracle's Top-16 decode and lookup tables against outputs the reference
produced (fixtures written by tests/golden/make_top16_cpu_golden.py from the
reference connector's CPU decoder, src/unchain_kv/vllm_connector.py:176-219, and
``_top16_tables``, src/unchain_kv/splitzip_cuda.py:283-298).

The payloads carry escape lists in shuffled order with random bytes in the unused
slots (what the reference's atomic-order encoder leaves), repeated positions, and
the payloads the CPU decoder refuses.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def golden():
    index = json.loads((GOLDEN / "top16_cpu_cases.json").read_text())
    with np.load(GOLDEN / "top16_cpu_payloads.npz") as data:
        arrays = {k: data[k] for k in data.files}
    return index, arrays


def _cases(golden, decoded=None):
    index, arrays = golden
    for case in index["cases"]:
        if decoded is None or case["decoded"] == decoded:
            yield case, arrays


def test_fixture_index_covers_the_advertised_cases(golden):
    index, arrays = golden
    names = {c["name"] for c in index["cases"]}
    assert {"count_above_capacity", "position_past_words", "one_byte_short", "one_byte_long",
            "mode_255", "raw_bytes_not_multiple_of_4", "short_codebook"} <= names
    assert sum(c["decoded"] for c in index["cases"]) == 20
    assert any(not c["distinct"] and c["decoded"] for c in index["cases"])
    assert arrays["tables"].shape == (index["layers"], 544)


def test_tables_of_every_embedded_codebook(golden):
    index, arrays = golden
    books = arrays["codebooks"].tobytes()
    shipped = Path(codec_format.__file__).resolve().parent / "data" / "llama_top16_codebooks.bin"
    assert shipped.read_bytes() == books
    assert (GOLDEN / "top16_codebooks.bin").read_bytes() == books
    for layer in range(index["layers"]):
        cb = books[32 * layer:32 * layer + 32]
        want = arrays["tables"][layer]
        assert np.array_equal(oracle.top16_tables(cb), want), layer
        assert oracle.top16_tables_py(cb) == want.tobytes(), layer
        assert codec_format.top16_tables(cb) == want.tobytes(), layer


def test_python_restatement_matches_every_case(golden):
    for case, arrays in _cases(golden):
        key = case["key"]
        payload = arrays[key + "_payload"].tobytes()
        books = arrays[key + "_books"].tobytes()
        got = oracle.decode_top16_payload_py(payload, case["raw_bytes"], books)
        if not case["decoded"]:
            assert got is None, case["name"]
        else:
            assert got is not None, case["name"]
            assert np.array_equal(np.frombuffer(got, dtype=np.uint16), arrays[key + "_words"]), \
                case["name"]


def test_c_restatement_matches_every_decoded_case(golden):
    for case, arrays in _cases(golden, decoded=True):
        key = case["key"]
        payload = arrays[key + "_payload"]
        n = case["raw_bytes"] // 2
        tables = oracle.top16_tables(arrays[key + "_books"].tobytes())
        got = oracle.top16_decode(payload, n, tables)
        assert np.array_equal(got, arrays[key + "_words"]), case["name"]


def test_planted_mistakes_fail_the_fixtures(golden):
    """Decoders with a plausible mistake disagree with the fixtures: escapes applied
    last-to-first (visible on repeated positions), the V plane read with the K
    codebook, and the sign bit dropped."""
    caught = {"reversed": 0, "one_book": 0, "sign": 0}
    for case, arrays in _cases(golden, decoded=True):
        key = case["key"]
        n = case["raw_bytes"] // 2
        payload = bytearray(arrays[key + "_payload"].tobytes())
        books = arrays[key + "_books"].tobytes()
        want = arrays[key + "_words"]
        count = int.from_bytes(payload[1:5], "little")
        at = 5 + n + (n + 1) // 2
        entries = [bytes(payload[at + 5 * s:at + 5 * s + 5]) for s in range(count)]
        rev = bytearray(payload)
        rev[at:at + 5 * count] = b"".join(entries[::-1])
        got = oracle.decode_top16_payload_py(bytes(rev), case["raw_bytes"], books)
        if not case["distinct"]:
            caught["reversed"] += not np.array_equal(np.frombuffer(got, np.uint16), want)
        one = oracle.decode_top16_payload_py(bytes(payload), case["raw_bytes"],
                                             books[:16] + books[:16])
        caught["one_book"] += not np.array_equal(np.frombuffer(one, np.uint16), want)
        nosign = np.frombuffer(oracle.decode_top16_payload_py(bytes(payload), case["raw_bytes"],
                                                              books), np.uint16) & 0x7FFF
        caught["sign"] += not np.array_equal(nosign, want)
    assert caught == {"reversed": 5, "one_book": 20, "sign": 20}
