#!/usr/bin/env python3
"""Write the golden fixtures for the splitzip Top-16 codec tests.

Run where the reference checkout is at /root/reference (the tests only read the
files it writes). It reads reference files as text only (nothing from the
reference is imported or executed) and writes small data files next to itself:

* top16_codebooks.bin   -- the 1024-byte embedded codebook table, parsed from the
                           hex literal at src/unchain_kv/splitzip_cuda.py:11-31.
* kat_top16_256.json    -- the 256-word Top-16 payload <-> words known answer,
                           rebuilt by the construction in
                           tests/test_vllm_connector.py:333-372 (and :2723-2780).
* kat_sizes.json        -- payload-size known answers: the 32k-token constant of
                           scripts/bench_bandwidth_replay.py:20-21 and
                           tests/test_bench_bandwidth_replay.py:30-31.
* kat_fit.json          -- the codebook-fit known answer of
                           tests/test_extract_llama_top16_codebooks.py:15-38.
* kat_abi_calls.json    -- the C-ABI argument tuples pinned by
                           tests/test_splitzip_cuda.py:87-89, 247, 330-335.
"""

from __future__ import annotations

import hashlib
import json
import re
from pathlib import Path

REFERENCE = Path("/root/reference")
HERE = Path(__file__).resolve().parent


def codebooks_from_reference_text() -> bytes:
    text = (REFERENCE / "src/unchain_kv/splitzip_cuda.py").read_text(encoding="utf-8")
    match = re.search(r'_TOP16_CODEBOOKS = bytes\.fromhex\(\s*"""(.*?)"""', text, re.S)
    if match is None:
        raise SystemExit("codebook literal not found")
    return bytes.fromhex(match.group(1))


def kat_256(codebooks: bytes) -> dict:
    # Construction of tests/test_vllm_connector.py:341-367, restated.
    count = 256
    books = codebooks[:32]
    words = []
    body = bytearray(count)
    codes = bytearray((count + 1) // 2)
    escape_position, escape_exponent = 3, 100
    for index in range(count):
        plane = index >= count // 2
        code = index % 16
        exponent = books[plane * 16 + code]
        if index == escape_position:
            exponent, code = escape_exponent, 0
        word = ((index % 2) << 15) | (exponent << 7) | (index % 128)
        words.append(word)
        body[index] = (word & 0x7F) | ((word >> 8) & 0x80)
        codes[index // 2] |= code << ((index % 2) * 4)
    capacity = (count + 199) // 200
    payload = bytearray(5 + count + len(codes) + capacity * 5)
    payload[0] = 5
    payload[1:5] = (1).to_bytes(4, "little")
    payload[5 : 5 + count] = body
    payload[5 + count : 5 + count + len(codes)] = codes
    entry = 5 + count + len(codes)
    payload[entry : entry + 4] = escape_position.to_bytes(4, "little")
    payload[entry + 4] = escape_exponent
    raw = b"".join(word.to_bytes(2, "little") for word in words)
    return {
        "source": "tests/test_vllm_connector.py:333-372",
        "layer": 0,
        "count_words": count,
        "raw_bytes": count * 2,
        "payload_hex": bytes(payload).hex(),
        "raw_hex": raw.hex(),
    }


def sizes() -> dict:
    text = (REFERENCE / "scripts/bench_bandwidth_replay.py").read_text(encoding="utf-8")
    raw = int(re.search(r"RAW_LAYER_BYTES_32K = ([0-9_]+)", text).group(1).replace("_", ""))
    top16 = int(re.search(r"TOP16_LAYER_BYTES_32K = ([0-9_]+)", text).group(1).replace("_", ""))
    return {
        "source": "scripts/bench_bandwidth_replay.py:20-21; tests/test_bench_bandwidth_replay.py:30-31",
        "tokens": 32000,
        "kv_heads": 4,
        "head_dim": 128,
        "raw_bytes": raw,
        "top16_bytes": top16,
    }


def fit() -> dict:
    histogram = [0] * 256
    for exponent in range(16):
        histogram[exponent] = 16 - exponent
    return {
        "source": "tests/test_extract_llama_top16_codebooks.py:15-38",
        "histogram": histogram,
        "layers": [28, 29, 30, 31],
        "extension_bytes": 128,
        "first_codebook_hex": bytes(range(16)).hex(),
    }


def abi_calls() -> dict:
    return {
        "source": "tests/test_splitzip_cuda.py:63-89, 226-247, 302-336",
        "encode_top16": {
            "source": {"ptr": 11, "shape": [8], "stride": [1], "dtype": "bfloat16"},
            "out": {"ptr": 22, "shape": [32], "stride": [1], "dtype": "uint8"},
            "tables_ptr": 44,
            "stream": 99,
            "layer": 7,
            "expected_call": [11, 22, 8, 32, 44, 99],
        },
        "decode_top16": {
            "source": {"ptr": 22, "shape": [32], "stride": [1], "dtype": "uint8"},
            "target": {"ptr": 33, "shape": [2, 8, 2], "stride": [16, 2, 1], "dtype": "bfloat16"},
            "block_ids": [3, 4],
            "raw_bytes": 16,
            "expected_call": [22, 32, 33, 8, 2, 2, 16, 2, 3, 44, 99],
        },
        "decode_fixed6": {
            "source": {"ptr": 11, "shape": [79], "stride": [1], "dtype": "uint8"},
            "target": {"ptr": 22, "shape": [2, 8, 2], "stride": [16, 2, 1], "dtype": "bfloat16"},
            "block_ids": [3, 4],
            "raw_bytes": 16,
            "expected_call": [11, 79, 22, 8, 2, 2, 16, 2, 3, 99],
        },
        "noncontiguous": {
            "block_ids": [3, 5],
            "block_map_ptr": 55,
            "expected_fixed6_blocks_call": [11, 79, 22, 8, 2, 2, 16, 2, 3, 55, 99],
            "expected_top16_blocks_call": [11, 79, 22, 8, 2, 2, 16, 2, 3, 55, 44, 99],
        },
    }


def main() -> None:
    codebooks = codebooks_from_reference_text()
    (HERE / "top16_codebooks.bin").write_bytes(codebooks)
    print("codebooks", len(codebooks), hashlib.sha256(codebooks).hexdigest())
    for name, data in (
        ("kat_top16_256.json", kat_256(codebooks)),
        ("kat_sizes.json", sizes()),
        ("kat_fit.json", fit()),
        ("kat_abi_calls.json", abi_calls()),
    ):
        (HERE / name).write_text(json.dumps(data, indent=1, sort_keys=True) + "\n", encoding="utf-8")
        print("wrote", name)


if __name__ == "__main__":
    main()
