"""The torch-op payload formats (modes 0, 1, 2) against fixtures the reference
produced: the connector's own encoders (src/unchain_kv/vllm_connector.py:
3204-3343), bit-packing helpers (:3345-3404) and restore decoders (:5168-5252),
run on the CPU by ``tests/golden/make_torchop_golden.py``.

Pins: every encoder payload byte for byte (mode choice, header, palettes, section
order, LSB-first packing, partial final bytes, declines); the decoders on payloads
no encoder writes (unsorted and garbage palettes, magnitudes past 127 once the
offset is added, nibble palettes with bytes above 15 that spill into the next
plane) and on headers the restore refuses; the bit helpers at odd counts. The
host's size check (``codec_format.torchop_encoded_size``) accepts exactly the
payloads the reference restores. Planted mistakes (most-significant-bit-first
packing, a palette one entry off, swapped mode-2 header fields) fail the
fixtures."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_cases():
    index = json.loads((GOLDEN / "torchop_cases.json").read_text())
    with np.load(GOLDEN / "torchop_payloads.npz") as z:
        arrays = {k: z[k] for k in z.files}
    cases = []
    for c in index["cases"]:
        c = dict(c)
        for part in ("words", "payload", "out"):
            c[part] = arrays.get(f"{c['key']}_{part}")
        cases.append(c)
    return cases


CASES = load_cases()
ENCODE = [c for c in CASES if c["kind"] == "encode"]
DECODE = [c for c in CASES if c["kind"] == "decode"]
PACK = [c for c in CASES if c["kind"] == "pack"]


def test_fixture_coverage():
    modes = {c["mode"] for c in ENCODE if not c["declined"]}
    assert modes == {0, 1, 2}
    widths = {(c["mode"], int(c["payload"][1])) for c in ENCODE if c["mode"] in (0, 2)}
    assert {(2, w) for w in range(1, 7)} <= widths
    assert {(0, w) for w in range(1, 8)} <= widths
    plane_widths = {(p, int(c["payload"][1 + p])) for c in ENCODE if c["mode"] == 1
                    for p in range(4)}
    assert plane_widths == {(p, w) for p in range(4) for w in (1, 2, 4)}
    assert any(c["declined"] for c in ENCODE)
    assert any(c["start"] > 0 for c in ENCODE)
    assert any(c["n"] * 3 % 8 for c in ENCODE)             # partial final bytes
    assert sum(1 for c in DECODE if c["declined"]) >= 8
    assert {c["n"] % 8 for c in PACK} >= {1, 5, 7}


@pytest.mark.parametrize("case", ENCODE, ids=[c["name"] for c in ENCODE])
def test_encoder_matches_reference_bytes(case):
    got = oracle.encode_torchop(case["words"])
    if case["declined"]:
        assert got is None
        return
    assert got is not None
    assert got.dtype == np.uint8
    assert bytes(got) == bytes(case["payload"])


@pytest.mark.parametrize("case", ENCODE + DECODE, ids=[c["name"] for c in ENCODE + DECODE])
def test_decoder_matches_reference_words(case):
    if case["payload"] is None:
        return
    got = oracle.decode_torchop(case["payload"], case["n"])
    if case["declined"]:
        assert got is None
    else:
        assert np.array_equal(got, case["out"])


@pytest.mark.parametrize("case", ENCODE + DECODE, ids=[c["name"] for c in ENCODE + DECODE])
def test_host_size_check_accepts_what_the_reference_restores(case):
    payload = case["payload"]
    if payload is None:
        return
    size = codec_format.torchop_encoded_size(bytes(payload[:258]), case["n"])
    assert (size == payload.size) == (not case["declined"])


@pytest.mark.parametrize("case", PACK, ids=[c["name"] for c in PACK])
def test_bit_helpers_match_reference(case):
    codes, width, count = case["words"], case["width"], case["n"]
    assert bytes(oracle.pack_bits_lsb(codes, width)) == bytes(case["payload"])
    assert np.array_equal(oracle.unpack_bits_lsb(case["payload"], count, width), case["out"])


def test_planted_msb_first_packing_fails(monkeypatch):
    def msb_first(codes, width):
        codes = np.asarray(codes, dtype=np.uint16).reshape(-1)
        bits = ((codes[:, None] >> np.arange(width)[::-1]) & 1).astype(np.uint8)
        return np.packbits(bits.reshape(-1), bitorder="little")

    monkeypatch.setattr(oracle, "pack_bits_lsb", msb_first)
    encoded = [c for c in ENCODE if not c["declined"]]
    wrong = [c for c in encoded if bytes(oracle.encode_torchop(c["words"])) != bytes(c["payload"])]
    # width-1 sections are the same either way, so an all-width-1 payload is not caught
    assert {c["mode"] for c in wrong} == {0, 1, 2}
    assert len(wrong) >= 0.8 * len(encoded)


def test_planted_palette_offset_and_header_swap_fail():
    pal = next(c for c in ENCODE if c["mode"] == 0 and c["payload"][1] >= 3)
    shifted = pal["payload"].copy()
    shifted[2:257] = pal["payload"][3:258]
    assert not np.array_equal(oracle.decode_torchop(shifted, pal["n"]), pal["out"])
    sm = next(c for c in ENCODE if c["mode"] == 2 and c["payload"][2] not in (0, c["payload"][1]))
    swapped = sm["payload"].copy()
    swapped[1], swapped[2] = sm["payload"][2], sm["payload"][1]
    got = oracle.decode_torchop(swapped, sm["n"])
    assert got is None or not np.array_equal(got, sm["out"])
