#!/usr/bin/env python3
"""Write reference-produced fixtures for the torch-op payload formats (modes 0/1/2).

Run in the build container only, where the reference checkout is at
/root/reference. Unlike ``make_golden.py`` this script imports the reference's
connector (src/unchain_kv/vllm_connector.py, pure Python + torch on the CPU):
its torch-op encoders (vllm_connector.py:3204-3343), their bit-packing helpers
(:3345-3404) and the restore decoders (:5168-5252) are pinned by nothing else --
the reference's own tests only round-trip them (tests/test_vllm_connector.py:
2437-2549) and hold no payload bytes. Nothing of the reference is written out:
only inputs and the outputs it produced, as data, in ``torchop_payloads.npz``
(numpy arrays, no pickled objects) and the case index ``torchop_cases.json``.

Cases (all seeded):

* ``encode``: gathered KV words of shape (2, blocks, block_words) through the
  connector's codec choice (``_splitzip_bf16_native_blocks`` with the native
  codec off): sign/magnitude (mode 2) at magnitude widths 1-6, the high-byte
  palette (mode 0) at widths 1-7, the nibble planes (mode 1) with each of the
  widths 1, 2, 4 on each plane, inputs that nothing compresses (recorded as
  declined), odd block words (partial final bytes) and a block span that does
  not start at block 0. Each payload is then restored through
  ``_copy_splitzip_bf16_native_blocks`` and the restored words recorded.
* ``decode``: payloads that no encoder writes (arbitrary codes and palettes,
  garbage in the unused palette bytes, magnitudes above 127 after the offset is
  added, headers the restore refuses) through the restore decoders alone.
* ``pack``: ``_pack_splitzip_bits`` and ``_unpack_splitzip_bits`` at widths 1-7
  and odd code counts.
"""

from __future__ import annotations

import json
import os
import sys
import tempfile
from pathlib import Path
from types import SimpleNamespace

import numpy as np

REFERENCE = Path("/root/reference")
HERE = Path(__file__).resolve().parent
NPZ = HERE / "torchop_payloads.npz"
INDEX = HERE / "torchop_cases.json"


def connector():
    sys.path.insert(0, str(REFERENCE / "src"))
    from unchain_kv.vllm_connector import UnchainKVConnector  # noqa: E402

    tmp = tempfile.mkdtemp(prefix="torchop_golden_")
    os.environ["UNCHAIN_KV_TRACE"] = str(Path(tmp) / "trace.jsonl")
    os.environ["UNCHAIN_KV_CODEC"] = "splitzip_bf16"
    os.environ["UNCHAIN_KV_CODEC_GPU_SLOTS"] = "1"
    for name in ("UNCHAIN_KV_SPLITZIP_TOP16", "UNCHAIN_KV_SPLITZIP_NATIVE_DECODE",
                 "UNCHAIN_KV_SPLITZIP_FIXED5"):
        os.environ.pop(name, None)
    config = SimpleNamespace(kv_transfer_config=SimpleNamespace(kv_role="kv_producer"))
    return UnchainKVConnector(config, "worker")


# --------------------------------------------------------------------------- inputs

def words_from_high(rng, high):
    low = rng.integers(0, 256, high.size)
    return ((high.astype(np.uint16) << 8) | low.astype(np.uint16)).astype(np.uint16)


def signmag_input(rng, n, width, mag_min):
    """High bytes whose magnitudes span exactly ``width`` bits above ``mag_min``
    (both ends present), random signs."""
    span = (1 << width) - 1
    mag = rng.integers(mag_min, mag_min + span + 1, n)
    mag[0], mag[-1] = mag_min, mag_min + span
    sign = rng.integers(0, 2, n)
    return words_from_high(rng, (sign << 7) | mag)


def palette_input(rng, n, k):
    """k distinct high bytes whose magnitudes span >= 64 (so sign/magnitude needs
    width 7 and declines); every palette entry used."""
    while True:
        pal = rng.choice(256, k, replace=False)
        mags = pal & 0x7F
        if mags.max() - mags.min() >= 64:
            break
    codes = rng.integers(0, k, n)
    codes[:k] = rng.permutation(k)
    return words_from_high(rng, pal[codes])


def nibble_input(rng, n, sizes):
    """Nibble p drawn from ``sizes[p]`` distinct values (every one present), redrawn
    until the high bytes' magnitudes span >= 64 (sign/magnitude then declines)."""
    for _ in range(1000):
        planes = []
        for k in sizes:
            values = np.sort(rng.choice(16, k, replace=False))
            idx = rng.integers(0, k, n)
            idx[:k] = rng.permutation(k)
            planes.append(values[idx].astype(np.uint16))
        words = (planes[0] | planes[1] << 4 | planes[2] << 8 | planes[3] << 12).astype(np.uint16)
        if mag_width(words) >= 7:
            return words
    raise SystemExit(f"no nibble input with a wide magnitude for {sizes}")


def mag_width(words):
    mag = (words >> 8) & 0x7F
    return max(1, int(mag.max() - mag.min()).bit_length())


# --------------------------------------------------------------------------- runs

def encode_case(conn, torch, words, nblk, bw, start=0, pool=None):
    """Gather ``nblk`` blocks starting at ``start`` from a layer of ``pool`` blocks
    holding ``words`` there (K plane then V plane), encode, restore."""
    pool = pool or (start + nblk)
    layer = np.zeros((2, pool, bw), np.uint16)
    layer[:, start:start + nblk] = words.reshape(2, nblk, bw)
    kv = torch.from_numpy(layer.view(np.int16)).view(torch.bfloat16)
    ids = list(range(start, start + nblk))
    encoded = conn._splitzip_bf16_native_blocks(kv, ids)
    # the one codec buffer slot goes back to the pool, as after a send
    conn._release_pending_codec_buffers()
    if encoded is None:
        return None, None
    data, _, raw_bytes, encoded_bytes, _ = encoded
    payload = np.frombuffer(bytes(data), np.uint8).copy()
    assert payload.size == encoded_bytes and raw_bytes == 2 * words.size
    target = torch.zeros_like(kv)
    restored, copied = conn._copy_splitzip_bf16_native_blocks(
        target, ids, [bytes(payload)],
        {"raw_bytes": raw_bytes, "encoded_bytes": encoded_bytes, "codec": "splitzip_bf16"})
    assert (restored, copied) == (nblk, raw_bytes), (restored, copied)
    got = target.view(torch.int16).numpy().view(np.uint16)[:, start:start + nblk].reshape(-1)
    return payload, got.copy()


def decode_case(conn, torch, payload, nblk, bw):
    kv = torch.zeros((2, nblk, bw), dtype=torch.bfloat16)
    raw_bytes = 2 * 2 * nblk * bw
    restored, copied = conn._copy_splitzip_bf16_native_blocks(
        kv, list(range(nblk)), [bytes(payload)],
        {"raw_bytes": raw_bytes, "encoded_bytes": int(payload.size)})
    if (restored, copied) == (0, 0):
        return None
    assert (restored, copied) == (nblk, raw_bytes)
    return kv.view(torch.int16).numpy().view(np.uint16).reshape(-1).copy()


def main() -> None:
    import torch

    conn = connector()
    arrays: dict[str, np.ndarray] = {}
    cases: list[dict] = []

    def add(kind, name, words, payload, out, **meta):
        key = f"c{len(cases):03d}"
        mode = None if kind == "pack" or payload is None else int(payload[0])
        if words is not None:
            arrays[f"{key}_words"] = words
        if payload is not None:
            arrays[f"{key}_payload"] = payload
        if out is not None:
            arrays[f"{key}_out"] = out
        cases.append({"key": key, "kind": kind, "name": name, "mode": mode,
                      "declined": out is None, **meta})

    rng = np.random.default_rng(20261202)

    def run_encode(name, words, nblk, bw, start=0, pool=None, expect=None):
        payload, out = encode_case(conn, torch, words, nblk, bw, start, pool)
        if expect is not None:
            got = None if payload is None else int(payload[0])
            assert got == expect, (name, got, expect)
        if payload is not None:
            assert np.array_equal(out, words), name
        add("encode", name, words, payload, out, n=int(words.size), blocks=nblk,
            block_words=bw, start=start)

    # mode 2, magnitude widths 1..6 (a constant magnitude is width 1 too)
    for width in range(1, 7):
        for nblk, bw in ((4, 96), (3, 7)):
            n = 2 * nblk * bw
            mag_min = int(rng.integers(0, 128 - (1 << width) + 1))
            words = signmag_input(rng, n, width, mag_min)
            assert mag_width(words) == width
            run_encode(f"signmag_w{width}_bw{bw}", words, nblk, bw, expect=2)
    high = np.full(200, 0x3F)
    high[::3] |= 0x80
    run_encode("signmag_constant_magnitude", words_from_high(rng, high), 4, 25, expect=2)

    # mode 0, palette widths 1..7 (sizes 2, 3-4, ..., 65-128)
    for width in range(1, 8):
        k_lo, k_hi = (2, 2) if width == 1 else ((1 << (width - 1)) + 1, 1 << width)
        for k, (nblk, bw) in ((k_lo, (9, 131)), (k_hi, (12, 128))):
            n = 2 * nblk * bw
            if 258 + n + (n * width + 7) // 8 >= 2 * n:
                nblk = (258 * 8 // (8 - width)) // (2 * bw) + 2
                n = 2 * nblk * bw
            words = palette_input(rng, n, k)
            run_encode(f"palette_w{width}_k{k}_bw{bw}", words, nblk, bw, expect=0)

    # mode 1: nibble planes; small n declines the palette by size, large n by
    # more than 128 distinct high bytes
    for sizes, nblk, bw in (((2, 3, 16, 2), 2, 64), ((3, 2, 2, 16), 2, 64),
                            ((16, 1, 9, 2), 2, 63), ((1, 16, 2, 4), 2, 64), ((2, 4, 3, 2), 2, 64),
                            ((2, 2, 16, 16), 8, 128), ((4, 1, 16, 12), 8, 127),
                            ((3, 4, 12, 16), 6, 101)):
        words = nibble_input(rng, 2 * nblk * bw, sizes)
        run_encode("nibbles_" + "_".join(map(str, sizes)) + f"_bw{bw}", words, nblk, bw,
                   expect=1)

    # nothing compresses: declined (no payload)
    run_encode("incompressible_small", rng.integers(0, 1 << 16, 12).astype(np.uint16), 2, 3)
    run_encode("incompressible_random", rng.integers(0, 1 << 16, 2048).astype(np.uint16),
               8, 128)

    # a block span that does not start at block 0 (contiguous gather, vllm_connector.py:2834-2837)
    run_encode("signmag_span_start_5", signmag_input(rng, 2 * 3 * 64, 4, 40), 3, 64,
               start=5, pool=11, expect=2)
    run_encode("palette_span_start_3", palette_input(rng, 2 * 6 * 128, 20), 6, 128,
               start=3, pool=12, expect=0)

    # decoders on payloads no encoder writes
    def rand_payload_mode0(n, width, garbage):
        pal = rng.integers(0, 256, 256).astype(np.uint8)
        if not garbage:
            pal[1 << width:] = 0
        codes = rng.integers(0, 1 << width, n)
        head = np.concatenate([np.array([0, width], np.uint8), pal])
        return np.concatenate([head, rng.integers(0, 256, n).astype(np.uint8),
                               conn_pack(codes, width)])

    def rand_payload_mode1(n, widths, garbage):
        head = np.zeros(69, np.uint8)
        head[0] = 1
        head[1:5] = widths
        planes = []
        for p, w in enumerate(widths):
            pal = rng.integers(0, 16, 16).astype(np.uint8)
            if garbage:
                pal = rng.integers(0, 256, 16).astype(np.uint8)
            head[5 + 16 * p:21 + 16 * p] = pal
            planes.append(conn_pack(rng.integers(0, 1 << w, n), w))
        return np.concatenate([head] + planes)

    def rand_payload_mode2(n, width, mag_min):
        sign = rng.integers(0, 2, n)
        mag = rng.integers(0, 1 << width, n)
        return np.concatenate([np.array([2, width, mag_min], np.uint8),
                               rng.integers(0, 256, n).astype(np.uint8),
                               conn_pack(sign, 1), conn_pack(mag, width)])

    def conn_pack(codes, width):
        codes = torch.as_tensor(np.asarray(codes, np.uint8))
        out = torch.empty(((codes.numel() * width + 7) // 8,), dtype=torch.uint8)
        conn._pack_splitzip_bits(codes, width, out, torch)
        return out.numpy().copy()

    for width in (1, 3, 5, 7):
        for garbage in (False, True):
            nblk, bw = 3, 37
            payload = rand_payload_mode0(2 * nblk * bw, width, garbage)
            add("decode", f"mode0_w{width}_{'garbage' if garbage else 'clean'}", None,
                payload, decode_case(conn, torch, payload, nblk, bw), n=2 * nblk * bw,
                blocks=nblk, block_words=bw)
    for widths in ((4, 4, 4, 4), (1, 2, 4, 1), (2, 1, 1, 2)):
        for garbage in (False, True):
            nblk, bw = 2, 29
            payload = rand_payload_mode1(2 * nblk * bw, widths, garbage)
            add("decode", f"mode1_{''.join(map(str, widths))}_{'garbage' if garbage else 'clean'}",
                None, payload, decode_case(conn, torch, payload, nblk, bw), n=2 * nblk * bw,
                blocks=nblk, block_words=bw)
    for width, mag_min in ((1, 0), (3, 200), (6, 255), (6, 100), (4, 127)):
        nblk, bw = 2, 41
        payload = rand_payload_mode2(2 * nblk * bw, width, mag_min)
        add("decode", f"mode2_w{width}_min{mag_min}", None, payload,
            decode_case(conn, torch, payload, nblk, bw), n=2 * nblk * bw, blocks=nblk,
            block_words=bw)
    # headers the restore refuses
    nblk, bw = 2, 41
    n = 2 * nblk * bw
    good2 = rand_payload_mode2(n, 3, 10)
    good0 = rand_payload_mode0(n, 3, False)
    good1 = rand_payload_mode1(n, (1, 2, 4, 1), False)
    refusals = {
        "refuse_mode2_width0": np.concatenate([[2, 0, 10], good2[3:]]).astype(np.uint8),
        "refuse_mode2_width7": np.concatenate([[2, 7, 10], good2[3:],
                                               np.zeros((n * 4 + 7) // 8, np.uint8)]).astype(np.uint8),
        "refuse_mode2_short": good2[:-1],
        "refuse_mode0_width0": np.concatenate([[0, 0], good0[2:]]).astype(np.uint8),
        "refuse_mode0_width8": np.concatenate([[0, 8], good0[2:],
                                               np.zeros(n - (n * 3 + 7) // 8, np.uint8)]).astype(np.uint8),
        "refuse_mode0_long": np.concatenate([good0, [0]]).astype(np.uint8),
        "refuse_mode1_width3": np.concatenate([[1, 3], good1[2:]]).astype(np.uint8),
        "refuse_mode1_short": good1[:-1],
        "refuse_mode7": np.concatenate([[7], good2[1:]]).astype(np.uint8),
    }
    for name, payload in refusals.items():
        got = decode_case(conn, torch, payload, nblk, bw)
        assert got is None, name
        add("decode", name, None, payload, None, n=n, blocks=nblk, block_words=bw)

    # the bit-packing helpers at odd counts
    for width in range(1, 8):
        for count in (1, 7, 13, 333):
            codes = rng.integers(0, 1 << width, count).astype(np.uint8)
            packed = conn_pack(codes, width)
            unpacked = conn._unpack_splitzip_bits(torch.from_numpy(packed), count, width, torch)
            unpacked = unpacked.numpy().copy()
            assert np.array_equal(unpacked, codes)
            add("pack", f"pack_w{width}_c{count}", codes, packed, unpacked, n=count,
                width=width)

    np.savez_compressed(NPZ, **arrays)
    INDEX.write_text(json.dumps({"source": "src/unchain_kv/vllm_connector.py:3204-3404,5168-5252",
                                 "cases": cases}, indent=1) + "\n")
    modes = {}
    for c in cases:
        modes[(c["kind"], c["mode"])] = modes.get((c["kind"], c["mode"]), 0) + 1
    print(f"wrote {len(cases)} cases to {NPZ.name} ({NPZ.stat().st_size} B): {modes}")


if __name__ == "__main__":
    main()
