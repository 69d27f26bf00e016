#!/usr/bin/env python3
"""Write reference-produced fixtures for the CPU Top-16 decoder and the Top-16
lookup tables.

Run in the build container only, where the reference checkout is at
/root/reference. Like ``make_torchop_golden.py`` it imports reference modules on
the CPU: the connector's CPU Top-16 decoder ``_decode_splitzip_top16_payload``
(src/unchain_kv/vllm_connector.py:176-219) and ``_top16_tables`` with the embedded
codebooks (src/unchain_kv/splitzip_cuda.py:11-31, 283-298; a CPU tensor, the
native library is never loaded). Nothing of the reference is written out: only
inputs and the outputs it produced, as data, in ``top16_cpu_payloads.npz`` (numpy
arrays, no pickled objects) and the case index ``top16_cpu_cases.json``.

Cases (all seeded):

* ``tables``: the 544-byte table of every one of the 32 embedded layer codebooks.
* ``decode``: payloads with many escapes in shuffled order (the reference's
  encoder appends escapes in atomic order), random bytes in the unused escape
  slots, escapes at the first and last word of each plane, repeated positions
  (the later entry wins), an escape count at the capacity, and the payloads the
  decoder refuses (count above the capacity, a position past the words, a wrong
  length, mode 255, a raw size that is not a multiple of 4, a short codebook).
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

REFERENCE = Path("/root/reference")
HERE = Path(__file__).resolve().parent
NPZ = HERE / "top16_cpu_payloads.npz"
INDEX = HERE / "top16_cpu_cases.json"


def reference_modules():
    sys.path.insert(0, str(REFERENCE / "src"))
    from unchain_kv import splitzip_cuda  # noqa: E402
    from unchain_kv.vllm_connector import _decode_splitzip_top16_payload  # noqa: E402

    return splitzip_cuda, _decode_splitzip_top16_payload


def escape_capacity(n: int) -> int:
    return (n + 199) // 200


def build_payload(rng, n: int, positions, exponents, count_field=None, slot_fill=None):
    """A mode-5 payload of n words: random body and code bytes, the given escape
    entries in the given order, random bytes in the unused slots."""
    cap = escape_capacity(n)
    code_bytes = (n + 1) // 2
    out = bytearray(5 + n + code_bytes + 5 * cap)
    out[0] = 5
    count = len(positions) if count_field is None else count_field
    out[1:5] = int(count).to_bytes(4, "little")
    out[5:5 + n] = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
    out[5 + n:5 + n + code_bytes] = rng.integers(0, 256, code_bytes, dtype=np.uint8).tobytes()
    at = 5 + n + code_bytes
    fill = rng.integers(0, 256, 5 * cap, dtype=np.uint8).tobytes() if slot_fill is None else slot_fill
    out[at:at + 5 * cap] = fill
    for slot, (pos, exp) in enumerate(zip(positions, exponents)):
        out[at + 5 * slot:at + 5 * slot + 4] = int(pos).to_bytes(4, "little")
        out[at + 5 * slot + 4] = int(exp)
    return bytes(out)


def main() -> None:
    splitzip_cuda, decode = reference_modules()
    import torch

    books_all = bytes(splitzip_cuda._TOP16_CODEBOOKS)
    layers = len(books_all) // 32
    arrays: dict[str, np.ndarray] = {}
    cases: list[dict] = []

    tables = np.stack([
        splitzip_cuda._top16_tables(layer, "cpu", torch).numpy().astype(np.uint8)
        for layer in range(layers)])
    arrays["tables"] = tables
    arrays["codebooks"] = np.frombuffer(books_all, dtype=np.uint8).copy()

    rng = np.random.default_rng(20261202)

    def add(name, payload, raw_bytes, books, **meta):
        result = decode(payload, raw_bytes, books)
        key = f"c{len(cases)}"
        arrays[key + "_payload"] = np.frombuffer(payload, dtype=np.uint8).copy()
        arrays[key + "_books"] = np.frombuffer(books, dtype=np.uint8).copy()
        if result is not None:
            arrays[key + "_words"] = np.frombuffer(result, dtype=np.uint16).copy()
        cases.append({"name": name, "key": key, "raw_bytes": raw_bytes,
                      "decoded": result is not None, **meta})

    for n, layer in ((256, 0), (1000, 7), (4096, 13), (2 * 8 * 1024, 31), (10004, 22)):
        books = books_all[32 * layer:32 * layer + 32]
        cap = escape_capacity(n)
        half = n // 2
        # many escapes, distinct positions, shuffled; the plane edges included
        edges = [0, half - 1, half, n - 1][:cap]
        others = rng.choice(np.setdiff1d(np.arange(n), edges), size=cap - len(edges),
                            replace=False)
        pos = np.concatenate([edges, others])
        rng.shuffle(pos)
        exp = rng.integers(0, 256, pos.size)
        add(f"shuffled_full_n{n}", build_payload(rng, n, pos, exp), 2 * n, books,
            layer=layer, distinct=True, escapes=int(pos.size))
        # fewer escapes, unused slots random
        few = rng.choice(n, size=max(1, cap // 3), replace=False)
        add(f"shuffled_partial_n{n}", build_payload(rng, n, few, rng.integers(0, 256, few.size)),
            2 * n, books, layer=layer, distinct=True, escapes=int(few.size))
        # no escapes
        add(f"no_escapes_n{n}", build_payload(rng, n, [], []), 2 * n, books, layer=layer,
            distinct=True, escapes=0)
        # repeated positions: each later entry overrides the earlier one
        rep = rng.choice(n, size=max(1, cap // 4), replace=False)
        rep = np.concatenate([rep, rep[::-1]])[:cap]
        add(f"repeated_n{n}", build_payload(rng, n, rep, rng.integers(0, 256, rep.size)), 2 * n,
            books, layer=layer, distinct=False, escapes=int(rep.size))

    # refusals
    n, layer = 1000, 3
    books = books_all[32 * layer:32 * layer + 32]
    cap = escape_capacity(n)
    add("count_above_capacity", build_payload(rng, n, [1, 2], [9, 9], count_field=cap + 1), 2 * n,
        books, layer=layer, distinct=True, escapes=cap + 1)
    add("position_past_words", build_payload(rng, n, [3, n], [1, 2]), 2 * n, books, layer=layer,
        distinct=True, escapes=2)
    good = build_payload(rng, n, [5], [77])
    add("one_byte_short", good[:-1], 2 * n, books, layer=layer, distinct=True, escapes=1)
    add("one_byte_long", good + b"\0", 2 * n, books, layer=layer, distinct=True, escapes=1)
    over = bytearray(good)
    over[0] = 255
    add("mode_255", bytes(over), 2 * n, books, layer=layer, distinct=True, escapes=1)
    odd = build_payload(rng, 999, [4], [1])
    add("raw_bytes_not_multiple_of_4", odd, 2 * 999, books, layer=layer, distinct=True, escapes=1)
    add("short_codebook", good, 2 * n, books[:31], layer=layer, distinct=True, escapes=1)

    np.savez_compressed(NPZ, **arrays)
    INDEX.write_text(json.dumps({"layers": layers, "cases": cases}, indent=1) + "\n")
    print(f"wrote {len(cases)} decode cases and {layers} tables to {NPZ.name}")


if __name__ == "__main__":
    main()
