"""Payload formats of the splitzip bf16 KV codec: closed-form sizes, the Top-16
lookup table, and the canonical comparison of Top-16 payloads.

Sizes follow native/unchain_kv/kvq_splitzip_cuda.cu:300-303 (fixed6/fixed5) and
:389-391 (Top-16); the table follows src/unchain_kv/splitzip_cuda.py:290-297.
"""

from __future__ import annotations

MODE_PALETTE = 0    # torch-op codecs of the reference connector (restore only)
MODE_NIBBLES = 1
MODE_SIGNMAG = 2
MODE_FIXED6 = 3
MODE_FIXED5 = 4
MODE_TOP16 = 5
MODE_RAW = 6
MODE_OVERFLOW = 255


def torchop_encoded_size(header, n: int) -> int | None:
    """Size a mode 0, 1 or 2 payload of n words must have, from its first bytes, or
    None when the header itself is refused (the restore checks of
    src/unchain_kv/vllm_connector.py:5168-5252)."""
    view = memoryview(header).cast("B")
    if len(view) < 1:
        return None
    mode = view[0]
    if mode == MODE_PALETTE:
        if len(view) < 258 or not 1 <= view[1] < 8:
            return None
        return 258 + n + (n * view[1] + 7) // 8
    if mode == MODE_NIBBLES:
        if len(view) < 69 or any(w not in (1, 2, 4) for w in view[1:5]):
            return None
        return 69 + sum((n * w + 7) // 8 for w in view[1:5])
    if mode == MODE_SIGNMAG:
        if len(view) < 3 or not 1 <= view[1] < 7:
            return None
        return 3 + n + (n + 7) // 8 + (n * view[1] + 7) // 8
    return None


def top16_escape_capacity(n: int) -> int:
    """Escape slots of an n-word Top-16 payload: ceil(n / 200)."""
    return (n + 199) // 200


def top16_encoded_size(n: int) -> int:
    """5-byte header + n body bytes + ceil(n/2) code bytes + 5 bytes per slot."""
    return 5 + n + (n + 1) // 2 + 5 * top16_escape_capacity(n)


def fixed6_encoded_size(n: int) -> int:
    return 65 + n + ((n + 3) // 4) * 3


def fixed5_encoded_size(n: int) -> int:
    return 33 + n + ((n + 7) // 8) * 5


def palette_encoded_size(n: int, bits: int) -> int:
    """fixed6 (bits 6) or fixed5 (bits 5) payload size."""
    if bits == 6:
        return fixed6_encoded_size(n)
    if bits == 5:
        return fixed5_encoded_size(n)
    raise ValueError("palette codecs have 5 or 6 bits")


def palette_header_bytes(bits: int) -> int:
    return 65 if bits == 6 else 33


def top16_ratio(n: int) -> float:
    return 2 * n / top16_encoded_size(n)


def top16_tables(codebooks: bytes) -> bytes:
    """544-byte table for one layer: ``[p*256 + exponent] -> code`` (255 when the
    exponent is not in plane p's codebook; for a repeated exponent the later code
    wins), followed by the 32 codebook bytes (16 K exponents, then 16 V)."""
    codebooks = bytes(codebooks)
    if len(codebooks) != 32:
        raise ValueError("a Top-16 layer codebook is 32 bytes")
    table = bytearray(b"\xff" * 512)
    for plane in range(2):
        for code in range(16):
            table[plane * 256 + codebooks[plane * 16 + code]] = code
    return bytes(table) + codebooks


def top16_sections(n: int) -> dict[str, tuple[int, int]]:
    """Byte ranges of the payload sections."""
    body = (5, 5 + n)
    codes = (body[1], body[1] + (n + 1) // 2)
    escapes = (codes[1], codes[1] + 5 * top16_escape_capacity(n))
    return {"header": (0, 5), "body": body, "codes": codes, "escapes": escapes}


def top16_escapes(payload, n: int) -> list[tuple[int, int]]:
    """The (position, exponent) entries a decoder applies: the first
    min(count, capacity) slots."""
    view = memoryview(payload).cast("B")
    count = min(int.from_bytes(view[1:5], "little"), top16_escape_capacity(n))
    at = top16_sections(n)["escapes"][0]
    entries = []
    for slot in range(count):
        e = at + 5 * slot
        entries.append((int.from_bytes(view[e:e + 4], "little"), int(view[e + 4])))
    return entries


def top16_equivalent(a, b, n: int) -> bool:
    """True when two Top-16 payloads are the same up to what the reference encoder
    leaves to chance: escape order (compared as a set) and unused slot bytes.
    For an overflowed payload (byte 0 == 255) the escape slots hold an arbitrary
    subset of the escapes, so only the header, body and codes are compared."""
    va, vb = memoryview(a).cast("B"), memoryview(b).cast("B")
    size = top16_encoded_size(n)
    if len(va) < size or len(vb) < size:
        return False
    end = top16_sections(n)["codes"][1]
    if bytes(va[:end]) != bytes(vb[:end]):
        return False
    if va[0] == MODE_OVERFLOW:
        return True
    return sorted(top16_escapes(va, n)) == sorted(top16_escapes(vb, n))
