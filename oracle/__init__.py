"""CPU oracle for the splitzip bf16 KV-cache codec.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` may import this package, and only to check
results against (or, for the baseline, as the timed CPU restatement). The product
package ``unchainkv_amd`` never imports it; its codec runs on the HIP library
and fails loudly when that library is missing.

Two restatements of the reference algorithm live here:

* ``splitzip_oracle.c`` (built to ``_build/libsplitzip_oracle.so``): the fast
  C restatement used at test sizes and as the multi-threaded CPU baseline.
* the pure-Python functions below, restated independently from the reference
  sources for brute-force cross-checks on small inputs.

Every function names the reference lines it follows. What pins each one (golden
vectors, closed forms, inverse properties, brute force) is tested in
``tests/test_oracle_golden.py``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libsplitzip_oracle.so"

_LIB = None


def build() -> Path:
    """Compile the C restatement (gcc, OpenMP) into ``_build/``."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load():
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    u64, p = ctypes.c_uint64, ctypes.c_void_p
    lib.sz_top16_escape_capacity.argtypes = [u64]
    lib.sz_top16_escape_capacity.restype = u64
    lib.sz_top16_encoded_size.argtypes = [u64]
    lib.sz_top16_encoded_size.restype = u64
    lib.sz_fixed6_encoded_size.argtypes = [u64]
    lib.sz_fixed6_encoded_size.restype = u64
    lib.sz_top16_tables.argtypes = [p, p]
    lib.sz_top16_tables.restype = None
    lib.sz_gather.argtypes = [p, u64, u64, u64, p, u64, p]
    lib.sz_gather.restype = None
    lib.sz_scatter.argtypes = [p, u64, u64, u64, u64, u64, u64, p, p]
    lib.sz_scatter.restype = None
    lib.sz_top16_encode.argtypes = [p, u64, p, p]
    lib.sz_top16_encode.restype = u64
    lib.sz_top16_decode.argtypes = [p, u64, p, p]
    lib.sz_top16_decode.restype = ctypes.c_int
    lib.sz_top16_decode_scatter.argtypes = [p, u64, p, u64, u64, u64, u64, u64, p, p]
    lib.sz_top16_decode_scatter.restype = ctypes.c_int
    lib.sz_exponent_histogram.argtypes = [p, u64, p]
    lib.sz_exponent_histogram.restype = None
    lib.sz_fixed6_encode.argtypes = [p, u64, p]
    lib.sz_fixed6_encode.restype = u64
    lib.sz_fixed6_decode.argtypes = [p, u64, p]
    lib.sz_fixed6_decode.restype = ctypes.c_int
    lib.sz_palette_encoded_size.argtypes = [u64, ctypes.c_int]
    lib.sz_palette_encoded_size.restype = u64
    lib.sz_palette_encode.argtypes = [p, u64, ctypes.c_int, p]
    lib.sz_palette_encode.restype = u64
    lib.sz_palette_decode.argtypes = [p, u64, ctypes.c_int, p]
    lib.sz_palette_decode.restype = ctypes.c_int
    lib.sz_top16_encode_paged_batch.argtypes = [
        p, u64, u64, u64, p, p, u64, p, p, p, u64, ctypes.c_int
    ]
    lib.sz_top16_encode_paged_batch.restype = ctypes.c_int
    lib.sz_top16_decode_paged_batch.argtypes = [
        p, p, u64, p, u64, u64, u64, p, p, p, u64, ctypes.c_int
    ]
    lib.sz_top16_decode_paged_batch.restype = ctypes.c_int
    _LIB = lib
    return lib


def _ptr(array: np.ndarray) -> int:
    return array.ctypes.data


# ---------------------------------------------------------------------------
# closed forms (kvq_splitzip_cuda.cu:389-391, :300-303)

def escape_capacity(n: int) -> int:
    return (n + 199) // 200


def top16_encoded_size(n: int) -> int:
    return 5 + n + (n + 1) // 2 + 5 * escape_capacity(n)


def fixed6_encoded_size(n: int) -> int:
    return 65 + n + ((n + 3) // 4) * 3


def palette_encoded_size(n: int, bits: int) -> int:
    return fixed6_encoded_size(n) if bits == 6 else 33 + n + ((n + 7) // 8) * 5


# ---------------------------------------------------------------------------
# C restatement wrappers (numpy in, numpy out)

def top16_tables(codebooks32: bytes) -> np.ndarray:
    cb = np.frombuffer(bytes(codebooks32), dtype=np.uint8).copy()
    if cb.size != 32:
        raise ValueError("a layer codebook is 32 bytes (16 K exponents, 16 V exponents)")
    out = np.empty(544, dtype=np.uint8)
    load().sz_top16_tables(_ptr(cb), _ptr(out))
    return out


def top16_encode(words: np.ndarray, tables: np.ndarray) -> np.ndarray | None:
    words = np.ascontiguousarray(words, dtype=np.uint16).reshape(-1)
    n = words.size
    out = np.zeros(top16_encoded_size(n), dtype=np.uint8)
    size = load().sz_top16_encode(_ptr(words), n, _ptr(np.ascontiguousarray(tables)), _ptr(out))
    return out if size else None


def top16_decode(payload: np.ndarray, n: int, tables: np.ndarray,
                 initial: np.ndarray | None = None) -> np.ndarray:
    """Words in payload order; when byte 0 != 5 the initial words come back unchanged."""
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    words = (np.zeros(n, dtype=np.uint16) if initial is None
             else np.array(initial, dtype=np.uint16).reshape(-1).copy())
    load().sz_top16_decode(_ptr(payload), n, _ptr(np.ascontiguousarray(tables)), _ptr(words))
    return words


def gather(kv: np.ndarray, plane_stride: int, block_stride: int, block_words: int,
           ids) -> np.ndarray:
    kv = np.ascontiguousarray(kv, dtype=np.uint16).reshape(-1)
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    out = np.empty(2 * ids.size * block_words, dtype=np.uint16)
    load().sz_gather(_ptr(kv), plane_stride, block_stride, block_words, _ptr(ids), ids.size,
                     _ptr(out))
    return out


def scatter(words: np.ndarray, kv: np.ndarray, block_count: int, block_words: int,
            plane_stride: int, block_stride: int, block_start: int = 0, ids=None) -> None:
    """In-place scatter of payload-order words into the flat uint16 array ``kv``."""
    words = np.ascontiguousarray(words, dtype=np.uint16)
    assert kv.dtype == np.uint16 and kv.flags.c_contiguous
    ids_arr = None if ids is None else np.ascontiguousarray(ids, dtype=np.int64)
    load().sz_scatter(_ptr(words), words.size, block_count, block_words, plane_stride,
                      block_stride, block_start, 0 if ids_arr is None else _ptr(ids_arr),
                      _ptr(kv))


def exponent_histogram(words: np.ndarray) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype=np.uint16).reshape(-1)
    counts = np.zeros(512, dtype=np.uint64)
    load().sz_exponent_histogram(_ptr(words), words.size, _ptr(counts))
    return counts.reshape(2, 256)


def fixed6_encode(words: np.ndarray) -> np.ndarray | None:
    words = np.ascontiguousarray(words, dtype=np.uint16).reshape(-1)
    out = np.zeros(fixed6_encoded_size(words.size), dtype=np.uint8)
    size = load().sz_fixed6_encode(_ptr(words), words.size, _ptr(out))
    return out if size else None


def fixed6_decode(payload: np.ndarray, n: int) -> np.ndarray:
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    words = np.zeros(n, dtype=np.uint16)
    load().sz_fixed6_decode(_ptr(payload), n, _ptr(words))
    return words


def palette_encode(words: np.ndarray, bits: int) -> np.ndarray | None:
    """fixed6 (bits 6, mode 3) or fixed5 (bits 5, mode 4) canonical payload."""
    words = np.ascontiguousarray(words, dtype=np.uint16).reshape(-1)
    out = np.zeros(palette_encoded_size(words.size, bits), dtype=np.uint8)
    size = load().sz_palette_encode(_ptr(words), words.size, bits, _ptr(out))
    return out if size else None


def palette_decode(payload: np.ndarray, n: int, bits: int,
                   initial: np.ndarray | None = None) -> np.ndarray:
    """Words in payload order; a payload without the format's mode byte leaves the
    initial words unchanged."""
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    words = (np.zeros(n, dtype=np.uint16) if initial is None
             else np.array(initial, dtype=np.uint16).reshape(-1).copy())
    load().sz_palette_decode(_ptr(payload), n, bits, _ptr(words))
    return words


def encode_paged_batch(kv: np.ndarray, plane_stride: int, block_stride: int, block_words: int,
                       block_tables, out_offsets, out_size: int, tables: np.ndarray,
                       chunk: int = 1 << 16, threads: int = 0) -> np.ndarray:
    """Gather + canonical Top-16 encode of one paged layer for several requests."""
    kv = np.ascontiguousarray(kv, dtype=np.uint16).reshape(-1)
    ids = np.ascontiguousarray(np.concatenate([np.asarray(t, dtype=np.int64)
                                               for t in block_tables]))
    offsets = np.zeros(len(block_tables) + 1, dtype=np.uint64)
    offsets[1:] = np.cumsum([len(t) for t in block_tables])
    outs = np.ascontiguousarray(out_offsets, dtype=np.uint64)
    out = np.zeros(out_size, dtype=np.uint8)
    rc = load().sz_top16_encode_paged_batch(
        _ptr(kv), plane_stride, block_stride, block_words, _ptr(ids), _ptr(offsets),
        len(block_tables), _ptr(out), _ptr(outs), _ptr(np.ascontiguousarray(tables)), chunk,
        threads)
    if rc != 0:
        raise RuntimeError("oracle paged encode failed")
    return out


def decode_paged_batch(src: np.ndarray, src_offsets, kv: np.ndarray, plane_stride: int,
                       block_stride: int, block_words: int, block_tables, tables: np.ndarray,
                       chunk: int = 1 << 16, threads: int = 0) -> None:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    assert kv.dtype == np.uint16 and kv.flags.c_contiguous
    ids = np.ascontiguousarray(np.concatenate([np.asarray(t, dtype=np.int64)
                                               for t in block_tables]))
    offsets = np.zeros(len(block_tables) + 1, dtype=np.uint64)
    offsets[1:] = np.cumsum([len(t) for t in block_tables])
    srcs = np.ascontiguousarray(src_offsets, dtype=np.uint64)
    rc = load().sz_top16_decode_paged_batch(
        _ptr(src), _ptr(srcs), len(block_tables), _ptr(kv), plane_stride, block_stride,
        block_words, _ptr(ids), _ptr(offsets), _ptr(np.ascontiguousarray(tables)), chunk,
        threads)
    if rc != 0:
        raise RuntimeError("oracle paged decode failed")


# ---------------------------------------------------------------------------
# pure-Python restatements (small inputs only)

def top16_tables_py(codebooks32: bytes) -> bytes:
    """splitzip_cuda.py:290-297: reverse map with later-code-wins, then the books."""
    values = bytearray([255]) * 512
    for plane in range(2):
        for code, exponent in enumerate(codebooks32[plane * 16:(plane + 1) * 16]):
            values[plane * 256 + exponent] = code
    return bytes(values) + bytes(codebooks32)


def encode_top16_py(words, tables: bytes) -> bytes | None:
    """Per-element restatement of EncodeTop16/FinalizeTop16 (kvq_splitzip_cuda.cu:
    154-208), escapes in ascending order and unused slots zeroed (canonical form)."""
    n = len(words)
    if n == 0 or n > 0xFFFFFFFF:
        return None
    size = top16_encoded_size(n)
    if size >= 2 * n:
        return None
    cap = escape_capacity(n)
    out = bytearray(size)
    body_at, codes_at = 5, 5 + n
    entries_at = codes_at + (n + 1) // 2
    escapes = []
    for index, word in enumerate(words):
        exponent = (word >> 7) & 0xFF
        code = tables[(index >= n // 2) * 256 + exponent]
        out[body_at + index] = (word & 0x7F) | ((word >> 8) & 0x80)
        if code == 255:
            escapes.append((index, exponent))
            code = 0
        out[codes_at + index // 2] |= (code & 0x0F) << ((index % 2) * 4)
    for slot, (position, exponent) in enumerate(escapes[:cap]):
        at = entries_at + slot * 5
        out[at:at + 4] = position.to_bytes(4, "little")
        out[at + 4] = exponent
    out[0] = 255 if len(escapes) > cap else 5
    out[1:5] = min(len(escapes), cap).to_bytes(4, "little")
    return bytes(out)


def decode_top16_payload_py(data, raw_bytes: int, codebooks: bytes) -> bytes | None:
    """Restatement of the reference's CPU Top-16 decoder,
    src/unchain_kv/vllm_connector.py:176-219 (same rejections, same result)."""
    view = memoryview(data).cast("B") if memoryview(data).format != "B" else memoryview(data)
    if (raw_bytes <= 0 or raw_bytes % 4 or len(codebooks) != 32 or len(view) < 5
            or view[0] != 5):
        return None
    count = raw_bytes // 2
    code_bytes = (count + 1) // 2
    cap = escape_capacity(count)
    if len(view) != 5 + count + code_bytes + cap * 5:
        return None
    escape_count = int.from_bytes(view[1:5], "little")
    if escape_count > cap:
        return None
    raw = bytearray(raw_bytes)
    plane_words = count // 2
    for index in range(count):
        code = (view[5 + count + index // 2] >> ((index % 2) * 4)) & 0x0F
        exponent = codebooks[(index >= plane_words) * 16 + code]
        value = view[5 + index]
        word = (value & 0x7F) | ((value & 0x80) << 8) | (exponent << 7)
        raw[2 * index] = word & 0xFF
        raw[2 * index + 1] = word >> 8
    entries = 5 + count + code_bytes
    for slot in range(escape_count):
        at = entries + slot * 5
        position = int.from_bytes(view[at:at + 4], "little")
        if position >= count:
            return None
        word = raw[2 * position] | (raw[2 * position + 1] << 8)
        word = (word & 0x807F) | (view[at + 4] << 7)
        raw[2 * position] = word & 0xFF
        raw[2 * position + 1] = word >> 8
    return bytes(raw)


def unpack_bits_py(packed: bytes, count: int, width: int) -> list[int]:
    """LSB-first bit unpacking of ``_unpack_splitzip_bits``
    (src/unchain_kv/vllm_connector.py:3376-3404): code i sits at bit i*width."""
    value = int.from_bytes(bytes(packed), "little")
    mask = (1 << width) - 1
    return [(value >> (index * width)) & mask for index in range(count)]


def fit_top16_py(histogram) -> list[int] | None:
    """Codebook fit of scripts/extract_llama_top16_codebooks.py:39-42: rank by
    (-count, value), keep the first 16 with a non-zero count; None if fewer."""
    ranked = sorted(range(256), key=lambda value: (-histogram[value], value))
    selected = [value for value in ranked if histogram[value] > 0][:16]
    return selected if len(selected) == 16 else None


def visible_cores() -> int:
    """Cores this process may run on (its CPU affinity)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def default_threads() -> int:
    """Threads for the oracle's multi-threaded calls: the host's CPU share for one
    GPU, ``OMP_NUM_THREADS`` when it is set (16 on a one-GPU share of an 8-GPU
    node), else at most 16, and never more than the visible cores."""
    try:
        share = int(os.environ.get("OMP_NUM_THREADS", "") or 16)
    except ValueError:
        share = 16
    return max(1, min(visible_cores(), share))


# ---------------------------------------------------------------------------
# the reference connector's torch-op codecs, payload modes 0, 1, 2
# (src/unchain_kv/vllm_connector.py:3204-3343 encode, :5168-5252 decode); numpy

def pack_bits_lsb(codes, width: int) -> np.ndarray:
    """``_pack_splitzip_bits`` (vllm_connector.py:3345-3374): code i at bits
    [i*width, i*width + width) of a little-endian bit stream, (count*width+7)//8
    bytes."""
    codes = np.asarray(codes, dtype=np.uint16).reshape(-1)
    bits = ((codes[:, None] >> np.arange(width, dtype=np.uint16)) & 1).astype(np.uint8)
    return np.packbits(bits.reshape(-1), bitorder="little")


def unpack_bits_lsb(packed, count: int, width: int) -> np.ndarray:
    """``_unpack_splitzip_bits`` (vllm_connector.py:3376-3404)."""
    bits = np.unpackbits(np.asarray(packed, dtype=np.uint8), bitorder="little")[:count * width]
    weights = (1 << np.arange(width, dtype=np.uint16)).astype(np.uint16)
    return (bits.reshape(count, width).astype(np.uint16) * weights).sum(axis=1).astype(np.uint16)


def _split_words(words):
    w = np.asarray(words, dtype=np.uint16).reshape(-1)
    return w, (w >> 8).astype(np.uint8), (w & 0xFF).astype(np.uint8)


def encode_signmag(words) -> np.ndarray | None:
    """Mode 2 (vllm_connector.py:3204-3247): [2][width][mag_min][low n][sign bits]
    [magnitude - mag_min in `width` bits]; None when the width is 7 or the payload
    is not smaller than the raw words."""
    w, high, low = _split_words(words)
    n = w.size
    sign, mag = high >> 7, high & 0x7F
    mag_min = int(mag.min())
    width = max(1, (int(mag.max()) - mag_min).bit_length())
    size = 3 + n + (n + 7) // 8 + (n * width + 7) // 8
    if width >= 7 or size >= 2 * n:
        return None
    return np.concatenate([np.array([2, width, mag_min], np.uint8), low, pack_bits_lsb(sign, 1),
                           pack_bits_lsb(mag - mag_min, width)])


def encode_palette(words) -> np.ndarray | None:
    """Mode 0 (vllm_connector.py:3249-3276): [0][width][256-byte sorted palette of
    high bytes, zero-filled][low n][palette index in `width` bits]."""
    w, high, low = _split_words(words)
    n = w.size
    palette, codes = np.unique(high, return_inverse=True)
    width = max(1, (palette.size - 1).bit_length())
    size = 258 + n + (n * width + 7) // 8
    if width >= 8 or size >= 2 * n:
        return None
    head = np.zeros(258, np.uint8)
    head[1] = width
    head[2:2 + palette.size] = palette
    return np.concatenate([head, low, pack_bits_lsb(codes, width)])


def encode_nibbles(words) -> np.ndarray | None:
    """Mode 1 (vllm_connector.py:3278-3343): [1][4 widths][4 x 16-byte sorted
    palettes of the nibble values][4 planes of indices], nibble p = bits 4p..4p+3;
    width 1, 2 or 4 by the plane's distinct values."""
    w = np.asarray(words, dtype=np.uint16).reshape(-1)
    n = w.size
    head = np.zeros(69, np.uint8)
    head[0] = 1
    planes = []
    for p, shift in enumerate((0, 4, 8, 12)):
        nibble = ((w >> shift) & 0xF).astype(np.uint8)
        palette, codes = np.unique(nibble, return_inverse=True)
        width = 1 if palette.size <= 2 else 2 if palette.size <= 4 else 4
        head[1 + p] = width
        head[5 + 16 * p:5 + 16 * p + palette.size] = palette
        planes.append(pack_bits_lsb(codes, width))
    payload = np.concatenate([head] + planes)
    return payload if payload.size < 2 * n else None


def encode_torchop(words) -> np.ndarray | None:
    """The reference's codec choice when the native codec is not used
    (vllm_connector.py:3204-3343): sign/magnitude, else palette, else nibble planes."""
    for encode in (encode_signmag, encode_palette, encode_nibbles):
        payload = encode(words)
        if payload is not None:
            return payload
    return None


def decode_torchop(payload, n: int) -> np.ndarray | None:
    """Words of a mode 0, 1 or 2 payload of n words, or None when the restore
    validation of vllm_connector.py:5168-5252 refuses it. The arithmetic is the
    reference's: int32 intermediates, the word truncated to 16 bits at the end."""
    p = np.asarray(payload, dtype=np.uint8).reshape(-1)
    size = p.size
    if size < 1:
        return None
    mode = int(p[0])
    if mode == 0:
        if size < 258:
            return None
        width = int(p[1])
        if not 1 <= width < 8 or size != 258 + n + (n * width + 7) // 8:
            return None
        codes = unpack_bits_lsb(p[258 + n:], n, width)
        high = p[2:258][codes].astype(np.int64)
        words = (high << 8) | p[258:258 + n].astype(np.int64)
    elif mode == 1:
        if size < 69:
            return None
        widths = [int(x) for x in p[1:5]]
        if any(x not in (1, 2, 4) for x in widths):
            return None
        sizes = [(n * x + 7) // 8 for x in widths]
        if size != 69 + sum(sizes):
            return None
        words = np.zeros(n, np.int64)
        at = 69
        for plane, (width, nbytes) in enumerate(zip(widths, sizes)):
            codes = unpack_bits_lsb(p[at:at + nbytes], n, width)
            words |= p[5 + 16 * plane:5 + 16 * plane + 16][codes].astype(np.int64) << (4 * plane)
            at += nbytes
    elif mode == 2:
        if size < 3:
            return None
        width, mag_min = int(p[1]), int(p[2])
        if not 1 <= width < 7:
            return None
        sign_bytes, mag_bytes = (n + 7) // 8, (n * width + 7) // 8
        if size != 3 + n + sign_bytes + mag_bytes:
            return None
        low = p[3:3 + n].astype(np.int64)
        sign = unpack_bits_lsb(p[3 + n:3 + n + sign_bytes], n, 1).astype(np.int64)
        mag = unpack_bits_lsb(p[3 + n + sign_bytes:], n, width).astype(np.int64)
        words = (((sign << 7) | (mag + mag_min)) << 8) | low
    else:
        return None
    return (words & 0xFFFF).astype(np.uint16)
