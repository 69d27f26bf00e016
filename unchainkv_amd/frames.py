"""Compressed-native layer frames (``KVC1`` / ``KVC2``): the byte layout a codec
payload travels in, so payloads from this library are wire-compatible with a
reference peer. No sockets: frames are built and parsed from bytes.

Layout (src/unchain_kv/tcp_data.py:612-652 for the sender, :282-361 for the
receiver; native/unchain_kv/kvq_tcp.cc:224-256 builds the same KVC1 header):

    envelope   u32 body length, u32 CRC-32 of the body        (network order, "!II")
    body       magic "KVC1" (whole layer) or "KVC2" (one chunk of a layer)
               string transfer_id, string request_id           (u32 length + UTF-8)
               u32 layer_index, block_count, raw_block_size, raw_bytes, codec_code
               [KVC2 only: u32 chunk_index, chunks_in_layer]
               u32 encoded_bytes
               payload (encoded_bytes bytes)

All integers are big-endian u32. ``raw_block_size`` is the raw bytes of one block
(K and V planes); codec codes are raw_passthrough = 0, splitzip_bf16 = 1. A
layer sent in two halves (tcp_data.py via vllm_connector.py:4785-4810) is two KVC2
frames with chunk_index 0 and 1 of chunks_in_layer 2, each carrying the payload
of its half of the block list.
"""

from __future__ import annotations

import struct
import zlib
from dataclasses import dataclass

ENVELOPE = struct.Struct("!II")
U32 = struct.Struct("!I")
LAYER_MAGIC = b"KVC1"
CHUNK_MAGIC = b"KVC2"
CODEC_CODES = {"raw_passthrough": 0, "splitzip_bf16": 1}
CODE_CODECS = {code: name for name, code in CODEC_CODES.items()}
U32_MAX = 0xFFFFFFFF


def _string(value: str) -> bytes:
    data = value.encode("utf-8")
    return U32.pack(len(data)) + data


def _read_string(data, offset: int) -> tuple[str, int]:
    (size,) = U32.unpack_from(data, offset)
    offset += U32.size
    end = offset + size
    if end > len(data):
        raise ValueError("truncated compressed native frame")
    return bytes(data[offset:end]).decode("utf-8"), end


@dataclass(frozen=True)
class CompressedNativeFrame:
    transfer_id: str
    request_id: str
    layer_index: int
    block_count: int
    raw_block_size: int
    raw_bytes: int
    codec: str
    chunk_index: int
    chunks_in_layer: int
    payload: memoryview

    @property
    def encoded_bytes(self) -> int:
        return len(self.payload)

    def metadata(self) -> dict:
        """The layer metadata a reference receiver stores with the payload
        (tcp_data.py:320-329): encoded_bytes for a whole layer, chunks_in_layer for a
        chunk."""
        meta = {"block_count": self.block_count, "raw_block_size": self.raw_block_size,
                "raw_bytes": self.raw_bytes, "codec": self.codec}
        if self.chunks_in_layer > 1:
            meta["chunks_in_layer"] = self.chunks_in_layer
        else:
            meta["encoded_bytes"] = self.encoded_bytes
        return meta


def compressed_native_header(transfer_id: str, request_id: str, layer_index: int,
                             encoded_bytes: int, *, raw_block_size: int, block_count: int,
                             raw_bytes: int, codec: str, chunk_index: int = 0,
                             chunks_in_layer: int = 1) -> bytes:
    """Body header of a compressed-native frame (everything before the payload).
    Errors follow the reference sender: an unknown codec is a KeyError, negative
    metadata or a chunk index outside [0, chunks_in_layer) a ValueError."""
    code = CODEC_CODES[codec]
    if raw_block_size < 0 or block_count < 0 or raw_bytes < 0:
        raise ValueError("compressed native metadata must be non-negative")
    for value in (layer_index, block_count, raw_block_size, raw_bytes, encoded_bytes):
        if not 0 <= value <= U32_MAX:
            raise ValueError("compressed native field does not fit 32 bits")
    chunked = chunks_in_layer > 1
    parts = [CHUNK_MAGIC if chunked else LAYER_MAGIC, _string(transfer_id), _string(request_id),
             U32.pack(layer_index), U32.pack(block_count), U32.pack(raw_block_size),
             U32.pack(raw_bytes), U32.pack(code)]
    if chunked:
        if not 0 <= chunk_index < chunks_in_layer:
            raise ValueError("compressed native chunk index out of range")
        parts += [U32.pack(chunk_index), U32.pack(chunks_in_layer)]
    parts.append(U32.pack(encoded_bytes))
    return b"".join(parts)


def envelope(parts) -> bytes:
    """The 8-byte frame prefix for a body made of ``parts``: total length and the
    CRC-32 of the parts in order (tcp_data.py:672-679, kvq_tcp.cc:155-170)."""
    total, crc = 0, 0
    for part in parts:
        view = memoryview(part).cast("B")
        total += len(view)
        crc = zlib.crc32(view, crc)
    if total > U32_MAX:
        raise ValueError("frame too large")
    return ENVELOPE.pack(total, crc & U32_MAX)


def pack_compressed_native(transfer_id: str, request_id: str, layer_index: int, payload, *,
                           raw_block_size: int, block_count: int, raw_bytes: int, codec: str,
                           chunk_index: int = 0, chunks_in_layer: int = 1) -> list:
    """Frame parts ``[envelope, header, payload]`` (payload unchanged, zero-copy) of
    one compressed-native frame; ``b"".join`` gives the bytes on the wire."""
    view = memoryview(payload).cast("B")
    header = compressed_native_header(transfer_id, request_id, layer_index, len(view),
                                      raw_block_size=raw_block_size, block_count=block_count,
                                      raw_bytes=raw_bytes, codec=codec, chunk_index=chunk_index,
                                      chunks_in_layer=chunks_in_layer)
    return [envelope([header, view]), header, view]


def parse_compressed_native(body) -> CompressedNativeFrame:
    """Parses a frame body that starts with KVC1 or KVC2 (tcp_data.py:282-318): an
    unknown codec code or a payload whose length differs from encoded_bytes is a
    ValueError."""
    data = memoryview(body).cast("B")
    magic = bytes(data[:4])
    if magic not in (LAYER_MAGIC, CHUNK_MAGIC):
        raise ValueError("not a compressed native frame")
    chunked = magic == CHUNK_MAGIC
    offset = 4
    transfer_id, offset = _read_string(data, offset)
    request_id, offset = _read_string(data, offset)
    count = 7 if chunked else 5
    if offset + U32.size * (count + 1) > len(data):
        raise ValueError("truncated compressed native frame")
    fields = struct.unpack_from("!" + "I" * count, data, offset)
    offset += U32.size * count
    (encoded_bytes,) = U32.unpack_from(data, offset)
    offset += U32.size
    layer_index, block_count, raw_block_size, raw_bytes, code = fields[:5]
    chunk_index, chunks_in_layer = (fields[5], fields[6]) if chunked else (0, 1)
    codec = CODE_CODECS.get(code)
    if codec is None:
        raise ValueError("unknown compressed native codec")
    if len(data) - offset != encoded_bytes:
        raise ValueError("bad compressed native payload size")
    return CompressedNativeFrame(transfer_id, request_id, layer_index, block_count, raw_block_size,
                                 raw_bytes, codec, chunk_index, chunks_in_layer, data[offset:])


def split_frame(buffer) -> tuple[memoryview, int]:
    """The body of the first frame in ``buffer`` and the bytes it spans (envelope
    included); a CRC mismatch or a truncated frame is a ValueError."""
    data = memoryview(buffer).cast("B")
    if len(data) < ENVELOPE.size:
        raise ValueError("truncated frame")
    size, crc = ENVELOPE.unpack_from(data, 0)
    end = ENVELOPE.size + size
    if end > len(data):
        raise ValueError("truncated frame")
    body = data[ENVELOPE.size:end]
    if zlib.crc32(body) & U32_MAX != crc:
        raise ValueError("frame checksum mismatch")
    return body, end
