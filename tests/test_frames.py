"""Compressed-native frames (KVC1 / KVC2): byte layout, envelope and validation.

The two frames of the reference's tests/test_tcp_data.py:191-265 (a KVC1
raw_passthrough layer of 2 blocks, and a splitzip_bf16 layer sent as two KVC2
chunks) are rebuilt field by field here and must parse to the metadata that test
expects; the builder must produce the same bytes.
"""

import struct
import zlib

import pytest

from unchainkv_amd import frames
from unchainkv_amd.connector import BITS_TOP16, LayerPayload, SplitzipLayerCodec

U32 = struct.Struct("!I")


def s(value: str) -> bytes:
    data = value.encode()
    return U32.pack(len(data)) + data


def test_kvc1_reference_vector():
    body = b"KVC1" + s("tx") + s("req") + b"".join(U32.pack(v) for v in (5, 2, 3, 6, 0, 6)) + \
        b"native"
    f = frames.parse_compressed_native(body)
    assert (f.transfer_id, f.request_id, f.layer_index) == ("tx", "req", 5)
    assert bytes(f.payload) == b"native"
    assert f.metadata() == {"block_count": 2, "raw_block_size": 3, "raw_bytes": 6,
                            "encoded_bytes": 6, "codec": "raw_passthrough"}
    parts = frames.pack_compressed_native("tx", "req", 5, b"native", raw_block_size=3,
                                          block_count=2, raw_bytes=6, codec="raw_passthrough")
    assert b"".join(parts[1:]) == body
    assert parts[0] == struct.pack("!II", len(body), zlib.crc32(body))


def test_kvc2_two_chunk_reference_vector():
    metas = []
    for chunk_index, payload in enumerate((b"zip", b"zap")):
        body = b"KVC2" + s("tx") + s("req") + b"".join(
            U32.pack(v) for v in (5, 4, 3, 12, 1, chunk_index, 2, len(payload))) + payload
        f = frames.parse_compressed_native(body)
        assert (f.chunk_index, f.chunks_in_layer, bytes(f.payload)) == (chunk_index, 2, payload)
        metas.append(f.metadata())
        parts = frames.pack_compressed_native("tx", "req", 5, payload, raw_block_size=3,
                                              block_count=4, raw_bytes=12, codec="splitzip_bf16",
                                              chunk_index=chunk_index, chunks_in_layer=2)
        assert b"".join(parts[1:]) == body
    assert metas[0] == metas[1] == {"block_count": 4, "raw_block_size": 3, "raw_bytes": 12,
                                    "codec": "splitzip_bf16", "chunks_in_layer": 2}


def test_envelope_checks_length_and_crc():
    parts = frames.pack_compressed_native("t", "r", 1, bytes(range(40)), raw_block_size=20,
                                          block_count=2, raw_bytes=40, codec="splitzip_bf16")
    wire = b"".join(parts) + b"next frame"
    body, end = frames.split_frame(wire)
    assert end == len(wire) - len(b"next frame")
    assert bytes(frames.parse_compressed_native(body).payload) == bytes(range(40))
    broken = bytearray(wire)
    broken[20] ^= 1
    with pytest.raises(ValueError, match="checksum"):
        frames.split_frame(broken)
    with pytest.raises(ValueError, match="truncated"):
        frames.split_frame(wire[:end - 1])


def test_parse_and_build_reject_bad_frames():
    good = b"KVC1" + s("tx") + s("req") + b"".join(U32.pack(v) for v in (5, 2, 3, 6, 0, 6))
    with pytest.raises(ValueError, match="size"):
        frames.parse_compressed_native(good + b"nativeX")
    bad_codec = b"KVC1" + s("tx") + s("req") + b"".join(U32.pack(v) for v in (5, 2, 3, 6, 7, 6))
    with pytest.raises(ValueError, match="codec"):
        frames.parse_compressed_native(bad_codec + b"native")
    with pytest.raises(ValueError):
        frames.parse_compressed_native(b"KVN1" + good[4:])
    with pytest.raises(ValueError, match="truncated"):
        frames.parse_compressed_native(good[:20])
    with pytest.raises(KeyError):
        frames.pack_compressed_native("t", "r", 0, b"x", raw_block_size=1, block_count=1,
                                      raw_bytes=1, codec="zstd")
    with pytest.raises(ValueError, match="non-negative"):
        frames.pack_compressed_native("t", "r", 0, b"x", raw_block_size=-1, block_count=1,
                                      raw_bytes=1, codec="splitzip_bf16")
    with pytest.raises(ValueError, match="chunk index"):
        frames.pack_compressed_native("t", "r", 0, b"x", raw_block_size=1, block_count=1,
                                      raw_bytes=1, codec="splitzip_bf16", chunk_index=2,
                                      chunks_in_layer=2)


def test_connector_frames_carry_payload_metadata():
    block_words = 2048
    payloads = [LayerPayload(0, [4, 9], 2 * 2 * 2 * block_words, BITS_TOP16, BITS_TOP16,
                             encoded_bytes=7, view=memoryview(b"\x05abcdef")),
                LayerPayload(1, [1], 2 * 2 * block_words, BITS_TOP16, BITS_TOP16,
                             encoded_bytes=3, view=memoryview(b"\x06xy"))]
    out = SplitzipLayerCodec.frames(12, payloads, block_words, "xfer", ["req-a", "req-b"])
    assert len(out) == 2
    for parts, p, name in zip(out, payloads, ["req-a", "req-b"]):
        body, end = frames.split_frame(b"".join(parts))
        f = frames.parse_compressed_native(body)
        assert (f.transfer_id, f.request_id, f.layer_index) == ("xfer", name, 12)
        assert bytes(f.payload) == bytes(p.view)
        assert f.metadata() == {"block_count": len(p.block_ids), "raw_block_size": 4 * block_words,
                                "raw_bytes": p.raw_bytes, "encoded_bytes": p.encoded_bytes,
                                "codec": "splitzip_bf16"}
