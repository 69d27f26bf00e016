"""Top-16 codec restated in torch CPU ops, in the op-by-op style of the reference
connector's torch codecs (TEST INFRASTRUCTURE: the ``ref-cpu-torch`` leg of the
benchmark's CPU baseline, and tests).

The reference has no torch Top-16 encoder; its torch codec paths
(src/unchain_kv/vllm_connector.py:3204-3343) split each bf16 word with bitwise
ops, look codes up by table indexing, pack sub-byte codes with strided adds
(`_pack_splitzip_bits`, :3345-3374) and unpack them with strided shifts
(`_unpack_splitzip_bits`, :3376-3404). The Top-16 arithmetic those ops carry out
here is that of kvq_splitzip_cuda.cu:154-208 (encode) and :210-284 (decode);
escapes are emitted in ascending position order (``nonzero``) with unused slots
zeroed, the canonical form of the C oracle, so both give identical bytes.
"""

from __future__ import annotations


def _le32(values, torch):
    """(k, 4) uint8 little-endian bytes of int64 values < 2^32."""
    shifts = torch.tensor([0, 8, 16, 24], dtype=torch.int64)
    return torch.bitwise_and(torch.bitwise_right_shift(values.unsqueeze(1), shifts), 0xFF).to(
        torch.uint8)


def encode_top16(words, tables, torch):
    """Canonical Top-16 payload (uint8 tensor) of n words (int16/uint16-bit tensor)
    with the 544-byte table (uint8 tensor)."""
    n = words.numel()
    w = torch.bitwise_and(words.reshape(-1).to(torch.int32), 0xFFFF)
    exponent = torch.bitwise_and(torch.bitwise_right_shift(w, 7), 0xFF)
    plane = (torch.arange(n, dtype=torch.int64) >= n // 2).to(torch.int64)
    code = tables[:512][plane * 256 + exponent.to(torch.int64)]
    escaped = code == 255
    body = torch.bitwise_or(torch.bitwise_and(w, 0x7F),
                            torch.bitwise_and(torch.bitwise_right_shift(w, 8), 0x80))
    code = torch.where(escaped, torch.zeros_like(code), torch.bitwise_and(code, 0x0F))
    cap = (n + 199) // 200
    code_bytes = (n + 1) // 2
    out = torch.zeros(5 + n + code_bytes + 5 * cap, dtype=torch.uint8)
    out[5:5 + n].copy_(body.to(torch.uint8))
    packed = out[5 + n:5 + n + code_bytes]
    # width-4 strided packing: even words in the low nibble, odd words in the high one
    packed.copy_(code[0::2])
    high = torch.bitwise_left_shift(code[1::2].to(torch.int16), 4).to(torch.uint8)
    if high.numel():
        packed[:high.numel()].add_(high)
    positions = torch.nonzero(escaped).reshape(-1)
    count = positions.numel()
    used = min(count, cap)
    if used:
        entries = out[5 + n + code_bytes:5 + n + code_bytes + 5 * used].view(used, 5)
        entries[:, :4].copy_(_le32(positions[:used], torch))
        entries[:, 4].copy_(exponent[positions[:used]].to(torch.uint8))
    out[0] = 255 if count > cap else 5
    out[1:5].copy_(_le32(torch.tensor([used], dtype=torch.int64), torch).reshape(4))
    return out


def decode_top16(payload, n, tables, torch):
    """Words (int32 tensor, 16-bit values) of a mode-5 payload of n words, or None
    for any other mode byte."""
    if int(payload[0]) != 5:
        return None
    code_bytes = (n + 1) // 2
    body = payload[5:5 + n].to(torch.int32)
    packed = payload[5 + n:5 + n + code_bytes]
    code = torch.empty(n, dtype=torch.uint8)
    code[0::2].copy_(torch.bitwise_and(packed, 0x0F))
    if n // 2:
        code[1::2].copy_(torch.bitwise_right_shift(packed[:n // 2].to(torch.int16), 4).to(
            torch.uint8))
    plane = (torch.arange(n, dtype=torch.int64) >= n // 2).to(torch.int64)
    exponent = tables[512:544][plane * 16 + code.to(torch.int64)].to(torch.int32)
    words = torch.bitwise_or(
        torch.bitwise_or(torch.bitwise_and(body, 0x7F),
                         torch.bitwise_left_shift(torch.bitwise_and(body, 0x80), 8)),
        torch.bitwise_left_shift(exponent, 7))
    cap = (n + 199) // 200
    count = min(int.from_bytes(bytes(payload[1:5].tolist()), "little"), cap)
    if count:
        at = 5 + n + code_bytes
        entries = payload[at:at + 5 * count].view(count, 5).to(torch.int64)
        positions = (entries[:, 0] | (entries[:, 1] << 8) | (entries[:, 2] << 16)
                     | (entries[:, 3] << 24))
        keep = positions < n
        positions = positions[keep]
        patched = torch.bitwise_or(torch.bitwise_and(words[positions], 0x807F),
                                   torch.bitwise_left_shift(entries[keep, 4].to(torch.int32), 7))
        words[positions] = patched
    return words


def encode_paged(kv_layer, block_tables, tables, torch):
    """Per request: gather its blocks with index_select (the reference connector's
    gather, vllm_connector.py:2862) and encode them. kv_layer: int16 CPU tensor
    (2, num_blocks, ...)."""
    out = []
    for ids in block_tables:
        index = torch.tensor(ids, dtype=torch.int64)
        out.append(encode_top16(kv_layer.index_select(1, index).reshape(-1), tables, torch))
    return out


def decode_paged(payloads, kv_layer, block_tables, tables, torch):
    """Decode each payload and scatter it into its blocks with index_copy_
    (vllm_connector.py:5305-5311)."""
    for payload, ids in zip(payloads, block_tables):
        index = torch.tensor(ids, dtype=torch.int64)
        n = 2 * len(ids) * kv_layer[0, 0].numel()
        words = decode_top16(payload, n, tables, torch)
        if words is None:
            continue
        source = words.to(torch.int16).reshape((2, len(ids)) + tuple(kv_layer.shape[2:]))
        kv_layer.index_copy_(1, index, source)
