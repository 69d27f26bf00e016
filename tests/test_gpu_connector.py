"""The connector codec hooks on the GPU: save -> ready -> load round trips for
every codec the policy picks (Top-16, the fixed6 fallback on overflow, raw mode 6
when fixed6 overflows too, fixed5), with the payload bytes checked against the
oracle and against the per-request drop-in encoder."""

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format
from unchainkv_amd.connector import (BITS_FIXED5, BITS_FIXED6, BITS_PASSTHROUGH, BITS_RAW,
                                     BITS_TOP16, BITS_TORCHOP, CodecConfig, SplitzipLayerCodec)
from unchainkv_amd.trace import RecordingTrace

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sz():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda

    assert splitzip_cuda.available(), splitzip_cuda.load_error()
    return splitzip_cuda


def say(*parts):
    print("[case]", *parts, flush=True)


def u16(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


BW = 16384  # Llama-3-8B block: 16 tokens x 8 heads x 128


def layer_from_words(words, pool):
    return torch.from_numpy(words.view(np.int16).copy()).cuda().view(torch.bfloat16).view(
        2, pool, 16, 8, 128)


def words_with_books(rng, books, pool, escape_rate=0.0, distinct_high=None):
    n = 2 * pool * BW
    half = n // 2
    exps = np.empty(n, np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:], np.uint8)[rng.integers(0, 16, n - half)]
    outside = np.array(sorted(set(range(256)) - set(books)), np.uint16)
    esc = rng.random(n) < escape_rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    words = ((rng.integers(0, 2, n).astype(np.uint16) << 15) | (exps << 7)
             | rng.integers(0, 128, n).astype(np.uint16))
    return words.astype(np.uint16)


def disjoint_tables(rng, pool, sizes):
    perm = rng.permutation(pool).tolist()
    tables, at = [], 0
    for size in sizes:
        tables.append(perm[at:at + size])
        at += size
    return tables


def roundtrip(codec, layer_index, kv, tables, pool):
    pending = codec.save_kv_layer(layer_index, kv, tables)
    payloads = codec.ready(pending)
    target = torch.zeros_like(kv)
    recv = [[(b + 7) % pool for b in t] for t in tables]  # receiver's own block ids
    requests = [(rt, bytes(p.view), p.metadata(layer_index, BW)) for rt, p in zip(recv, payloads)]
    results = codec.load_kv_layer_batch(layer_index, target, requests)
    torch.cuda.synchronize()
    src, dst = u16(kv).reshape(2, pool, BW), u16(target).reshape(2, pool, BW)
    for t, rt, res in zip(tables, recv, results):
        assert res == (len(t), 2 * 2 * len(t) * BW)
        assert np.array_equal(dst[:, rt], src[:, t])
    return payloads


def test_top16_roundtrip_matches_dropin_payload_bytes(sz, codebooks):
    say("connector top16")
    books = codebooks[5 * 32:6 * 32]
    rng = np.random.default_rng(1)
    pool = 64
    kv = layer_from_words(words_with_books(rng, books, pool, 0.001), pool)
    tables = disjoint_tables(rng, pool, [16, 20, 17])  # >= 1 MiB each: Top-16
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=trace)
    payloads = roundtrip(codec, 5, kv, tables, pool)
    assert [p.bits for p in payloads] == [BITS_TOP16] * 3
    for t, p in zip(tables, payloads):
        # the per-request drop-in call on the gathered blocks gives the same bytes
        source = kv[:, t].contiguous()
        out = torch.empty(source.numel() * 2, dtype=torch.uint8, device="cuda")
        size = sz.encode_top16(source, out, 5)
        torch.cuda.synchronize()
        assert size == p.encoded_bytes
        assert bytes(out[:size].cpu().numpy()) == bytes(p.view)
        ref = oracle.top16_encode(u16(source).reshape(-1), oracle.top16_tables(books))
        assert bytes(ref) == bytes(p.view)
    assert "codec_encode_submitted" in trace.names()


def test_top16_overflow_falls_back_to_fixed6_and_backs_off(sz, codebooks):
    say("connector overflow -> fixed6")
    books = codebooks[2 * 32:3 * 32]
    rng = np.random.default_rng(2)
    pool = 64
    words = words_with_books(rng, books, pool, 0.0)
    kv_host = words.reshape(2, pool, BW)
    tables = disjoint_tables(rng, pool, [16, 16, 16])
    # request 1 gets 1.2% escapes: more than the 0.5% capacity
    outside = np.array(sorted(set(range(256)) - set(books))[:16], np.uint16)
    for b in tables[1]:
        hit = rng.random((2, BW)) < 0.012
        block = kv_host[:, b]
        block[hit] = (block[hit] & 0x807F) | (outside[rng.integers(0, 16, int(hit.sum()))] << 7)
        kv_host[:, b] = block
    kv = layer_from_words(kv_host.reshape(-1), pool)
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=trace)
    payloads = roundtrip(codec, 2, kv, tables, pool)
    assert [p.bits for p in payloads] == [BITS_TOP16, BITS_FIXED6, BITS_TOP16]
    assert payloads[1].fallback and payloads[1].view[0] == codec_format.MODE_FIXED6
    assert bytes(payloads[1].view) == bytes(oracle.fixed6_encode(kv_host[:, tables[1]].reshape(-1)))
    assert codec.top16_gate.window(2) == 1
    assert "splitzip_top16_overflow" in trace.names()
    # the next payload of the layer waits out the window, then probes
    assert codec._choose_bits(2, 1 << 20)[0] == BITS_FIXED6


def test_probe_after_an_overflow_reencodes_from_presence_masks(sz, codebooks):
    """Save 1 overflows (fixed6 fallback), save 2 waits out the window (fixed6
    chosen directly), save 3 probes: the probe's Top-16 encode records presence
    masks, overflows again, and the fixed6 re-encode starts from the masks. Every
    fixed6 payload equals the oracle's."""
    say("connector probe with presence masks")
    books = codebooks[2 * 32:3 * 32]
    rng = np.random.default_rng(12)
    pool = 40
    words = words_with_books(rng, books, pool, 0.0)
    # 1.2% escapes (above the 0.5% capacity) over 16 exponents outside the
    # codebooks, so the high bytes still fit the fixed6 palette
    outside = np.array(sorted(set(range(256)) - set(books))[:16], np.uint16)
    hit = rng.random(words.size) < 0.012
    words[hit] = (words[hit] & 0x807F) | (outside[rng.integers(0, 16, int(hit.sum()))] << 7)
    table = rng.permutation(pool)[:16].tolist()
    expect = oracle.fixed6_encode(words.reshape(2, pool, BW)[:, table].reshape(-1))
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=trace)
    for step, (probe, bits, fallback) in enumerate([(False, BITS_TOP16, True),
                                                     (False, BITS_FIXED6, False),
                                                     (True, BITS_TOP16, True)]):
        kv = layer_from_words(words, pool)
        pending = codec.save_kv_layer(2, kv, [table])
        p = pending.payloads[0]
        assert (p.probe, p.bits) == (probe, bits), step
        assert (pending.presence is not None) == probe, step
        assert (p._mask_first == 0) == probe, step
        # the probe's payload is not copied before its mode byte is known
        assert (not pending.groups and len(pending.deferred) == 1) == probe, step
        payloads = codec.ready(pending)
        assert pending.presence is None
        assert payloads[0].bits == BITS_FIXED6 and payloads[0].fallback == fallback, step
        assert bytes(payloads[0].view) == bytes(expect), step
    assert trace.names().count("splitzip_top16_probe") == 1


def test_fixed6_overflow_falls_back_to_raw_mode(sz, codebooks):
    say("connector fixed6 overflow -> raw")
    rng = np.random.default_rng(3)
    pool = 8
    words = rng.integers(0, 1 << 16, 2 * pool * BW).astype(np.uint16)  # every high byte
    kv = layer_from_words(words, pool)
    tables = [[0, 1, 2], [5]]
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=trace)
    payloads = roundtrip(codec, 0, kv, tables, pool)
    assert [p.bits for p in payloads] == [BITS_RAW, BITS_RAW]
    assert payloads[0].view[0] == codec_format.MODE_RAW
    assert payloads[0].encoded_bytes == payloads[0].raw_bytes + 1
    assert trace.names().count("splitzip_fixed6_overflow") == 2


def test_layer_without_codebook_is_unavailable_and_sticks_to_fixed6(sz, codebooks):
    say("connector layer 40 without codebook")
    rng = np.random.default_rng(4)
    pool = 24
    books = codebooks[:32]
    kv = layer_from_words(words_with_books(rng, books, pool, 0.0), pool)
    tables = disjoint_tables(rng, pool, [16])
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=trace)
    first = roundtrip(codec, 40, kv, tables, pool)
    assert first[0].bits == BITS_FIXED6 and first[0].fallback
    assert codec.top16_gate.closed(40)
    second = roundtrip(codec, 40, kv, tables, pool)
    assert second[0].bits == BITS_FIXED6 and not second[0].fallback
    # with an explicit codebook the layer uses Top-16
    with_books = SplitzipLayerCodec(CodecConfig(top16=True), codebooks={40: books})
    assert roundtrip(with_books, 40, kv, tables, pool)[0].bits == BITS_TOP16


def test_small_requests_fixed5_and_its_overflow_downgrade(sz, codebooks):
    say("connector fixed5")
    rng = np.random.default_rng(5)
    pool = 6
    highs = np.array(sorted(rng.choice(256, 20, replace=False)), np.uint16)
    words = ((highs[rng.integers(0, 20, 2 * pool * BW)] << 8)
             | rng.integers(0, 256, 2 * pool * BW)).astype(np.uint16)
    kv_host = words.reshape(2, pool, BW)
    kv_host[:, 4] = (np.arange(BW, dtype=np.uint16) % 40) << 8  # 40 distinct: fixed5 overflows
    kv = layer_from_words(kv_host.reshape(-1), pool)
    codec = SplitzipLayerCodec(CodecConfig(top16=True, fixed5=True))
    payloads = roundtrip(codec, 3, kv, [[0], [4]], pool)  # 64 KiB each: below the Top-16 size
    assert payloads[0].bits == BITS_FIXED5 and payloads[0].view[0] == codec_format.MODE_FIXED5
    assert payloads[1].bits == BITS_FIXED6 and payloads[1].fallback
    assert 3 in codec._splitzip_fixed6_layers
    assert codec._choose_bits(3, 4096)[0] == BITS_FIXED6


def test_single_request_load_signature_matches_reference(sz, codebooks):
    say("connector load_kv_layer")
    rng = np.random.default_rng(6)
    pool = 40
    books = codebooks[:32]
    kv = layer_from_words(words_with_books(rng, books, pool, 0.002), pool)
    src, dst = disjoint_tables(rng, pool, [16, 16])
    codec = SplitzipLayerCodec(CodecConfig(top16=True))
    payload = codec.ready(codec.save_kv_layer(0, kv, [src]))[0]
    assert payload.bits == BITS_TOP16
    target = torch.zeros_like(kv)
    meta = payload.metadata(0, BW)
    assert codec.load_kv_layer(target, dst, [bytes(payload.view)], meta) == (16, meta["raw_bytes"])
    torch.cuda.synchronize()
    assert np.array_equal(u16(target).reshape(2, pool, BW)[:, dst],
                          u16(kv).reshape(2, pool, BW)[:, src])
    assert codec.load_kv_layer(target, dst[:2], [bytes(payload.view)], meta) == (0, 0)


def test_layer_travels_in_compressed_native_frames(sz, codebooks):
    """save -> ready -> KVC1 frames on the wire -> parse -> restore into the
    receiver's own blocks; plus one request sent as two KVC2 halves and a
    raw_passthrough frame (tcp_data.py:612-652, vllm_connector.py:4785-4810)."""
    from unchainkv_amd import frames

    say("connector frames")
    books = codebooks[5 * 32:6 * 32]
    rng = np.random.default_rng(9)
    pool = 96
    kv = layer_from_words(words_with_books(rng, books, pool, 0.001), pool)
    tables = disjoint_tables(rng, pool, [16, 20, 18])
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=RecordingTrace())
    payloads = codec.ready(codec.save_kv_layer(5, kv, tables))
    names = ["r0", "r1", "r2"]
    wire = b"".join(b"".join(p) for p in SplitzipLayerCodec.frames(5, payloads, BW, "x", names))
    # request r2 again, as two halves in KVC2 frames
    halves = [tables[2][:9], tables[2][9:]]
    half_payloads = codec.ready(codec.save_kv_layer(5, kv, halves))
    for i, p in enumerate(half_payloads):
        wire += b"".join(frames.pack_compressed_native(
            "x", "r2h", 5, p.view, raw_block_size=4 * BW, block_count=18,
            raw_bytes=4 * BW * 18, codec="splitzip_bf16", chunk_index=i, chunks_in_layer=2))
    # request r1 as raw native words
    raw = u16(kv[:, tables[1]]).tobytes()
    wire += b"".join(frames.pack_compressed_native("x", "r1raw", 5, raw, raw_block_size=4 * BW,
                                                   block_count=20, raw_bytes=len(raw),
                                                   codec="raw_passthrough"))
    bodies, at = [], 0
    while at < len(wire):
        body, used = frames.split_frame(memoryview(wire)[at:])
        bodies.append(body)
        at += used
    assert len(bodies) == 6
    recv_perm = rng.permutation(pool).tolist()
    recv = {"r0": recv_perm[0:16], "r1": recv_perm[16:36], "r2": recv_perm[36:54],
            "r2h": recv_perm[54:72], "r1raw": recv_perm[72:92]}
    target = torch.zeros_like(kv)
    got = codec.restore_frames(target, bodies, recv)
    torch.cuda.synchronize()
    src, dst = u16(kv).reshape(2, pool, BW), u16(target).reshape(2, pool, BW)
    for name, t in (("r0", tables[0]), ("r1", tables[1]), ("r2", tables[2]),
                    ("r2h", tables[2]), ("r1raw", tables[1])):
        assert got[name] == (len(t), 4 * BW * len(t)), name
        assert np.array_equal(dst[:, recv[name]], src[:, t]), name


def test_sender_splits_requests_into_two_kvc2_chunks(sz, codebooks):
    """UNCHAIN_KV_SPLITZIP_CHUNKS=2 without Top-16 (vllm_connector.py:2718-2799): a
    request with an even number of blocks in one run leaves as two half-payloads in
    KVC2 frames -- fixed6 for halves of 1 MiB or more, a torch-op format below --
    the others as one KVC1 frame (torch-op below 1 MiB); every payload equals the
    oracle's encoding of its blocks and the receiver restores all of them."""
    from unchainkv_amd import frames

    say("connector two-chunk frames")
    rng = np.random.default_rng(19)
    pool = 80
    highs = rng.choice(256, 40, replace=False).astype(np.uint16)   # fits the fixed6 palette
    n = 2 * pool * BW
    words = ((highs[rng.integers(0, 40, n)] << 8) | rng.integers(0, 256, n).astype(np.uint16))
    words = words.astype(np.uint16)
    kv = layer_from_words(words, pool)
    # a 32-block run (halves of 1 MiB), a 12-block run (halves below 1 MiB), odd, not a run
    tables = [list(range(10, 42)), list(range(50, 62)), [66, 67, 68], [70, 72, 71, 73]]
    codec = SplitzipLayerCodec(CodecConfig(chunks=2), trace=RecordingTrace())
    pending = codec.save_kv_layer(3, kv, tables)
    payloads = codec.ready(pending)
    assert [(p.request, p.chunk_index, p.chunks_in_layer, p.bits) for p in payloads] == \
        [(0, 0, 2, BITS_FIXED6), (0, 1, 2, BITS_FIXED6), (1, 0, 2, BITS_TORCHOP),
         (1, 1, 2, BITS_TORCHOP), (2, 0, 1, BITS_TORCHOP), (3, 0, 1, BITS_TORCHOP)]
    host = words.reshape(2, pool, BW)
    for p in payloads:
        blocks = host[:, p.block_ids].reshape(-1)
        expected = oracle.fixed6_encode(blocks) if p.bits == BITS_FIXED6 else \
            oracle.encode_torchop(blocks)
        assert bytes(p.view) == bytes(expected)
    assert {p.view[0] for p in payloads if p.bits == BITS_TORCHOP} == {codec_format.MODE_PALETTE}
    parts = SplitzipLayerCodec.frames(3, payloads, BW, "t2", ["a", "b", "c", "d"])
    parsed = [frames.parse_compressed_native(b"".join(x[1:])) for x in parts]
    assert [(f.request_id, f.chunks_in_layer, f.block_count) for f in parsed] == \
        [("a", 2, 32), ("a", 2, 32), ("b", 2, 12), ("b", 2, 12), ("c", 1, 3), ("d", 1, 4)]
    perm = rng.permutation(pool).tolist()
    recv = {"a": perm[:32], "b": perm[32:44], "c": perm[44:47], "d": perm[47:51]}
    target = torch.zeros_like(kv)
    got = codec.restore_frames(target, [b"".join(x[1:]) for x in parts], recv)
    torch.cuda.synchronize()
    codec.release(pending)
    dst = u16(target).reshape(2, pool, BW)
    for name, t in zip("abcd", tables):
        assert got[name] == (len(t), 4 * BW * len(t)), name
        assert np.array_equal(dst[:, recv[name]], host[:, t]), name


def test_small_requests_take_the_torchop_formats(sz, codebooks):
    """Without Top-16 a request below 1 MiB leaves in the reference's torch-op
    formats (vllm_connector.py:3043-3046, 3204-3343): sign/magnitude, the high-byte
    palette or the nibble planes, byte for byte the oracle's (which the reference
    connector's own payloads pin); an incompressible one as raw words with codec
    raw_passthrough (:2685-2711); a 1 MiB request with the native fixed6. All of
    them go through KVC1 frames and are restored into the receiver's blocks."""
    from unchainkv_amd import frames

    say("connector torch-op sender")
    rng = np.random.default_rng(23)
    pool = 40
    host = np.empty((2, pool, BW), np.uint16)
    low = rng.integers(0, 256, (2, pool, BW)).astype(np.uint16)
    sign = rng.integers(0, 2, (2, pool, BW)).astype(np.uint16) << 15
    host[:] = sign | ((0x38 + rng.integers(0, 8, (2, pool, BW)).astype(np.uint16)) << 8) | low
    palette = np.array([0x00, 0x7F, 0x81, 0x3C, 0xC0], np.uint16)   # 7-bit magnitudes
    host[:, 4:7] = (palette[rng.integers(0, 5, (2, 3, BW))] << 8) | low[:, 4:7]
    nib = rng.integers(0, 1 << 16, (2, 2, BW)).astype(np.uint16) & 0xF0F3
    nib[..., :256] = (np.arange(256, dtype=np.uint16) << 8) | (nib[..., :256] & 0xF3)
    host[:, 8:10] = nib                                              # 256 high bytes
    host[:, 12:14] = rng.integers(0, 1 << 16, (2, 2, BW))            # incompressible
    highs = rng.choice(256, 50, replace=False).astype(np.uint16)
    host[:, 20:36] = (highs[rng.integers(0, 50, (2, 16, BW))] << 8) | low[:, 20:36]
    kv = layer_from_words(host.reshape(-1), pool)
    tables = [[1, 3], [4, 5, 6], [8, 9], [12, 13], list(range(20, 36))]
    codec = SplitzipLayerCodec(CodecConfig(), trace=RecordingTrace())
    pending = codec.save_kv_layer(2, kv, tables)
    payloads = codec.ready(pending)
    assert [p.bits for p in payloads] == [BITS_TORCHOP] * 3 + [BITS_PASSTHROUGH, BITS_FIXED6]
    for p, mode in zip(payloads[:3], (codec_format.MODE_SIGNMAG, codec_format.MODE_PALETTE,
                                      codec_format.MODE_NIBBLES)):
        blocks = host[:, p.block_ids].reshape(-1)
        assert p.view[0] == mode
        assert bytes(p.view) == bytes(oracle.encode_torchop(blocks))
        assert p.metadata(2, BW)["codec"] == "splitzip_bf16"
    raw = payloads[3]
    assert raw.metadata(2, BW)["codec"] == "raw_passthrough"
    assert raw.encoded_bytes == raw.raw_bytes
    assert bytes(raw.view) == host[:, [12, 13]].tobytes()
    assert bytes(payloads[4].view) == bytes(oracle.fixed6_encode(host[:, 20:36].reshape(-1)))
    names = [f"r{r}" for r in range(len(tables))]
    parts = SplitzipLayerCodec.frames(2, payloads, BW, "t3", names)
    perm = rng.permutation(pool).tolist()
    recv, at = {}, 0
    for name, t in zip(names, tables):
        recv[name] = perm[at:at + len(t)]
        at += len(t)
    target = torch.zeros_like(kv)
    got = codec.restore_frames(target, [b"".join(x[1:]) for x in parts], recv)
    # the same payloads through the per-layer batch restore, metadata as sent
    target2 = torch.zeros_like(kv)
    results = codec.load_kv_layer_batch(2, target2, [
        (recv[name], bytes(p.view), p.metadata(2, BW)) for name, p in zip(names, payloads)])
    torch.cuda.synchronize()
    codec.release(pending)
    for dst_kv in (target, target2):
        dst = u16(dst_kv).reshape(2, pool, BW)
        for name, t in zip(names, tables):
            assert np.array_equal(dst[:, recv[name]], host[:, t]), name
    assert [got[name] for name in names] == [(len(t), 4 * BW * len(t)) for t in tables]
    assert results == [(len(t), 4 * BW * len(t)) for t in tables]
    # UNCHAIN_KV_CODEC_MIN_BLOCKS=3: the requests of fewer blocks get no payload
    # (vllm_connector.py:5315-5321); the others are the same payloads
    short = SplitzipLayerCodec(CodecConfig(min_blocks=3), trace=RecordingTrace())
    pending = short.save_kv_layer(2, kv, tables)
    kept = short.ready(pending)
    assert [p.request for p in kept] == [1, 4]
    assert [bytes(p.view) for p in kept] == [bytes(payloads[1].view), bytes(payloads[4].view)]
    short.release(pending)


# ---------------------------------------------------------------------------
# payload staging: copy stream and pinned pool (vllm_connector.py:3406-3458)

SLEEP_CYCLES = 200_000_000  # about 0.1 s of GPU clock


def _timed_event(stream):
    event = torch.cuda.Event(enable_timing=True)
    event.record(stream)
    return event


def _independent_stream(copy, candidates):
    """A candidate stream whose work is not held back by work on `copy`. HIP
    multiplexes a process's streams over a few hardware queues
    (GPU_MAX_HW_QUEUES), and two streams on one queue run in submission order. A
    marker on the candidate, queued right after a long spin on `copy`, whose GPU
    timestamp comes before the spin's end shows separate queues (event times, no
    polling)."""
    for s in candidates:
        with torch.cuda.stream(copy):
            torch.cuda._sleep(SLEEP_CYCLES)
            spin_end = _timed_event(copy)
        marker = _timed_event(s)
        torch.cuda.synchronize()
        if marker.elapsed_time(spin_end) > 0:
            return s
    return None


def test_payload_copy_runs_beside_the_forward_stream(sz, codebooks):
    """Forward work queued after save_kv_layer does not wait for the layer's
    device-to-host copy: the copy stream is held back by a long spin queued on it
    first, and the GPU timestamps show a marker queued on the forward stream after
    the save hook running before any copy of the layer starts (the copy waits for
    the forward stream's work up to the save, nothing later). The payloads still
    arrive whole."""
    say("connector staging overlap")
    books = codebooks[3 * 32:4 * 32]
    rng = np.random.default_rng(12)
    pool = 1100
    kv = layer_from_words(words_with_books(rng, books, pool, 0.0005), pool)
    tables = disjoint_tables(rng, pool, [256, 256, 256, 256])  # ~50 MB of payloads
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=False, trace_cuda=True))
    copy = codec.copy_streams.get(kv.device, torch)
    forward = _independent_stream(copy, [torch.cuda.Stream() for _ in range(4)])
    assert forward is not None, "every candidate stream shares the copy stream's queue"
    torch.cuda.synchronize()
    with torch.cuda.stream(copy):
        torch.cuda._sleep(SLEEP_CYCLES)
    with torch.cuda.stream(forward):
        pending = codec.save_kv_layer(3, kv, tables)
        marker = _timed_event(forward)            # forward work after the save hook
    starts = [start for kind, start, _ in pending.timing if kind == "d2h"]
    assert starts
    payloads = codec.ready(pending)
    torch.cuda.synchronize()
    assert all(marker.elapsed_time(start) > 0 for start in starts)
    tab = oracle.top16_tables(books)
    src = u16(kv).reshape(2, pool, BW)
    for t, p in zip(tables[:2], payloads[:2]):
        assert bytes(p.view) == bytes(oracle.top16_encode(src[:, t].reshape(-1), tab))
    codec.release(pending)


def test_pinned_pool_reuse_and_cap(sz, codebooks):
    """Released buffers are reused for the next layer (no new pinned allocation);
    with a one-buffer cap a second layer in flight falls back to a fresh pinned
    buffer (trace host_mirror_full); every round trip stays exact."""
    say("connector pinned pool")
    books = codebooks[5 * 32:6 * 32]
    rng = np.random.default_rng(13)
    pool = 80
    kv = layer_from_words(words_with_books(rng, books, pool, 0.001), pool)
    tables = disjoint_tables(rng, pool, [16, 20])
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, host_mirror_layers=1), trace=trace)
    first = codec.save_kv_layer(5, kv, tables)
    second = codec.save_kv_layer(5, kv, tables)          # the cap's one buffer is busy
    assert codec.pinned.allocations == 1
    assert "host_mirror_full" in trace.names()
    a, b = codec.ready(first), codec.ready(second)
    assert [bytes(p.view) for p in a] == [bytes(p.view) for p in b]
    codec.release(first)
    codec.release(second)
    torch.cuda.synchronize()
    payloads = roundtrip(codec, 5, kv, tables, pool)      # reuses the released buffer
    assert codec.pinned.allocations == 1
    assert [bytes(p.view) for p in payloads] == [bytes(p.view) for p in a]


def test_restore_of_reference_ordered_escapes_through_the_host_directory(sz, codebooks):
    """A Top-16 payload whose escape list is in the reference encoder's atomic order
    (shuffled) and whose unused slots hold garbage: the restore builds the escape
    directory on the host (sorting the list in its staging copy) and decodes in one
    kernel, exactly."""
    say("connector restore, shuffled escapes")
    books = codebooks[5 * 32:6 * 32]
    rng = np.random.default_rng(21)
    pool = 64
    kv = layer_from_words(words_with_books(rng, books, pool, 0.002), pool)
    tables = disjoint_tables(rng, pool, [16, 24])
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=RecordingTrace())
    payloads = codec.ready(codec.save_kv_layer(5, kv, tables))
    sent = []
    for p in payloads:
        data = bytearray(p.view)
        n = p.raw_bytes // 2
        lo, hi = codec_format.top16_sections(n)["escapes"]
        count = int.from_bytes(data[1:5], "little")
        assert count > 10
        entries = [bytes(data[lo + 5 * i:lo + 5 * i + 5]) for i in range(count)]
        order = rng.permutation(count)
        data[lo:lo + 5 * count] = b"".join(entries[i] for i in order)
        data[lo + 5 * count:hi] = rng.integers(0, 256, hi - lo - 5 * count, dtype=np.uint8).tobytes()
        sent.append(bytes(data))
    target = torch.zeros_like(kv)
    recv = [[(b + 11) % pool for b in t] for t in tables]
    requests = [(rt, data, p.metadata(5, BW)) for rt, data, p in zip(recv, sent, payloads)]
    assert codec.load_kv_layer_batch(5, target, requests) == [(len(t), 4 * len(t) * BW)
                                                              for t in tables]
    torch.cuda.synchronize()
    src, dst = u16(kv).reshape(2, pool, BW), u16(target).reshape(2, pool, BW)
    for t, rt in zip(tables, recv):
        assert np.array_equal(dst[:, rt], src[:, t])


def test_restore_streams_large_batches_and_resends_sorted_escape_lists(sz, codebooks):
    """About 22 MB of Top-16 payloads in one restore: the staging buffer goes to the
    GPU in several ranges while later payloads are still being staged, and the
    escape lists that arrive in atomic order (two of the payloads, one in the first
    range and one in the last) are sorted by the host directory build after their
    range has left, so they go up again. Every block is restored exactly."""
    say("connector restore, streamed ranges")
    books = codebooks[9 * 32:10 * 32]
    rng = np.random.default_rng(23)
    pool = 9 * 48
    kv = layer_from_words(words_with_books(rng, books, pool, 0.002), pool)
    tables = disjoint_tables(rng, pool, [48] * 9)
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=RecordingTrace())
    payloads = codec.ready(codec.save_kv_layer(9, kv, tables))
    assert sum(p.encoded_bytes for p in payloads) > 16 << 20  # more than one range
    sent = []
    for k, p in enumerate(payloads):
        data = bytearray(p.view)
        if k in (0, 8):
            n = p.raw_bytes // 2
            lo, _ = codec_format.top16_sections(n)["escapes"]
            count = int.from_bytes(data[1:5], "little")
            assert count > 100
            entries = [bytes(data[lo + 5 * i:lo + 5 * i + 5]) for i in range(count)]
            data[lo:lo + 5 * count] = b"".join(entries[i] for i in rng.permutation(count))
        sent.append(bytes(data))
    target = torch.zeros_like(kv)
    recv = [[(b + 5) % pool for b in t] for t in tables]
    requests = [(rt, data, p.metadata(9, BW)) for rt, data, p in zip(recv, sent, payloads)]
    assert codec.load_kv_layer_batch(9, target, requests) == [(len(t), 4 * len(t) * BW)
                                                              for t in tables]
    torch.cuda.synchronize()
    src, dst = u16(kv).reshape(2, pool, BW), u16(target).reshape(2, pool, BW)
    for t, rt in zip(tables, recv):
        assert np.array_equal(dst[:, rt], src[:, t])


def _in_pool(codec, view):
    """The pinned pool buffer that holds a payload's bytes, or None."""
    addr = np.frombuffer(view, np.uint8).ctypes.data
    for slot in codec.pinned._slots:
        base = slot.tensor.data_ptr()
        if base <= addr and addr + len(view) <= base + slot.capacity:
            return slot
    return None


def _spy_copies(codec, monkeypatch):
    """Records the stream of every staging copy the codec queues."""
    used = []
    begin = codec._begin_copies

    def spy(device, torch_):
        stream = begin(device, torch_)
        used.append(stream)
        return stream

    monkeypatch.setattr(codec, "_begin_copies", spy)
    return used


def test_fallback_payloads_are_staged_on_the_copy_stream(sz, codebooks, monkeypatch):
    """An overflowed Top-16 payload's fixed6 re-encode, and a fixed6 overflow's raw
    mode-6 payload, reach the host like every other payload: copies queued on the
    copy stream into pinned pool buffers (no blocking pageable copy), with the
    bytes of the oracle."""
    say("connector fallback staging")
    books = codebooks[2 * 32:3 * 32]
    rng = np.random.default_rng(31)
    pool = 56
    words = words_with_books(rng, books, pool, 0.0)
    kv_host = words.reshape(2, pool, BW)
    tables = disjoint_tables(rng, pool, [16, 16, 3])
    outside = np.array(sorted(set(range(256)) - set(books))[:16], np.uint16)
    for b in tables[1]:                            # 1.2% escapes: Top-16 overflows
        hit = rng.random((2, BW)) < 0.012
        block = kv_host[:, b]
        block[hit] = (block[hit] & 0x807F) | (outside[rng.integers(0, 16, int(hit.sum()))] << 7)
        kv_host[:, b] = block
    for b in tables[2]:                            # every high byte: fixed6 overflows
        kv_host[:, b] = rng.integers(0, 1 << 16, (2, BW))
    kv = layer_from_words(kv_host.reshape(-1), pool)
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=False), trace=RecordingTrace())
    copy = codec.copy_streams.get(kv.device, torch)
    used = _spy_copies(codec, monkeypatch)
    pending = codec.save_kv_layer(2, kv, tables)
    at_save = len(used)
    payloads = codec.ready(pending)
    assert [p.bits for p in payloads] == [BITS_TOP16, BITS_FIXED6, BITS_RAW]
    # ready staged the fixed6 re-encode and the raw payload: two more copies
    assert len(used) == at_save + 2 and all(s is copy for s in used)
    assert copy is not torch.cuda.current_stream(kv.device)
    for p in payloads:
        slot = _in_pool(codec, p.view)
        assert slot is not None and slot.tensor.is_pinned()
    assert bytes(payloads[1].view) == bytes(oracle.fixed6_encode(kv_host[:, tables[1]].reshape(-1)))
    assert payloads[2].view[0] == codec_format.MODE_RAW
    assert bytes(payloads[2].view[1:]) == kv_host[:, tables[2]].tobytes()
    codec.release(pending)


def test_probe_that_fits_copies_its_payload_after_the_mode_byte(sz, codebooks):
    """A probe of a layer that overflowed before stages only the mode byte at save;
    when it fits, ready copies the Top-16 payload (the oracle's bytes) and the
    layer's backoff reopens."""
    say("connector deferred probe that fits")
    books = codebooks[4 * 32:5 * 32]
    rng = np.random.default_rng(33)
    pool = 40
    table = rng.permutation(pool)[:16].tolist()
    normal = words_with_books(rng, books, pool, 0.001)
    over = normal.copy()
    outside = np.array(sorted(set(range(256)) - set(books))[:16], np.uint16)
    hit = rng.random(over.size) < 0.012
    over[hit] = (over[hit] & 0x807F) | (outside[rng.integers(0, 16, int(hit.sum()))] << 7)
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True), trace=trace)
    for words in (over, normal):                   # overflow, then the window's skip
        codec.ready(codec.save_kv_layer(4, layer_from_words(words, pool), [table]))
    pending = codec.save_kv_layer(4, layer_from_words(normal, pool), [table])
    assert pending.payloads[0].probe and not pending.groups and len(pending.deferred) == 1
    payload = codec.ready(pending)[0]
    assert payload.bits == BITS_TOP16 and not payload.fallback
    expect = oracle.top16_encode(normal.reshape(2, pool, BW)[:, table].reshape(-1),
                                 oracle.top16_tables(books))
    assert bytes(payload.view) == bytes(expect)
    assert _in_pool(codec, payload.view) is not None
    assert "splitzip_top16_probe_success" in trace.names()
    assert codec.top16_gate.window(4) == 0


def test_pinned_pool_stays_flat_without_release(sz, codebooks):
    """A caller that never calls release(): each layer's pinned buffer goes back to
    the pool once its payloads' memoryviews are gone, so 12 save -> ready cycles
    allocate no more than two buffers."""
    say("connector pool without release")
    books = codebooks[5 * 32:6 * 32]
    rng = np.random.default_rng(35)
    pool = 48
    kv = layer_from_words(words_with_books(rng, books, pool, 0.001), pool)
    tables = disjoint_tables(rng, pool, [16, 20])
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=False))
    first = None
    for _ in range(12):
        payloads = codec.ready(codec.save_kv_layer(5, kv, tables))
        data = [bytes(p.view) for p in payloads]
        first = first or data
        assert data == first
        del payloads
    assert codec.pinned.allocations <= 2


def test_restore_returns_its_pinned_buffer_when_staging_raises(sz, codebooks, monkeypatch):
    """A restore whose host staging raises (here the copier) hands its pinned buffer
    back to the pool: the next restore of the same layer reuses it and decodes
    exactly."""
    say("connector restore slot on error")
    books = codebooks[5 * 32:6 * 32]
    rng = np.random.default_rng(36)
    pool = 48
    kv = layer_from_words(words_with_books(rng, books, pool, 0.001), pool)
    tables = disjoint_tables(rng, pool, [16, 20])
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=False))
    pending = codec.save_kv_layer(5, kv, tables)
    payloads = codec.ready(pending)
    requests = [(t, p.view, p.metadata(5, kv[0, 0].numel())) for t, p in zip(tables, payloads)]
    receiver = torch.zeros_like(kv)

    def broken(*args, **kwargs):
        raise RuntimeError("staging failed")

    leased = sum(s.leased for s in codec.pinned._slots)  # the saved payloads' buffer
    monkeypatch.setattr(codec.host_copier, "copy_streamed", broken)
    with pytest.raises(RuntimeError, match="staging failed"):
        codec.load_kv_layer_batch(5, receiver, requests)
    torch.cuda.synchronize()
    assert sum(s.leased for s in codec.pinned._slots) == leased
    allocations = codec.pinned.allocations
    monkeypatch.undo()
    got = codec.load_kv_layer_batch(5, receiver, requests)
    torch.cuda.synchronize()
    assert got == [(len(t), 4 * len(t) * kv[0, 0].numel()) for t in tables]
    assert codec.pinned.allocations == allocations
    for t in tables:
        assert torch.equal(receiver[:, t].view(torch.int16), kv[:, t].view(torch.int16))
    codec.release(pending)


def test_payload_ready_carries_gpu_times_on_the_gpu(sz, codebooks):
    """UNCHAIN_KV_TRACE_CUDA=1 on the GPU (vllm_connector.py:473, 4634-4664): the
    splitzip_payload_ready event of a Top-16 layer and of a small-request layer
    (torch-op payloads, whose plan and encode are timed as the layer's encode)
    carries positive GPU times from the recorded events, each payload's bits and
    fallback flag, and the wall time since the save hook began."""
    from unchainkv_amd.connector import BITS_TORCHOP

    say("connector trace_cuda fields")
    books = codebooks[2 * 32:3 * 32]
    rng = np.random.default_rng(31)
    pool = 48
    # no escapes: the small requests' magnitudes then span few bits (sign/magnitude)
    words = words_with_books(rng, books, pool, 0.0)
    kv = layer_from_words(words, pool)
    for config, tables, bits in (
            (CodecConfig(top16=True, writeback=False, trace_cuda=True),
             disjoint_tables(rng, pool, [16, 20]), [BITS_TOP16, BITS_TOP16]),
            (CodecConfig(trace_cuda=True), disjoint_tables(rng, pool, [3, 5]),
             [BITS_TORCHOP, BITS_TORCHOP])):
        trace = RecordingTrace()
        codec = SplitzipLayerCodec(config, trace=trace, codebooks={2: books})
        pending = codec.save_kv_layer(2, kv, tables)
        payloads = codec.ready(pending)
        rows = [f for name, f in trace.rows if name == "splitzip_payload_ready"]
        assert len(rows) == 1
        row = rows[0]
        assert row["bits"] == bits and row["fallback"] == [False, False]
        assert row["encode_gpu_s"] > 0 and row["d2h_gpu_s"] > 0
        assert row["payload_elapsed_s"] > 0
        assert row["encoded_bytes"] == sum(p.encoded_bytes for p in payloads)
        codec.release(pending)
