"""Codec policy of the connector hooks (no GPU): Top-16 backoff, codec choice,
environment knobs and restore validation. The backoff cases follow the
reference's tests/test_vllm_connector.py:2966-3045."""

from concurrent.futures import ThreadPoolExecutor
from types import SimpleNamespace

import pytest

from unchainkv_amd import codec_format
from unchainkv_amd.connector import (BITS_FIXED5, BITS_FIXED6, BITS_TOP16, CodecConfig,
                                     SplitzipLayerCodec)
from unchainkv_amd.trace import RecordingTrace

MIB = 1 << 20


def codec(**kwargs):
    trace = RecordingTrace()
    return SplitzipLayerCodec(CodecConfig(**kwargs), trace=trace), trace


def test_backoff_single_flight_and_recovery():
    c, trace = codec(top16=True, top16_max_cooldown=32)
    attempt = c._should_try_splitzip_top16(7, MIB)
    assert attempt == (True, 0, False)
    c._finish_splitzip_top16_attempt(7, *attempt[1:], True)
    assert c.top16_gate.window(7) == 1
    for expected_window in (2, 4, 8, 16, 32, 32):
        while c.top16_gate.skips_left(7) > 0:
            assert not c._should_try_splitzip_top16(7, MIB)[0]
        with ThreadPoolExecutor(max_workers=8) as pool:
            attempts = list(pool.map(lambda _: c._should_try_splitzip_top16(7, MIB), range(16)))
        probes = [a for a in attempts if a[0]]
        assert len(probes) == 1  # one probe in flight
        c._finish_splitzip_top16_attempt(7, probes[0][1], probes[0][2], True)
        assert c.top16_gate.window(7) == expected_window
    while c.top16_gate.skips_left(7) > 0:
        c._should_try_splitzip_top16(7, MIB)
    probe = c._should_try_splitzip_top16(7, MIB)
    c._finish_splitzip_top16_attempt(7, *probe[1:], False)
    assert c.top16_gate.skips_left(7) is None and c.top16_gate.window(7) == 0
    assert "splitzip_top16_probe_success" in trace.names()
    before = (c.top16_gate.epoch(7), c.top16_gate.skips_left(7))
    assert not c._should_try_splitzip_top16(7, MIB - 1)[0]
    assert (c.top16_gate.epoch(7), c.top16_gate.skips_left(7)) == before


def test_stale_ready_result_cannot_reset_backoff():
    c, trace = codec(top16=True)
    first = c._should_try_splitzip_top16(7, MIB)
    late = c._should_try_splitzip_top16(7, MIB)
    c._finish_splitzip_top16_attempt(7, *first[1:], True)
    c._finish_splitzip_top16_attempt(7, *late[1:], False)
    assert c.top16_gate.skips_left(7) == 1
    assert c.top16_gate.window(7) == 1
    assert trace.names()[-1] == "splitzip_top16_stale_result"


def test_disable_is_sticky_and_epoch_guarded():
    c, trace = codec(top16=True)
    ok, epoch, _ = c._should_try_splitzip_top16(3, MIB)
    c._disable_splitzip_top16(3, epoch + 5)  # stale epoch: ignored
    assert not c.top16_gate.closed(3)
    c._disable_splitzip_top16(3, epoch)
    assert c.top16_gate.closed(3)
    assert not c._should_try_splitzip_top16(3, MIB)[0]
    assert trace.names()[-2:] == ["splitzip_top16_stale_result", "splitzip_top16_unavailable"]


def test_cancelled_probe_allows_the_next_probe():
    c, trace = codec(top16=True)
    first = c._should_try_splitzip_top16(1, MIB)
    c._finish_splitzip_top16_attempt(1, *first[1:], True)  # window 1
    c._should_try_splitzip_top16(1, MIB)  # cooldown 1 -> 0
    probe = c._should_try_splitzip_top16(1, MIB)
    assert probe[0] and probe[2]
    assert not c._should_try_splitzip_top16(1, MIB)[0]  # single flight
    c._cancel_splitzip_top16_probe(1, probe[1], probe[2])
    again = c._should_try_splitzip_top16(1, MIB)
    assert again[0] and again[2] and again[1] == probe[1] + 1
    assert "splitzip_top16_probe_error" in trace.names()


def test_codec_choice_top16_large_fixed6_small_and_fixed5_rules():
    c, _ = codec(top16=True)
    assert c._choose_bits(7, MIB)[0] == BITS_TOP16
    assert c._choose_bits(7, MIB - 2)[0] == BITS_FIXED6
    c5, _ = codec(fixed5=True, fixed5_layers={1, 3})
    assert c5._choose_bits(1, 4096)[0] == BITS_FIXED5
    assert c5._choose_bits(2, 4096)[0] == BITS_FIXED6  # not in the layer list
    c5._splitzip_fixed6_layers.add(3)                   # downgraded after an overflow
    assert c5._choose_bits(3, 4096)[0] == BITS_FIXED6
    both, _ = codec(top16=True, fixed5=True)
    assert both._choose_bits(0, MIB)[0] == BITS_TOP16
    assert both._choose_bits(0, 4096)[0] == BITS_FIXED5
    both.top16_gate.close(0)
    # Top-16 requested but unavailable for the layer: fixed6, not fixed5
    assert both._choose_bits(0, MIB)[0] == BITS_FIXED6


def test_native_codec_from_1_mib_or_with_top16_native_decode():
    """prefer_native (vllm_connector.py:3043-3046): the native codec for 1 MiB or
    more, or for every size while Top-16 with native decode is on; below that the
    torch-op formats."""
    plain, _ = codec()
    assert plain._prefer_native(MIB) and not plain._prefer_native(MIB - 2)
    assert codec(top16=True)[0]._prefer_native(4096)
    no_native = codec(top16=True, native_decode=False)[0]
    assert not no_native._prefer_native(4096) and no_native._prefer_native(MIB)
    assert not codec(fixed5=True)[0]._prefer_native(4096)


def test_torchop_declines_go_raw_and_a_declined_first_half_sends_the_request_whole():
    """A request that no torch-op format compresses is sent as raw words
    (raw_passthrough, vllm_connector.py:2685-2711); a two-chunk request whose first
    half is declined is sent whole with the codec choice for its full size
    (:2741-2747, here a torch-op payload again, or fixed6 from 1 MiB); a declined
    second half alone fails (:2745-2746)."""
    from unchainkv_amd.connector import (BITS_PASSTHROUGH, BITS_TORCHOP, LayerPayload,
                                         PendingLayer)

    bw = 8

    def pending_for(c, tables):
        payloads = []
        for r, ids in enumerate(tables):
            raw = 2 * len(ids) * bw * 2
            if c._two_chunks(ids):
                half = len(ids) // 2
                for k in range(2):
                    payloads.append(LayerPayload(r, ids[k * half:(k + 1) * half], raw // 2,
                                                 BITS_TORCHOP, BITS_TORCHOP, chunk_index=k,
                                                 chunks_in_layer=2, request_blocks=len(ids)))
            else:
                payloads.append(LayerPayload(r, ids, raw, BITS_TORCHOP, BITS_TORCHOP))
        return PendingLayer(3, None, bw, payloads)

    def run(c, pending, declines):
        calls, raw = [], []

        def group(pending_, members, torch):
            calls.append([(p.request, p.chunk_index, p.chunks_in_layer, tuple(p.block_ids))
                          for p in members])
            return [p for p in members if declines(p)]

        def stage(pending_, members, torch):
            raw.extend(members)
            for p in members:
                p.bits = BITS_PASSTHROUGH

        c._torchop_group, c._stage_passthrough = group, stage
        c._torchop_payloads(pending, torch=None)
        return calls, raw

    c, _ = codec(chunks=2)
    pending = pending_for(c, [[1], [10, 11, 12, 13], [20, 21], [30, 31, 32, 33]])
    # request 0 incompressible; request 1's first half declined, its whole request
    # then accepted; request 2's halves accepted; request 3's first half declined and
    # the whole request declined again
    calls, raw = run(c, pending, lambda p: p.request == 0 or
                     (p.request in (1, 3) and p.chunks_in_layer == 2 and p.chunk_index == 0) or
                     (p.request == 3 and p.chunks_in_layer == 1))
    assert calls[0] == [(0, 0, 1, (1,)), (1, 0, 2, (10, 11)), (1, 1, 2, (12, 13)),
                        (2, 0, 2, (20,)), (2, 1, 2, (21,)), (3, 0, 2, (30, 31)),
                        (3, 1, 2, (32, 33))]
    assert calls[1] == [(1, 0, 1, (10, 11, 12, 13)), (3, 0, 1, (30, 31, 32, 33))]
    assert [(p.request, p.chunks_in_layer, p.bits) for p in pending.payloads] == [
        (0, 1, BITS_PASSTHROUGH), (1, 1, BITS_TORCHOP), (2, 2, BITS_TORCHOP),
        (2, 2, BITS_TORCHOP), (3, 1, BITS_PASSTHROUGH)]
    assert [p.request for p in raw] == [0, 3]
    assert pending.payloads[0].metadata(3, bw)["codec"] == "raw_passthrough"
    assert pending.payloads[1].metadata(3, bw)["codec"] == "splitzip_bf16"

    # a whole request of 1 MiB or more goes to the native codec (fixed6)
    big = 1 << 14   # 16 blocks of 64 KiB
    c2, _ = codec(chunks=2)
    bw = big
    pending = pending_for(c2, [list(range(16))])
    calls, raw = run(c2, pending, lambda p: p.chunk_index == 0)
    assert len(calls) == 1 and not raw
    assert [(p.chunks_in_layer, p.bits, p.raw_bytes) for p in pending.payloads] == \
        [(1, BITS_FIXED6, 16 * 4 * big)]

    c3, _ = codec(chunks=2)
    bw = 8
    pending = pending_for(c3, [[5, 6]])
    with pytest.raises(RuntimeError, match="second chunk"):
        run(c3, pending, lambda p: p.chunk_index == 1)


def test_config_from_environment():
    cfg = CodecConfig.from_env({
        "UNCHAIN_KV_SPLITZIP_TOP16": "1",
        "UNCHAIN_KV_SPLITZIP_FIXED5": "1",
        "UNCHAIN_KV_SPLITZIP_FIXED5_LAYERS": "1, 3,5",
        "UNCHAIN_KV_SPLITZIP_TOP16_MAX_COOLDOWN": "0",
        "UNCHAIN_KV_CODEC_MIN_BLOCKS": "64",
    })
    assert cfg.top16 and cfg.fixed5 and cfg.min_blocks == 64
    assert cfg.fixed5_layers == {1, 3, 5}
    assert cfg.top16_max_cooldown == 1  # clamped to at least 1, as the reference does
    default = CodecConfig.from_env({})
    assert not default.top16 and default.top16_max_cooldown == 32 and not default.fixed5_layers
    assert default.min_blocks == 0
    assert CodecConfig.from_env({"UNCHAIN_KV_CODEC_MIN_BLOCKS": "-3"}).min_blocks == 0
    # codec writeback defaults to on with Top-16 (vllm_connector.py:406-412)
    assert cfg.writeback and not default.writeback
    assert not CodecConfig.from_env({"UNCHAIN_KV_SPLITZIP_TOP16": "1",
                                     "UNCHAIN_KV_CODEC_WRITEBACK": "0"}).writeback
    codec = SplitzipLayerCodec(cfg)
    assert codec.codec_writeback and codec.codec_writeback_overwrite
    cfg.preserve_source = True
    assert not SplitzipLayerCodec(cfg).codec_writeback_overwrite


def test_writeback_skips_fragmented_tables():
    from unchainkv_amd.connector import LayerPayload

    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True), trace=trace)
    members = [LayerPayload(0, [4, 5, 6], 3 << 20, BITS_TOP16, BITS_TOP16, encoded_bytes=100),
               LayerPayload(1, [7, 9, 10], 3 << 20, BITS_TOP16, BITS_TOP16, encoded_bytes=100),
               LayerPayload(2, [11], 1 << 20, BITS_TOP16, BITS_TOP16, encoded_bytes=100)]
    assert codec._writeback_members(members, 3) == [0, 2]
    assert trace.rows == [("codec_writeback_skip", {"layer": 3, "reason": "fragmented",
                                                     "segments": 4})]


def test_writeback_skips_blocks_shared_with_another_request():
    """A request whose run shares a block with another request of the layer (prefix
    caching) is not written back: the other request's fallback or raw copy must
    still read the block's KV words."""
    from unchainkv_amd.connector import LayerPayload

    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True), trace=trace)
    a = LayerPayload(0, [4, 5, 6], 3 << 20, BITS_TOP16, BITS_TOP16, encoded_bytes=100)
    b = LayerPayload(1, [6, 7], 2 << 20, BITS_TOP16, BITS_TOP16, encoded_bytes=100)
    c = LayerPayload(2, [9, 10], 2 << 20, BITS_TOP16, BITS_TOP16, encoded_bytes=100)
    d = LayerPayload(3, [10], 1 << 20, BITS_FIXED6, BITS_FIXED6, encoded_bytes=100)
    assert codec._writeback_members([a, b, c], 3, [a, b, c, d]) == []
    assert [e[1]["reason"] for e in trace.rows] == ["shared", "shared", "shared"]
    trace.rows.clear()
    assert codec._writeback_members([a, c], 3, [a, c]) == [0, 1]
    assert trace.rows == []


torch = pytest.importorskip("torch")


@pytest.mark.parametrize("payload,encoded_bytes,raw_bytes", [
    (b"\xff", 1, 16),             # mode out of range
    (b"\x03", 79, 16),            # length differs from the metadata
    (b"\x05" + bytes(4), 5, 16),  # Top-16 size mismatch
    (b"\x06" + bytes(15), 16, 16),  # raw payload one byte short
    (b"\x06" + bytes(16), 17, 12),  # raw_bytes disagrees with the blocks
])
def test_restore_rejects_bad_payloads_before_any_gpu_work(payload, encoded_bytes, raw_bytes):
    """tests/test_vllm_connector.py:2679-2721 of the reference: refused payloads
    never reach the device."""
    c, _ = codec()
    kv = torch.zeros((2, 2, 2), dtype=torch.bfloat16)  # CPU tensor: any GPU use would fail
    got = c.load_kv_layer_batch(0, kv, [([0, 1], payload, {"raw_bytes": raw_bytes,
                                                          "encoded_bytes": encoded_bytes})])
    assert got == [(0, 0)]


@pytest.mark.parametrize("payload", [
    b"\x01\x00\x00",                                   # nibble planes: shorter than the header
    b"\x01\x04\x04\x04\x03" + bytes(64) + bytes(16),   # a plane width of 3
    b"\x02\x07\x00" + bytes(8 + 1 + 7),                # sign/magnitude width 7
    b"\x02\x01\x00" + bytes(8 + 1 + 1 + 1),            # one byte too long
    b"\x00\x00" + bytes(256 + 8 + 1),                   # palette width 0
])
def test_restore_refuses_torchop_payloads_with_bad_headers(payload):
    """Modes 0, 1 and 2 pass the reference's header checks
    (vllm_connector.py:5168-5252) before any GPU work (a CPU layer here)."""
    c, trace = codec()
    kv = torch.zeros((2, 2, 2), dtype=torch.bfloat16)
    meta = {"raw_bytes": 16, "encoded_bytes": len(payload)}
    assert c.load_kv_layer_batch(0, kv, [([0, 1], payload, meta)]) == [(0, 0)]
    assert trace.names() == []


def test_torchop_sizes_follow_the_reference_rules():
    n = 8
    assert codec_format.torchop_encoded_size(b"\x02\x01\x00", n) == 3 + 8 + 1 + 1
    assert codec_format.torchop_encoded_size(b"\x02\x06\x05", n) == 3 + 8 + 1 + 6
    head = bytes([1, 4, 2, 1, 4]) + bytes(64)
    assert codec_format.torchop_encoded_size(head, n) == 69 + 4 + 2 + 1 + 4
    assert codec_format.torchop_encoded_size(bytes([0, 7]) + bytes(256), n) == 258 + 8 + 7
    assert codec_format.torchop_encoded_size(bytes([0, 8]) + bytes(256), n) is None
    assert codec_format.torchop_encoded_size(b"\x05", n) is None


def test_restore_rejects_bad_blocks():
    c, trace = codec()
    kv = torch.zeros((2, 4, 2), dtype=torch.bfloat16)
    raw = {"raw_bytes": 16, "encoded_bytes": 17}
    assert c.load_kv_layer_batch(0, kv, [([0, 0], b"\x06" + bytes(16), raw)]) == [(0, 0)]
    assert c.load_kv_layer_batch(0, kv, [([0, 9], b"\x06" + bytes(16), raw)]) == [(0, 0)]
    assert codec_format.MODE_RAW == 6


def test_exponent_trace_once_per_transfer_layer_and_retry_after_error():
    """bf16_exponent_stats is emitted once per (transfer, layer) with the
    summarised K and V histograms; a failure emits bf16_exponent_stats_error and
    leaves the key free for a retry (vllm_connector.py:2871-2904)."""
    import numpy as np

    class FakeCounts:
        def __init__(self, rows):
            self.rows = rows

        def cpu(self):
            return self

        def tolist(self):
            return self.rows

    k = [0] * 256
    v = [0] * 256
    k[120], k[121], v[110] = 30, 10, 40
    calls = []

    class FakeLib:
        fail = True

        def available(self):
            return True

        def PagedBatch(self, tables, block_words, device):
            calls.append((tables, block_words))
            return SimpleNamespace()

        def exponent_histogram_paged(self, kv, batch):
            if FakeLib.fail:
                raise RuntimeError("boom")
            return FakeCounts([k, v])

    class FakeLayer:
        device = "cuda:0"

        def __getitem__(self, index):
            return SimpleNamespace(numel=lambda: 2048)

    trace = RecordingTrace()
    c = SplitzipLayerCodec(CodecConfig(), trace=trace, lib=FakeLib())
    c._trace_bf16_exponents(FakeLayer(), [[3, 4]], "t1", 2)
    assert trace.names()[-1] == "bf16_exponent_stats_error"
    FakeLib.fail = False
    c._trace_bf16_exponents(FakeLayer(), [[3, 4]], "t1", 2)
    c._trace_bf16_exponents(FakeLayer(), [[3, 4]], "t1", 2)  # traced already
    stats = [e for e in trace.rows if e[0] == "bf16_exponent_stats"]
    assert len(stats) == 1
    fields = stats[0][1]
    assert fields["transfer"] == "t1" and fields["layer"] == 2
    assert fields["k"]["words"] == 40 and fields["k"]["top8_exponents"][:2] == [120, 121]
    assert fields["v"]["unique_exponents"] == 1
    assert np.isclose(fields["k"]["top16_coverage"], 1.0)
    assert calls[-1] == ([[3, 4]], 2048)


def test_writeback_skips_a_layer_that_is_not_contiguous():
    from types import SimpleNamespace

    from unchainkv_amd.connector import LayerPayload, PendingLayer

    class FakeLib:
        @staticmethod
        def available():
            return True

        @staticmethod
        def writeback_top16_paged(*args, **kwargs):
            raise AssertionError("not called for a non-contiguous layer")

    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True), trace=trace,
                               lib=FakeLib())
    layer = SimpleNamespace(is_contiguous=lambda: False)
    members = [LayerPayload(0, [4, 5], 2 * MIB, BITS_TOP16, BITS_TOP16, encoded_bytes=100)]
    pending = PendingLayer(7, layer, 16384, members)
    assert not codec._stage_writeback(pending, members, (None, [0], [100], None), None)
    assert trace.rows == [("codec_writeback_skip", {"layer": 7, "reason": "layout"})]


def test_deferred_writebacks_finish_only_settled_payloads_of_their_layer():
    """Early-stage writebacks (vllm_connector.py:3565-3718): at the layer's next
    finish, payloads whose layer is not ready yet, that overflowed, or whose blocks
    are fragmented are skipped; the rest of one encode group go to one writeback
    launch; entries of other layers and transfer ids stay until their own finish or
    a cancel."""
    from types import SimpleNamespace

    from unchainkv_amd.connector import LayerPayload, PendingLayer

    calls = []

    class FakeLib:
        @staticmethod
        def available():
            return True

        @staticmethod
        def writeback_top16_paged(out, batch, kv_layer, members):
            calls.append((out, batch, kv_layer, list(members)))
            return 700, None

    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True), trace=trace,
                               lib=FakeLib())
    layer = SimpleNamespace(is_contiguous=lambda: True)

    def payload(r, ids, bits=BITS_TOP16):
        return LayerPayload(r, ids, 2 * MIB, bits, BITS_TOP16, encoded_bytes=300)

    a, b, c, d = payload(0, [4, 5]), payload(1, [7, 9]), payload(2, [11, 12]), payload(3, [20])
    c.bits, c.fallback = BITS_FIXED6, True          # overflowed -> fixed6 in ready()
    settled = PendingLayer(3, layer, 16384, [a, b, c, d], ready_done=True)
    result = ("codec buffer", [0, 300, 600, 900], [300] * 4, "batch")
    e = payload(0, [30, 31])
    unsettled = PendingLayer(4, layer, 16384, [e])
    f = payload(5, [40])
    other = PendingLayer(3, layer, 16384, [f], ready_done=True)
    for p in (a, b, c, d, e, f):
        p.deferred_writeback = True
    codec._deferred_codec_writebacks.update({
        ("t0", 3): (settled, a, result, 0), ("t1", 3): (settled, b, result, 1),
        ("t2", 3): (settled, c, result, 2), ("t3", 3): (settled, d, result, 3),
        ("t0", 4): (unsettled, e, ("buf", [0], [300], "b4"), 0),
        ("t5", 3): (other, f, ("buf5", [0], [300], "b5"), 0)})

    assert codec.finish_deferred_writebacks(3, layer, ["t0", "t1", "t2", "t3"]) == 700
    assert calls == [("codec buffer", "batch", layer, [0, 3])]
    assert not any(p.deferred_writeback for p in (a, b, c, d))
    assert trace.rows == [
        ("codec_writeback_skip", {"layer": 3, "reason": "overflow", "source": "early"}),
        ("codec_writeback_skip", {"layer": 3, "reason": "fragmented", "segments": 4,
                                  "source": "early"}),
        ("codec_writeback_submitted", {"layer": 3, "bytes": 300, "raw_bytes": 2 * MIB,
                                       "segments": 2, "source": "early"}),
        ("codec_writeback_submitted", {"layer": 3, "bytes": 300, "raw_bytes": 2 * MIB,
                                       "segments": 2, "source": "early"})]
    assert set(codec._deferred_codec_writebacks) == {("t0", 4), ("t5", 3)}
    trace.rows.clear()
    calls.clear()
    # a layer whose ready() has not returned: skipped and dropped, nothing launched
    assert codec.finish_deferred_writebacks(4, layer) == 0
    assert calls == [] and not e.deferred_writeback
    assert trace.rows == [("codec_writeback_skip", {"layer": 4, "reason": "d2h_pending",
                                                     "source": "early"})]
    trace.rows.clear()
    assert codec.cancel_deferred_writebacks(transfer_ids=["t9"]) == 0
    assert codec.cancel_deferred_writebacks(layer_index=3, reason="metadata_clear") == 1
    assert codec._deferred_codec_writebacks == {} and not f.deferred_writeback
    assert trace.rows == [("codec_writeback_skip", {"layer": 3, "reason": "metadata_clear",
                                                     "source": "early"})]


def test_two_chunk_rule_and_kvc2_frames():
    """UNCHAIN_KV_SPLITZIP_CHUNKS=2 (vllm_connector.py:446-447, 2718-2737): only
    with neither Top-16 nor fixed5 enabled, and only for an even number of blocks
    in one ascending run; each half's frame is KVC2 with the whole request's block
    count and raw bytes (:5551-5563)."""
    from unchainkv_amd import frames
    from unchainkv_amd.connector import LayerPayload

    assert CodecConfig.from_env({"UNCHAIN_KV_SPLITZIP_CHUNKS": "2"}).chunks == 2
    assert CodecConfig.from_env({"UNCHAIN_KV_SPLITZIP_CHUNKS": "3"}).chunks == 1
    two, _ = codec(chunks=2)
    assert two._two_chunks([4, 5, 6, 7]) and two._two_chunks([9, 10])
    assert not two._two_chunks([4, 5, 6])         # odd
    assert not two._two_chunks([4])               # a single block
    assert not two._two_chunks([4, 6, 5, 7])      # not one ascending run
    assert not codec(chunks=2, top16=True)[0]._two_chunks([4, 5, 6, 7])
    assert not codec(chunks=2, fixed5=True)[0]._two_chunks([4, 5, 6, 7])
    assert not codec()[0]._two_chunks([4, 5, 6, 7])

    bw = 8
    halves = []
    for k, ids in enumerate(([4, 5], [6, 7])):
        p = LayerPayload(0, ids, 2 * 2 * bw * 2, BITS_FIXED6, BITS_FIXED6, chunk_index=k,
                         chunks_in_layer=2, request_blocks=4)
        p.view = memoryview(bytes([3]) + bytes(40 + k))
        p.encoded_bytes = len(p.view)
        halves.append(p)
    whole = LayerPayload(1, [9], 2 * bw * 2, BITS_FIXED6, BITS_FIXED6)
    whole.view = memoryview(bytes([3]) + bytes(30))
    whole.encoded_bytes = len(whole.view)
    parts = SplitzipLayerCodec.frames(7, halves + [whole], bw, "t", ["req-a", "req-b"])
    parsed = [frames.parse_compressed_native(b"".join(p[1:])) for p in parts]
    for k, f in enumerate(parsed[:2]):
        assert (f.request_id, f.layer_index, f.chunk_index, f.chunks_in_layer) == ("req-a", 7, k, 2)
        assert (f.block_count, f.raw_block_size, f.raw_bytes) == (4, 2 * bw * 2, 4 * 2 * bw * 2)
        assert bytes(f.payload) == bytes(halves[k].view)
    assert (parsed[2].chunks_in_layer, parsed[2].block_count, parsed[2].request_id) == (1, 1, "req-b")


def test_batches_are_reused_for_recurring_block_tables():
    """The codec builds one PagedBatch per block-table set and reuses it while the
    set recurs (a request keeps its block ids in every layer); the least recently
    used set goes once more than BATCH_CACHE sets are held."""
    built = []

    class FakeLib:
        def available(self):
            return True

        def PagedBatch(self, tables, block_words, device):
            built.append((tuple(map(tuple, tables)), block_words, device))
            return SimpleNamespace(tables=tables)

    c = SplitzipLayerCodec(CodecConfig(), trace=RecordingTrace(), lib=FakeLib())
    a = c._batch([[1, 2], [7]], 2048, "cuda:0")
    assert c._batch([[1, 2], [7]], 2048, "cuda:0") is a
    assert c._batch([(1, 2), (7,)], 2048, "cuda:0") is a    # same ids, any sequence type
    assert c._batch([[1, 2], [7]], 1024, "cuda:0") is not a  # other geometry
    assert c._batch([[1, 2], [7]], 2048, "cuda:1") is not a  # other device
    assert len(built) == 3
    for k in range(c.BATCH_CACHE):
        c._batch([[100 + k]], 2048, "cuda:0")
    assert len(c._batches) == c.BATCH_CACHE
    before = len(built)
    c._batch([[1, 2], [7]], 2048, "cuda:0")  # evicted meanwhile: built again
    assert len(built) == before + 1
    c._batch([[100 + c.BATCH_CACHE - 1]], 2048, "cuda:0")  # still held
    assert len(built) == before + 1


class _FakeEvent:
    """A completed GPU event whose timestamp is ``ms``."""

    def __init__(self, ms):
        self.ms = ms

    def synchronize(self):
        pass

    def query(self):
        return True

    def elapsed_time(self, end):
        return end.ms - self.ms


def test_payload_ready_carries_gpu_timing_under_trace_cuda():
    """UNCHAIN_KV_TRACE_CUDA=1 adds the GPU time of the layer's encodes and copies
    to the splitzip_payload_ready event (vllm_connector.py:473, 4634-4664): the sums
    of the recorded (start, end) event pairs in seconds, each payload's bits and
    fallback flag, and the time since the save hook began. Without it the event
    carries the byte counts only."""
    import numpy as np

    from unchainkv_amd.connector import LayerPayload, PendingLayer

    assert CodecConfig.from_env({"UNCHAIN_KV_TRACE_CUDA": "1"}).trace_cuda
    assert not CodecConfig.from_env({}).trace_cuda
    for traced in (True, False):
        c, trace = codec(top16=True, trace_cuda=traced)
        host = np.zeros(64, np.uint8)
        host[0], host[32] = codec_format.MODE_TOP16, codec_format.MODE_FIXED6
        payloads = [LayerPayload(0, [1], 2 * MIB, BITS_TOP16, BITS_TOP16, epoch=0,
                                 encoded_bytes=20, _group=0, _offset=0),
                    LayerPayload(1, [2], 2 * MIB, BITS_FIXED6, BITS_FIXED6,
                                 encoded_bytes=24, _group=0, _offset=32)]
        pending = PendingLayer(3, None, 16384, payloads, started=0.0)
        pending.groups.append((host, _FakeEvent(9.0), None, None))
        pending.timing += [("encode", _FakeEvent(1.0), _FakeEvent(1.25)),
                           ("d2h", _FakeEvent(1.5), _FakeEvent(3.5)),
                           ("encode", _FakeEvent(4.0), _FakeEvent(4.5)),
                           ("d2h", _FakeEvent(5.0), _FakeEvent(5.5))]
        got = c.ready(pending)
        assert [bytes(p.view)[:1] for p in got] == [bytes([5]), bytes([3])]
        row = next(f for name, f in trace.rows if name == "splitzip_payload_ready")
        assert row["raw_bytes"] == 4 * MIB and row["encoded_bytes"] == 44
        if traced:
            assert row["encode_gpu_s"] == pytest.approx(0.00075)
            assert row["d2h_gpu_s"] == pytest.approx(0.0025)
            assert row["bits"] == [BITS_TOP16, BITS_FIXED6]
            assert row["fallback"] == [False, False]
            assert row["payload_elapsed_s"] > 0
        else:
            assert set(row) == {"layer", "raw_bytes", "encoded_bytes"}
        assert not pending.timing


def test_save_needs_one_transfer_id_per_block_table():
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True))
    with pytest.raises(ValueError, match="transfer id"):
        codec.save_kv_layer(0, object(), [[1], [2]], transfer_ids=["only-one"], early=True)


def test_cancel_deferred_writebacks_by_transfer_and_layer():
    from unchainkv_amd.connector import LayerPayload

    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True), trace=trace)
    entries = {}
    for tid in ("a", "b"):
        for layer in (1, 2):
            p = LayerPayload(0, [layer], 2 * MIB, BITS_TOP16, BITS_TOP16, encoded_bytes=9)
            p.deferred_writeback = True
            entries[(tid, layer)] = (None, p, None, 0)
    codec._deferred_codec_writebacks.update(entries)
    assert codec.cancel_deferred_writebacks(["a"], reason="request_finished") == 2
    assert set(codec._deferred_codec_writebacks) == {("b", 1), ("b", 2)}
    assert not entries[("a", 1)][1].deferred_writeback
    assert codec.cancel_deferred_writebacks(layer_index=2) == 1
    assert set(codec._deferred_codec_writebacks) == {("b", 1)}
    assert [f["reason"] for _, f in trace.rows] == ["request_finished"] * 2 + ["cancelled"]
    assert all(f["source"] == "early" for _, f in trace.rows)
