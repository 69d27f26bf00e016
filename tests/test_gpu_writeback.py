"""Codec writeback on the GPU: Top-16 payloads moved into the sender's own blocks.

The reference (src/unchain_kv/vllm_connector.py:3460-3563, segments :3720-3738)
copies a payload of a request holding one contiguous block run into the K-plane
run of those blocks, then the V-plane run, and stages the host copy from there.
The checks here are that rule on bytes: after the launch, each run's first bytes
are the payload's bytes (K run first), every other byte of the layer is unchanged,
payloads whose mode byte is not 5 (an overflow) leave their blocks intact, and the
connector's save -> ready -> load round trip still restores the original words.
"""

import ctypes

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format
from unchainkv_amd.connector import BITS_FIXED6, BITS_TOP16, CodecConfig, SplitzipLayerCodec
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


def layer_bytes(kv):
    return kv.detach().contiguous().view(-1).view(torch.uint8).cpu().numpy().copy()


def expected_after(before, payloads, runs, seg_bytes, plane_bytes, block_bytes):
    """The layer's bytes after writing each (payload bytes, run) whose mode byte is 5:
    K-plane run first, then the V-plane run (vllm_connector.py:3512-3521)."""
    exp = before.copy()
    for data, (start, count) in zip(payloads, runs):
        if data[0] != codec_format.MODE_TOP16:
            continue
        seg = seg_bytes(count)
        k = start * block_bytes
        head = min(len(data), seg)
        exp[k:k + head] = data[:head]
        if len(data) > seg:
            exp[plane_bytes + k:plane_bytes + k + len(data) - seg] = data[seg:]
    return exp


def books_words(rng, books, n, escape_rate):
    half = n // 2
    exps = np.empty(n, np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:], np.uint8)[rng.integers(0, 16, n - half)]
    outside = np.array(sorted(set(range(256)) - set(books)), np.uint16)
    esc = rng.random(n) < escape_rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    return ((rng.integers(0, 2, n).astype(np.uint16) << 15) | (exps << 7)
            | rng.integers(0, 128, n).astype(np.uint16))


@pytest.mark.parametrize("bw,pool,runs,hot", [
    (16384, 40, [(2, 3), (10, 4), (20, 1), (30, 8)], 1),  # Llama-3-8B blocks; 16-B path
    (40, 64, [(1, 2), (5, 1), (9, 6), (40, 3)], 2),       # small blocks, runs of 80 B multiples
    (12, 64, [(3, 1), (7, 2), (12, 5), (30, 1)], 0),      # 24-byte runs: byte path
])
def test_writeback_moves_encoded_payloads_into_their_runs(sz, codebooks, bw, pool, runs, hot):
    say("writeback encoded", bw, runs)
    books = codebooks[7 * 32:8 * 32]
    rng = np.random.default_rng(bw)
    words = books_words(rng, books, 2 * pool * bw, 0.0005).reshape(2, pool, bw)
    # request `hot` gets every tenth word escaped (10% > the 0.5% capacity): its
    # Top-16 payload overflows (header 255)
    start, count = runs[hot]
    blk = books_words(rng, books, 2 * count * bw, 0.0)
    outside = sorted(set(range(256)) - set(books))[0]
    blk[::10] = (blk[::10] & 0x807F) | (outside << 7)
    words[:, start:start + count] = blk.reshape(2, count, bw)
    kv = torch.from_numpy(words.reshape(-1).view(np.int16).copy()).cuda().view(
        torch.bfloat16).view(2, pool, bw)
    tables = [list(range(s, s + c)) for s, c in runs]
    batch = sz.PagedBatch(tables, bw, "cuda")
    out = batch.new_payload_buffer()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(),
                                 codebooks=books) == batch.total_encoded_bytes
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    payloads = [host[o:o + e] for o, e in zip(batch.out_offsets, batch.encoded_bytes)]
    assert payloads[hot][0] == codec_format.MODE_OVERFLOW
    before = layer_bytes(kv)
    moved, status = sz.writeback_top16_paged(out, batch, kv, range(len(runs)))
    torch.cuda.synchronize()
    assert moved == batch.total_encoded_bytes
    assert status.cpu().tolist() == [int(p[0]) for p in payloads]
    exp = expected_after(before, payloads, runs, lambda c: 2 * c * bw, 2 * pool * bw, 2 * bw)
    assert np.array_equal(layer_bytes(kv), exp)
    # the moved bytes are the oracle's payloads
    tab = oracle.top16_tables(books)
    for r, t in enumerate(tables):
        if r != hot:
            assert bytes(oracle.top16_encode(words[:, t].reshape(-1), tab)) == bytes(payloads[r])


@pytest.mark.parametrize("misalign", [0, 1, 2, 3])
def test_writeback_any_source_alignment_and_tails(sz, misalign):
    """Synthetic payloads at every byte alignment, with lengths that end inside the
    K run, exactly at it, inside the V run and at its end, and shorter than one
    lane's 20-byte window; a mode byte other than 5 is not written."""
    say("writeback synthetic", misalign)
    bw, pool = 64, 48
    runs = [(0, 1), (2, 3), (6, 2), (9, 1), (11, 4), (16, 1), (18, 2), (21, 3)]
    # run bytes per plane: 128 per block; a payload may fill both planes' runs
    lengths = [1, 19, 256, 128 + 17, 1024, 33, 500, 700]
    modes = [5, 5, 5, 5, 5, 7, 5, 255]
    rng = np.random.default_rng(misalign)
    offsets, at = [], misalign
    for e in lengths:
        offsets.append(at)
        at += e + int(rng.integers(0, 9))
    buf = rng.integers(0, 256, at + 16, dtype=np.uint8)
    for o, m in zip(offsets, modes):
        buf[o] = m
    src = torch.from_numpy(buf).cuda()
    kv = torch.from_numpy(rng.integers(-32768, 32768, 2 * pool * bw).astype(np.int16)).cuda()
    kv = kv.view(torch.bfloat16).view(2, pool, bw)
    before = layer_bytes(kv)
    status = torch.full((len(runs),), 0xAA, dtype=torch.uint8, device="cuda")
    u = ctypes.c_ulonglong
    arr = lambda v: (u * len(v))(*v)  # noqa: E731
    lib = sz._load()
    got = lib.kvq_splitzip_top16_writeback_paged(
        int(src.data_ptr()), arr(offsets), arr(lengths), len(runs), int(kv.data_ptr()),
        kv.stride(0), kv.stride(1), bw, arr([s for s, _ in runs]), arr([c for _, c in runs]),
        int(status.data_ptr()), int(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert got == sum(lengths)
    assert status.cpu().tolist() == modes
    payloads = [buf[o:o + e] for o, e in zip(offsets, lengths)]
    exp = expected_after(before, payloads, runs, lambda c: 2 * c * bw, 2 * pool * bw, 2 * bw)
    assert np.array_equal(layer_bytes(kv), exp)


def test_writeback_more_than_one_launch(sz, codebooks):
    """70 one-block requests: two launches of the 64-payload kernel."""
    say("writeback 70 payloads")
    books = codebooks[3 * 32:4 * 32]
    bw, pool = 2048, 150
    rng = np.random.default_rng(70)
    words = books_words(rng, books, 2 * pool * bw, 0.001).reshape(2, pool, bw)
    kv = torch.from_numpy(words.reshape(-1).view(np.int16).copy()).cuda().view(
        torch.bfloat16).view(2, pool, bw)
    runs = [(2 * r + 1, 1) for r in range(70)]
    batch = sz.PagedBatch([[s] for s, _ in runs], bw, "cuda")
    out = batch.new_payload_buffer()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), codebooks=books)
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    payloads = [host[o:o + e] for o, e in zip(batch.out_offsets, batch.encoded_bytes)]
    before = layer_bytes(kv)
    members = list(range(0, 70, 1))
    moved, status = sz.writeback_top16_paged(out, batch, kv, members)
    torch.cuda.synchronize()
    assert moved == batch.total_encoded_bytes
    assert status.cpu().tolist() == [int(p[0]) for p in payloads]
    exp = expected_after(before, payloads, runs, lambda c: 2 * c * bw, 2 * pool * bw, 2 * bw)
    assert np.array_equal(layer_bytes(kv), exp)


def test_connector_writeback_roundtrip(sz, codebooks):
    """save -> ready -> load with writeback: contiguous requests are moved into
    their blocks, a fragmented one is skipped, an overflowed one keeps its blocks
    and falls back to fixed6; the receiver gets the original words back."""
    say("connector writeback")
    books = codebooks[5 * 32:6 * 32]
    bw, pool = 16384, 96
    rng = np.random.default_rng(5)
    words = books_words(rng, books, 2 * pool * bw, 0.0005).reshape(2, pool, bw)
    tables = [list(range(4, 20)), list(range(30, 48)), [50, 52] + list(range(53, 67)),
              list(range(70, 86))]
    hot = 3
    # 1.2% escapes (over the 0.5% capacity) from 16 exponents outside the codebook,
    # so that the fixed6 palette (at most 64 distinct high bytes) holds them
    blk = books_words(rng, books, 2 * 16 * bw, 0.0)
    outside = np.array(sorted(set(range(256)) - set(books))[:16], np.uint16)
    hit = rng.random(blk.size) < 0.012
    blk[hit] = (blk[hit] & 0x807F) | (outside[rng.integers(0, 16, int(hit.sum()))] << 7)
    words[:, tables[hot]] = blk.reshape(2, 16, bw)
    original = words.copy()
    kv = torch.from_numpy(words.reshape(-1).view(np.int16).copy()).cuda().view(
        torch.bfloat16).view(2, pool, 16, 8, 128)
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True), trace=trace)
    pending = codec.save_kv_layer(5, kv, tables)
    payloads = codec.ready(pending)
    assert [p.bits for p in payloads] == [BITS_TOP16, BITS_TOP16, BITS_TOP16, BITS_FIXED6]
    assert [p.writeback for p in payloads] == [True, True, False, True]
    tab = oracle.top16_tables(books)
    for r in range(3):
        ref = oracle.top16_encode(original[:, tables[r]].reshape(-1), tab)
        assert bytes(payloads[r].view) == bytes(ref)
    assert bytes(payloads[hot].view) == bytes(oracle.fixed6_encode(
        original[:, tables[hot]].reshape(-1)))
    # the moved payloads now occupy their requests' blocks; the rest is unchanged
    after = layer_bytes(kv)
    base = original.reshape(-1).view(np.uint8)
    exp = expected_after(base, [np.frombuffer(bytes(payloads[r].view), np.uint8) for r in (0, 1)],
                         [(tables[r][0], len(tables[r])) for r in (0, 1)],
                         lambda c: 2 * c * bw, 2 * pool * bw, 2 * bw)
    assert np.array_equal(after, exp)
    names = trace.names()
    assert names.count("codec_writeback_submitted") == 3
    assert names.count("codec_writeback_done") == 3
    done = [f for n, f in trace.rows if n == "codec_writeback_done"]
    assert [f["overflow"] for f in done] == [False, False, True]
    skips = [f for n, f in trace.rows if n == "codec_writeback_skip"]
    assert skips == [{"layer": 5, "reason": "fragmented", "segments": 4}]
    # the receiver restores the original words
    target = torch.zeros_like(kv)
    recv = [[(b + 11) % pool for b in t] for t in tables]
    requests = [(rt, bytes(p.view), p.metadata(5, bw)) for rt, p in zip(recv, payloads)]
    codec.load_kv_layer_batch(5, target, requests)
    torch.cuda.synchronize()
    got = target.view(torch.int16).cpu().numpy().view(np.uint16).reshape(2, pool, bw)
    for t, rt in zip(tables, recv):
        assert np.array_equal(got[:, rt], original[:, t])


def test_connector_deferred_writeback_of_early_saves(sz, codebooks):
    """Early-stage saves (vllm_connector.py:2148-2165, 3565-3688): no block is
    overwritten during the early save and its ready; the payloads come from the
    codec buffer, byte-exact. At the layer's next save hook outside the early stage,
    finish_deferred_writebacks with the step's active transfer ids moves the settled
    payloads into their blocks (K run, then V run); the fragmented request and the
    overflowed one keep their blocks; the new save's own request is encoded from
    its untouched blocks."""
    say("connector deferred writeback")
    books = codebooks[5 * 32:6 * 32]
    bw, pool = 16384, 128
    rng = np.random.default_rng(15)
    words = books_words(rng, books, 2 * pool * bw, 0.0005).reshape(2, pool, bw)
    tables = [list(range(4, 20)), list(range(30, 48)), [50, 52] + list(range(53, 67)),
              list(range(70, 86))]
    hot = 3
    blk = books_words(rng, books, 2 * 16 * bw, 0.0)
    outside = np.array(sorted(set(range(256)) - set(books))[:16], np.uint16)
    hit = rng.random(blk.size) < 0.012
    blk[hit] = (blk[hit] & 0x807F) | (outside[rng.integers(0, 16, int(hit.sum()))] << 7)
    words[:, tables[hot]] = blk.reshape(2, 16, bw)
    # the next step's request: no escapes, so fixed6 (at most 64 high bytes) takes it
    words[:, 90:106] = books_words(rng, books, 2 * 16 * bw, 0.0).reshape(2, 16, bw)
    original = words.copy()
    kv = torch.from_numpy(words.reshape(-1).view(np.int16).copy()).cuda().view(
        torch.bfloat16).view(2, pool, 16, 8, 128)
    trace = RecordingTrace()
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True), trace=trace)
    ids = ["req-a", "req-b", "req-c", "req-d"]
    pending = codec.save_kv_layer(5, kv, tables, transfer_ids=ids, early=True)
    payloads = codec.ready(pending)
    assert [p.bits for p in payloads] == [BITS_TOP16, BITS_TOP16, BITS_TOP16, BITS_FIXED6]
    assert not any(p.writeback for p in payloads)
    tab = oracle.top16_tables(books)
    for r in range(3):
        ref = oracle.top16_encode(original[:, tables[r]].reshape(-1), tab)
        assert bytes(payloads[r].view) == bytes(ref)
    assert bytes(payloads[hot].view) == bytes(oracle.fixed6_encode(
        original[:, tables[hot]].reshape(-1)))
    base = original.reshape(-1).view(np.uint8)
    torch.cuda.synchronize()
    assert np.array_equal(layer_bytes(kv), base)
    assert "codec_writeback_submitted" not in trace.names()
    sent = [bytes(p.view) for p in payloads]
    codec.release(pending)
    # the layer's next save hook outside the early stage: the deferred writebacks of
    # the step's active transfers, then the save of a new request
    assert codec.finish_deferred_writebacks(5, kv, ["req-x"]) == 0
    assert len(codec._deferred_codec_writebacks) == 4   # every Top-16 attempt
    moved = codec.finish_deferred_writebacks(5, kv, ids + ["req-e"])
    assert moved == len(sent[0]) + len(sent[1])
    later = [list(range(90, 106))]
    out = codec.ready(codec.save_kv_layer(5, kv, later, transfer_ids=["req-e"]))
    # request d's overflow opened a backoff window on the layer: this save is fixed6
    assert out[0].bits == BITS_FIXED6
    same = bytes(out[0].view) == bytes(oracle.fixed6_encode(original[:, later[0]].reshape(-1)))
    assert same
    torch.cuda.synchronize()
    exp = expected_after(base, [np.frombuffer(sent[r], np.uint8) for r in (0,)],
                         [(tables[0][0], len(tables[0]))], lambda c: 2 * c * bw, 2 * pool * bw,
                         2 * bw)
    # request b's table [30..48) is one run as well
    exp = expected_after(exp, [np.frombuffer(sent[1], np.uint8)], [(30, 18)],
                         lambda c: 2 * c * bw, 2 * pool * bw, 2 * bw)
    assert np.array_equal(layer_bytes(kv), exp)
    early = [(n, f) for n, f in trace.rows if f.get("source") == "early"]
    assert [n for n, _ in early].count("codec_writeback_submitted") == 2
    assert [f["reason"] for n, f in early if n == "codec_writeback_skip"] == \
        ["overflow", "fragmented"]
    assert codec._deferred_codec_writebacks == {}
    # the layer's next Top-16 attempt is the backoff's probe (a Top-16 encode that
    # records presence masks, its payload copied once its mode byte shows it fits):
    # deferred in the early stage too, and moved once its layer is ready
    pend = codec.save_kv_layer(5, kv, [list(range(112, 128))], transfer_ids=["req-f"],
                               early=True)
    assert pend.presence is not None and pend.payloads[0].probe
    got = codec.ready(pend)
    assert got[0].bits == BITS_TOP16
    probe_payload = bytes(got[0].view)
    assert probe_payload == bytes(oracle.top16_encode(original[:, 112:128].reshape(-1), tab))
    torch.cuda.synchronize()
    assert np.array_equal(layer_bytes(kv), exp)
    assert codec.finish_deferred_writebacks(5, kv, ["req-f"]) == len(probe_payload)
    exp = expected_after(exp, [np.frombuffer(probe_payload, np.uint8)], [(112, 16)],
                         lambda c: 2 * c * bw, 2 * pool * bw, 2 * bw)
    torch.cuda.synchronize()
    assert np.array_equal(layer_bytes(kv), exp)
    codec.release(pend)
    # with preserve_source (prefix caching or chunked prefill may reuse the blocks)
    # an early save defers nothing and nothing is ever written into the blocks
    keep = SplitzipLayerCodec(CodecConfig(top16=True, writeback=True, preserve_source=True),
                              trace=RecordingTrace())
    pend = keep.save_kv_layer(5, kv, [list(range(96, 112))], transfer_ids=["req-g"],
                              early=True)
    assert keep.ready(pend)[0].bits == BITS_TOP16
    assert keep._deferred_codec_writebacks == {}
    assert keep.finish_deferred_writebacks(5, kv) == 0
    torch.cuda.synchronize()
    assert np.array_equal(layer_bytes(kv), exp)
    keep.release(pend)
