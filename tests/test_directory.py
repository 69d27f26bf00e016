"""Escape directory of Top-16 payloads, on the CPU: the library's host builder
(kvq_splitzip_top16_build_directory) against an independent numpy construction,
and a numpy emulation of the directory decode (escapes applied per 1024-word
chunk from the record's inline entries, or from the payload's sorted list for
chunks with more) against the oracle's decoder. The directory is this library's
own side data (the wire format is the reference's and unchanged); its GPU use is
checked in tests/test_gpu_directory.py."""

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def sz():
    from unchainkv_amd import splitzip_cuda

    if not splitzip_cuda.available():
        pytest.skip(f"HIP library not built: {splitzip_cuda.load_error()}")
    return splitzip_cuda


def _words(rng, n, books, rate, dense=None):
    """Words drawn from the codebooks with escapes at `rate`; `dense` = (start, count)
    escapes every word of a range."""
    half = n // 2
    outside = np.array(sorted(set(range(256)) - set(books)), dtype=np.uint16)
    exps = np.empty(n, dtype=np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:], np.uint8)[rng.integers(0, 16, n - half)]
    esc = rng.random(n) < rate
    if dense:
        esc[dense[0]:dense[0] + dense[1]] = True
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    low = rng.integers(0, 256, n).astype(np.uint16)
    return ((exps << 7) | (low & 0x7F) | ((low & 0x80) << 8)).astype(np.uint16)


def _batch_payloads(sz, rng, books, block_words, blocks, rate, dense=None):
    batch = sz.PagedBatch([list(range(c)) for c in blocks], block_words, "cpu")
    tables = oracle.top16_tables(books)
    buf = np.zeros(batch.out_bytes, dtype=np.uint8)
    words = []
    for r, c in enumerate(blocks):
        w = _words(rng, 2 * c * block_words, books, rate, dense if r == 0 else None)
        payload = oracle.top16_encode(w, tables)
        buf[batch.out_offsets[r]:batch.out_offsets[r] + payload.size] = payload
        words.append(w)
    return batch, buf, words, tables


def _expected_directory(batch, buf):
    """Independent construction: chunk records and tile bases from the sorted list."""
    tiles = [2 * -(-(n // 2) // 4096) for n in batch.count_words]
    total = sum(tiles)
    rec = np.zeros((total, 4, 4), dtype=np.uint32)
    base = np.zeros(total, dtype=np.uint32)
    t0 = 0
    for r, n in enumerate(batch.count_words):
        payload = buf[batch.out_offsets[r]:batch.out_offsets[r] + batch.encoded_bytes[r]]
        entries = sorted(codec_format.top16_escapes(payload, n), key=lambda e: e[0])
        half, tpp = n // 2, tiles[r] // 2
        pos = np.array([p for p, _ in entries], dtype=np.int64)
        for j in range(2 * tpp):
            plane = int(j >= tpp)
            lo = plane * half + (j - plane * tpp) * 4096
            hi = min(lo + 4096, (plane + 1) * half)
            first = int(np.searchsorted(pos, lo))
            base[t0 + j] = first if payload[0] == 5 else 0
            if payload[0] != 5:
                continue
            for k in range(first, int(np.searchsorted(pos, hi))):
                local = int(pos[k]) - lo
                c = rec[t0 + j, local >> 10]
                count = c[0] >> 16
                if count == 0:
                    c[0] = k - first
                if count < 3:
                    c[1 + count] = (local << 8) | entries[k][1]
                c[0] = (c[0] & 0xFFFF) | ((count + 1) << 16)
        t0 += 2 * tpp
    return rec, base


def _apply_directory(batch, buf, directory, tables):
    """Decode every payload with code-0 words left as decoded, then apply the
    escapes the directory names, chunk by chunk, as the GPU kernel does."""
    total = directory.size // 68
    rec = directory[:64 * total].view(np.uint32).reshape(total, 4, 4)
    base = directory[64 * total:].view(np.uint32)
    out, t0 = [], 0
    for r, n in enumerate(batch.count_words):
        payload = buf[batch.out_offsets[r]:batch.out_offsets[r] + batch.encoded_bytes[r]].copy()
        if payload[0] != 5:
            out.append(None)
            t0 += 2 * -(-(n // 2) // 4096)
            continue
        plain = payload.copy()
        plain[1:5] = 0                     # no escapes: every word from its code
        words = oracle.top16_decode(plain, n, tables)
        entries = codec_format.top16_escapes(payload, n)
        half, tpp = n // 2, -(-(n // 2) // 4096)
        for j in range(2 * tpp):
            plane = int(j >= tpp)
            lo = plane * half + (j - plane * tpp) * 4096
            for w in range(4):
                first, count = int(rec[t0 + j, w, 0] & 0xFFFF), int(rec[t0 + j, w, 0] >> 16)
                if count <= 3:
                    picked = [(lo + (int(e) >> 8), int(e) & 0xFF) for e in rec[t0 + j, w, 1:1 + count]]
                else:
                    s0 = int(base[t0 + j]) + first
                    picked = entries[s0:s0 + count]
                for pos, exponent in picked:
                    assert lo + 1024 * w <= pos < lo + 1024 * w + 1024
                    words[pos] = (words[pos] & 0x807F) | (exponent << 7)
        out.append(words)
        t0 += 2 * tpp
    return out


@pytest.mark.parametrize("block_words,blocks,rate,dense", [
    (1024, [3, 5, 1], 0.004, None),
    (2048, [4, 2], 0.0005, None),
    (16384, [2], 0.0005, (100, 200)),    # one chunk with 200 escapes: the list path
    (1024, [8], 0.004, (5000, 9)),       # chunks with 4..9 escapes
])
def test_host_directory_matches_independent_construction(sz, codebooks, block_words, blocks,
                                                         rate, dense):
    rng = np.random.default_rng(block_words + len(blocks))
    books = codebooks[7 * 32:8 * 32]
    batch, buf, words, tables = _batch_payloads(sz, rng, books, block_words, blocks, rate, dense)
    before = buf.copy()
    directory = sz.build_directory(buf, batch.out_offsets, batch.encoded_bytes, batch)
    assert directory is not None and directory.size == batch.directory_bytes()
    assert np.array_equal(buf, before)      # the oracle's lists are ascending already
    rec, base = _expected_directory(batch, buf)
    total = rec.shape[0]
    got_rec = directory[:64 * total].view(np.uint32).reshape(total, 4, 4)
    got_base = directory[64 * total:].view(np.uint32)
    assert np.array_equal(got_base, base)
    assert np.array_equal(got_rec[:, :, 0] >> 16, rec[:, :, 0] >> 16)       # counts
    used = (rec[:, :, 0] >> 16) > 0
    assert np.array_equal(got_rec[:, :, 0][used], rec[:, :, 0][used])      # first slots
    for i in range(3):
        live = (rec[:, :, 0] >> 16) > i
        assert np.array_equal(got_rec[:, :, 1 + i][live], rec[:, :, 1 + i][live])
    if dense:
        assert (rec[:, :, 0] >> 16).max() > 3
    for got, want in zip(_apply_directory(batch, buf, directory, tables), words):
        assert np.array_equal(got, want)


def test_host_directory_sorts_shuffled_lists_and_keeps_the_decode(sz, codebooks):
    rng = np.random.default_rng(17)
    books = codebooks[:32]
    batch, buf, words, tables = _batch_payloads(sz, rng, books, 2048, [6, 3], 0.003)
    for r, n in enumerate(batch.count_words):
        # the reference encoder's list is in atomic order; padding is never written
        o = batch.out_offsets[r]
        payload = buf[o:o + batch.encoded_bytes[r]]
        lo, _ = codec_format.top16_sections(n)["escapes"]
        count = int.from_bytes(bytes(payload[1:5]), "little")
        entries = payload[lo:lo + 5 * count].reshape(count, 5).copy()
        payload[lo:lo + 5 * count] = entries[rng.permutation(count)].reshape(-1)
        cap = codec_format.top16_escape_capacity(n)
        payload[lo + 5 * count:lo + 5 * cap] = rng.integers(0, 256, 5 * (cap - count))
    directory = sz.build_directory(buf, batch.out_offsets, batch.encoded_bytes, batch)
    for r, n in enumerate(batch.count_words):
        o = batch.out_offsets[r]
        got = codec_format.top16_escapes(buf[o:o + batch.encoded_bytes[r]], n)
        assert [p for p, _ in got] == sorted(p for p, _ in got)
    for got, want in zip(_apply_directory(batch, buf, directory, tables), words):
        assert np.array_equal(got, want)


def test_host_directory_of_overflow_and_unsupported_geometry(sz, codebooks):
    rng = np.random.default_rng(3)
    books = codebooks[:32]
    batch, buf, _, _ = _batch_payloads(sz, rng, books, 1024, [2, 2], 0.02)  # 2 % > 0.5 % cap
    assert all(buf[o] == 255 for o in batch.out_offsets)
    directory = sz.build_directory(buf, batch.out_offsets, batch.encoded_bytes, batch)
    assert directory is not None and not directory.any()
    small = sz.PagedBatch([[0, 1]], 512, "cpu")
    assert small.directory_bytes() == 0
    assert sz.build_directory(np.zeros(small.out_bytes, np.uint8), small.out_offsets,
                              small.encoded_bytes, small) is None
    with pytest.raises(ValueError):
        sz.build_directory(np.zeros(4, np.int16), [0], [4], small)
