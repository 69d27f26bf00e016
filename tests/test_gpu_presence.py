"""Top-16 encode that also writes each tile's high-byte presence mask, and the
palette (fixed6/fixed5) re-encode of overflowed requests that starts from those
masks instead of a presence pass of its own.

Checked against: the masks computed with numpy from the gathered words (one
256-bit mask per 4096-word tile of each plane), the Top-16 payload bytes of the
plain encode and of the oracle, and the palette payload bytes of the plain
palette encode and of the oracle, for overflowed subsets in any order, including
a request whose distinct high bytes exceed the palette (byte 0 = 255 alone)."""

import numpy as np
import pytest

import oracle

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


def u8(t) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy()


def request_words(rng, n, books, outlier_rate, distinct_highs):
    """Words whose exponents come from each plane's codebook except a fraction
    `outlier_rate` (any exponent); or, with `distinct_highs`, words over that many
    random high bytes (almost all of them escapes: the Top-16 payload overflows)."""
    if distinct_highs is not None:
        highs = rng.choice(256, distinct_highs, replace=False).astype(np.uint16)
        return ((highs[rng.integers(0, distinct_highs, n)] << 8) |
                rng.integers(0, 256, n).astype(np.uint16)).astype(np.uint16)
    half = n // 2
    exps = np.empty(n, np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:32], np.uint8)[rng.integers(0, 16, n - half)]
    hits = rng.random(n) < outlier_rate
    exps[hits] = rng.integers(0, 256, int(hits.sum()))
    return ((exps << 7) | rng.integers(0, 128, n).astype(np.uint16) |
            (rng.integers(0, 2, n).astype(np.uint16) << 15)).astype(np.uint16)


def masks_of(words, tile=4096):
    """(tiles, 8) uint32 presence masks of one payload's words, per plane."""
    half = words.size // 2
    out = []
    for p in range(2):
        plane = words[p * half:(p + 1) * half]
        for j in range(0, half, tile):
            m = np.zeros(8, np.uint32)
            for h in np.unique(plane[j:j + tile] >> 8):
                m[h >> 5] |= np.uint32(1 << (int(h) & 31))
            out.append(m)
    return np.array(out, np.uint32)


def build(rng, books, bw, requests):
    """Layer (2, pool, bw) with each request's words in shuffled blocks."""
    pool = sum(c for c, _, _ in requests) + 3
    perm = rng.permutation(pool).tolist()
    layer = np.zeros((2, pool, bw), np.uint16)
    tables, words, at = [], [], 0
    for count, rate, distinct in requests:
        ids = perm[at:at + count]
        at += count
        w = request_words(rng, 2 * count * bw, books, rate, distinct)
        layer[:, ids] = w.reshape(2, count, bw)
        tables.append(ids)
        words.append(w)
    kv = torch.from_numpy(layer.view(np.int16)).cuda().view(torch.bfloat16)
    return kv, tables, words


@pytest.mark.parametrize("bw", [16384, 1024, 3072])
@pytest.mark.parametrize("bits", [6, 5])
def test_presence_masks_and_palette_fallback_without_presence_pass(sz, codebooks, bw, bits):
    say("presence", bw, bits)
    rng = np.random.default_rng(bw + bits)
    books = codebooks[3 * 32:4 * 32]
    limit = 64 if bits == 6 else 32
    # (blocks, outlier rate, distinct high bytes): the requests with few distinct
    # high bytes overflow Top-16 and fit the palette, except one with more high
    # bytes than palette entries
    requests = [(3, 0.0, limit - 5), (2, 0.0, None), (5, 0.0, limit), (1, 0.0, limit + 9),
                (4, 0.001, None), (2, 0.0, 7)]
    if bw == 1024:
        requests = [(c * 8 + 1, r, d) for c, r, d in requests]
    kv, tables, words = build(rng, books, bw, requests)
    tables_t = torch.from_numpy(oracle.top16_tables(books).copy()).cuda()
    batch = sz.PagedBatch(tables, bw, "cuda")

    plain = batch.new_payload_buffer()
    assert sz.encode_top16_paged(kv, batch, plain, batch.new_workspace(), tables=tables_t) == \
        batch.total_encoded_bytes
    out = batch.new_payload_buffer()
    presence = batch.new_presence()
    assert presence is not None and presence.numel() == batch.presence_bytes()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), tables=tables_t,
                                 presence=presence) == batch.total_encoded_bytes
    torch.cuda.synchronize()
    got, ref_plain = u8(out), u8(plain)
    for o, e in zip(batch.out_offsets, batch.encoded_bytes):
        assert bytes(got[o:o + e]) == bytes(ref_plain[o:o + e])

    masks = u8(presence).view(np.uint32).reshape(-1, 8)
    firsts = batch.presence_first(range(batch.payload_count))
    overflowed = []
    for r, w in enumerate(words):
        o, e = batch.out_offsets[r], batch.encoded_bytes[r]
        ref = oracle.top16_encode(w, oracle.top16_tables(books))
        assert bytes(got[o:o + e]) == bytes(ref), f"top16 payload {r}"
        expect = masks_of(w)
        assert np.array_equal(masks[firsts[r]:firsts[r] + len(expect)], expect), f"masks {r}"
        if ref[0] == 255:
            overflowed.append(r)
    assert len(overflowed) >= 3

    # the fallback re-encode of the overflowed requests, in another order
    members = overflowed[::-1]
    sub = sz.PagedBatch([tables[r] for r in members], bw, "cuda")
    offsets, sizes, _ = sub.palette_layout(bits)
    plain6 = sub.new_palette_buffer(bits)
    assert sz.encode_bf16_paged(kv, sub, plain6, sub.new_palette_workspace(), bits=bits) == \
        sum(sizes)
    fast6 = torch.full_like(plain6, 0x5A)
    assert sz.encode_bf16_paged(kv, sub, fast6, sub.new_palette_workspace(), bits=bits,
                                presence=presence,
                                presence_first=batch.presence_first(members)) == sum(sizes)
    torch.cuda.synchronize()
    a, b = u8(plain6), u8(fast6)
    for k, r in enumerate(members):
        ref = oracle.palette_encode(words[r], bits)
        o = offsets[k]
        if ref[0] == 255:
            assert b[o] == 255 and a[o] == 255
            continue
        assert bytes(b[o:o + sizes[k]]) == bytes(ref), f"palette payload {r}"
        assert bytes(a[o:o + sizes[k]]) == bytes(ref)


def test_presence_is_declined_without_tile_geometry(sz, codebooks):
    say("presence declined")
    books = codebooks[:32]
    kv = torch.zeros((2, 8, 16, 1, 24), dtype=torch.bfloat16, device="cuda")  # 384-word blocks
    batch = sz.PagedBatch([[0, 1], [3]], 384, "cuda")
    assert batch.presence_bytes() == 0 and batch.new_presence() is None
    tables_t = torch.from_numpy(oracle.top16_tables(books).copy()).cuda()
    dummy = torch.empty(4096, dtype=torch.uint8, device="cuda")
    assert sz.encode_top16_paged(kv, batch, batch.new_payload_buffer(), batch.new_workspace(),
                                 tables=tables_t, presence=dummy) is None


def palette_record(words):
    """The 512-byte palette record of one payload's words, as the probe encode
    writes it: 256-bit presence mask, distinct count, rank table (0 for absent
    bytes) at byte 64, ascending palette of up to 64 bytes at byte 320."""
    highs = np.unique(words >> 8).astype(np.int64)
    rec = np.zeros(512, np.uint8)
    mask = np.zeros(8, np.uint32)
    for h in highs:
        mask[h >> 5] |= np.uint32(1 << (int(h) & 31))
    rec[0:32] = mask.view(np.uint8)
    rec[32:36] = np.array([highs.size], np.uint32).view(np.uint8)
    rank = np.zeros(256, np.uint8)
    rank[highs] = np.arange(highs.size) % 256
    rec[64:320] = rank
    rec[320:320 + min(64, highs.size)] = highs[:64]
    return rec


@pytest.mark.parametrize("bw", [16384, 1024])
@pytest.mark.parametrize("bits", [6, 5])
def test_probe_encode_palettes_and_unplaced_overflow(sz, codebooks, bw, bits):
    """The probe encode (presence masks + palette records, no escape placement in an
    overflowed payload): payloads that fit are the oracle's bytes; overflowed
    payloads have the oracle's header, body and codes; every palette record equals
    numpy's; the palette re-encode from the records (one pass) equals the oracle's
    fixed6 / fixed5 payloads, for a subset of the requests in another order."""
    say("probe", bw, bits)
    rng = np.random.default_rng(3 * bw + bits)
    books = codebooks[6 * 32:7 * 32]
    limit = 64 if bits == 6 else 32
    requests = [(3, 0.0, limit - 5), (2, 0.0, None), (5, 0.0, limit), (1, 0.0, limit + 9),
                (4, 0.001, None), (2, 0.0, 7), (3, 0.012, None)]
    if bw == 1024:
        requests = [(c * 8 + 1, r, d) for c, r, d in requests]
    kv, tables, words = build(rng, books, bw, requests)
    tab = oracle.top16_tables(books)
    tables_t = torch.from_numpy(tab.copy()).cuda()
    batch = sz.PagedBatch(tables, bw, "cuda")
    out = torch.full((batch.out_bytes,), 0xA5, dtype=torch.uint8, device="cuda")
    presence, info = batch.new_presence(), batch.new_palette_info()
    directory = batch.new_directory()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), tables=tables_t,
                                 presence=presence, palette_info=info,
                                 directory=directory) == batch.total_encoded_bytes
    torch.cuda.synchronize()
    got, records = u8(out), u8(info).reshape(-1, 512)
    overflowed = []
    for r, w in enumerate(words):
        o, e = batch.out_offsets[r], batch.encoded_bytes[r]
        ref = oracle.top16_encode(w, tab)
        n = w.size
        if ref[0] == 255:
            overflowed.append(r)
            body_end = 5 + n + (n + 1) // 2
            assert bytes(got[o:o + body_end]) == bytes(ref[:body_end]), f"overflowed {r}"
            assert not got[o + body_end:o + e].any(), f"escape slots of {r}"
        else:
            assert bytes(got[o:o + e]) == bytes(ref), f"payload {r}"
        want = palette_record(w)
        # mask and distinct count, rank table and palette (the padding is not written)
        assert bytes(records[r][:36]) == bytes(want[:36]), f"palette record {r}"
        assert bytes(records[r][64:384]) == bytes(want[64:384]), f"palette record {r}"
    assert len(overflowed) >= 4
    # the fitting payloads decode through the directory the probe wrote
    target = torch.zeros_like(kv)
    assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, batch,
                                 tables=tables_t, directory=directory) == batch.total_raw_bytes
    torch.cuda.synchronize()
    src, dst = u8(kv.view(torch.uint8)), u8(target.view(torch.uint8))
    pool = kv.shape[1]
    for r, t in enumerate(tables):
        if r not in overflowed:
            assert np.array_equal(dst.reshape(2, pool, -1)[:, t], src.reshape(2, pool, -1)[:, t])
    members = overflowed[::-1]
    sub = sz.PagedBatch([tables[r] for r in members], bw, "cuda")
    offsets, sizes, _ = sub.palette_layout(bits)
    fast = torch.full_like(sub.new_palette_buffer(bits), 0x5A)
    assert sz.encode_bf16_paged(kv, sub, fast, None, bits=bits, palette_info=info,
                                info_first=members) == sum(sizes)
    torch.cuda.synchronize()
    b = u8(fast)
    for k, r in enumerate(members):
        ref = oracle.palette_encode(words[r], bits)
        o = offsets[k]
        if ref[0] == 255:
            assert b[o] == 255
            continue
        assert bytes(b[o:o + sizes[k]]) == bytes(ref), f"palette payload {r}"


def test_probe_needs_presence_and_info_indices_in_range(sz, codebooks):
    say("probe declines")
    books = codebooks[:32]
    rng = np.random.default_rng(8)
    kv, tables, words = build(rng, books, 16384, [(2, 0.0, 7), (1, 0.0, 9)])
    batch = sz.PagedBatch(tables, 16384, "cuda")
    tables_t = torch.from_numpy(oracle.top16_tables(books).copy()).cuda()
    with pytest.raises(ValueError):
        sz.encode_top16_paged(kv, batch, batch.new_payload_buffer(), batch.new_workspace(),
                              tables=tables_t, palette_info=batch.new_palette_info())
    info = batch.new_palette_info()
    assert sz.encode_top16_paged(kv, batch, batch.new_payload_buffer(), batch.new_workspace(),
                                 tables=tables_t, presence=batch.new_presence(),
                                 palette_info=info) == batch.total_encoded_bytes
    sub = sz.PagedBatch([tables[1]], 16384, "cuda")
    # record index 2 does not exist (2 records)
    assert sz.encode_bf16_paged(kv, sub, sub.new_palette_buffer(6), None, bits=6,
                                palette_info=info, info_first=[2]) is None
    torch.cuda.synchronize()
