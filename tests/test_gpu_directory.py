"""GPU decode with the escape directory (one kernel, escapes applied in registers)
against the oracle: directories written by the encoder and built on the host,
escape-dense chunks (the list path), shuffled escape lists, two launches, and
overflowed payloads next to good ones. The encoder's payloads must not change
when it also writes a directory."""

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


def u16(t) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def bf16(words: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(words).view(np.int16).copy()).to("cuda").view(
        torch.bfloat16)


def random_words(rng, n, books, rate):
    half = n // 2
    outside = np.array(sorted(set(range(256)) - set(books)), dtype=np.uint16)
    exps = np.empty(n, dtype=np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:], np.uint8)[rng.integers(0, 16, n - half)]
    esc = rng.random(n) < rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    low = rng.integers(0, 128, n).astype(np.uint16)
    sign = rng.integers(0, 2, n).astype(np.uint16) << 15
    return (sign | (exps << 7) | low).astype(np.uint16)


def _tables(rng, pool, requests):
    perm = rng.permutation(pool).tolist()
    out, at = [], 0
    for r in requests:
        out.append(perm[at:at + r])
        at += r
    return out


def _meaningful(directory: np.ndarray):
    """Fields a decoder reads: counts, first slots and inline entries of chunks
    with escapes, and every tile base."""
    total = directory.size // 68
    rec = directory[:64 * total].view(np.uint32).reshape(total, 4, 4).copy()
    count = rec[:, :, 0] >> 16
    rec[:, :, 0] = np.where(count > 0, rec[:, :, 0], 0)
    for i in range(3):
        rec[:, :, 1 + i] = np.where(count > i, rec[:, :, 1 + i], 0)
    return rec, directory[64 * total:].view(np.uint32)


@pytest.mark.parametrize("bw,pool,requests,rate,dense", [
    (16384, 64, [8, 16, 3], 0.0005, None),      # Llama-3-8B block
    (2048, 400, [3] * 70 + [5], 0.002, None),   # 71 payloads: two launches
    (2048, 64, [20, 6, 12], 0.0, [(1, 2048 + 100, 300), (12, 0, 9), (40, 1500, 5)]),
    (1024, 200, [30, 50, 7], 0.004, None),      # ~4 escapes per chunk: both paths
])
def test_directory_decode_matches_oracle(sz, codebooks, bw, pool, requests, rate, dense):
    say("directory", bw, pool, len(requests), rate, bool(dense))
    rng = np.random.default_rng(bw + pool)
    books = codebooks[11 * 32:12 * 32]
    tables = oracle.top16_tables(books)
    kv_host = random_words(rng, 2 * pool * bw, books, rate).reshape(2, pool, bw)
    if dense:
        outside = sorted(set(range(256)) - set(books))
        for blk, lo, count in dense:
            plane = 1 if lo >= bw else 0
            for w in range(lo % bw, lo % bw + count):
                kv_host[plane, blk, w] = (kv_host[plane, blk, w] & 0x807F) | (
                    outside[w % len(outside)] << 7)
    kv = bf16(kv_host.reshape(-1)).view(2, pool, bw)
    send_tables = _tables(rng, pool, requests)
    if dense:
        send_tables[0] = [5, 1] + [b for b in send_tables[0] if b not in (1, 5, 12, 40)][:18]
        send_tables[2] = [12, 40] + [b for b in send_tables[2] if b not in (1, 5, 12, 40)][:10]
    batch = sz.PagedBatch(send_tables, bw, "cuda")
    plain = batch.new_payload_buffer()
    out = batch.new_payload_buffer()
    directory = batch.new_directory()
    assert directory is not None
    ws = batch.new_workspace()
    assert sz.encode_top16_paged(kv, batch, plain, ws, codebooks=books) == batch.total_encoded_bytes
    assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books,
                                 directory=directory) == batch.total_encoded_bytes
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    for r in range(batch.payload_count):
        a, b = batch.out_offsets[r], batch.out_offsets[r] + batch.encoded_bytes[r]
        assert bytes(host[a:b]) == bytes(plain.cpu().numpy()[a:b]), f"payload {r}"
        ref = oracle.top16_encode(kv_host[:, send_tables[r]].reshape(-1), tables)
        assert bytes(host[a:b]) == bytes(ref), f"payload {r}"
    # the encoder's directory equals the host builder's on the same payloads
    built = sz.build_directory(host.copy(), batch.out_offsets, batch.encoded_bytes, batch)
    dev_rec, dev_base = _meaningful(directory.cpu().numpy())
    host_rec, host_base = _meaningful(built)
    assert np.array_equal(dev_base, host_base)
    assert np.array_equal(dev_rec, host_rec)
    if dense:
        assert (dev_rec[:, :, 0] >> 16).max() > 3
    # decode into an independent receiver table, with and without the directory
    recv = sz.PagedBatch(_tables(rng, pool, requests), bw, "cuda")
    for label, kwargs in (("device directory", {"directory": directory}),
                          ("host directory", {"directory": torch.from_numpy(built).cuda()}),
                          ("patch kernel", {})):
        target = torch.zeros_like(kv)
        got = sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, recv,
                                    codebooks=books, **kwargs)
        torch.cuda.synchronize()
        assert got == batch.total_raw_bytes, label
        back = u16(target).reshape(2, pool, bw)
        for src_t, dst_t in zip(send_tables, recv.block_tables):
            assert np.array_equal(back[:, dst_t], kv_host[:, src_t]), label


def test_directory_of_shuffled_lists_and_overflow(sz, codebooks):
    """Reference-order payloads (escapes shuffled, garbage padding) decoded through
    a host-built directory, next to an overflowed payload whose blocks stay
    untouched."""
    say("directory shuffled + overflow")
    from unchainkv_amd import codec_format

    rng = np.random.default_rng(77)
    bw, pool = 2048, 120
    books = codebooks[2 * 32:3 * 32]
    tables = oracle.top16_tables(books)
    requests = [16, 24, 8]
    send_tables = _tables(rng, pool, requests)
    batch = sz.PagedBatch(send_tables, bw, "cpu")
    buf = np.full(batch.out_bytes, 0x3C, dtype=np.uint8)
    sources = []
    for r, blocks in enumerate(requests):
        n = 2 * blocks * bw
        words = random_words(rng, n, books, 0.02 if r == 1 else 0.003)
        sources.append(words)
        payload = oracle.top16_encode(words, tables)
        o = batch.out_offsets[r]
        buf[o:o + payload.size] = payload
        if payload[0] == 5:
            lo, _ = codec_format.top16_sections(n)["escapes"]
            count = int.from_bytes(bytes(payload[1:5]), "little")
            entries = payload[lo:lo + 5 * count].reshape(count, 5)
            buf[o + lo:o + lo + 5 * count] = entries[rng.permutation(count)].reshape(-1)
            cap = codec_format.top16_escape_capacity(n)
            buf[o + lo + 5 * count:o + lo + 5 * cap] = rng.integers(0, 256, 5 * (cap - count))
    assert buf[batch.out_offsets[1]] == 255
    directory = sz.build_directory(buf, batch.out_offsets, batch.encoded_bytes, batch)
    recv = sz.PagedBatch(_tables(rng, pool, requests), bw, "cuda")
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    got = sz.decode_top16_paged(torch.from_numpy(buf).cuda(), batch.out_offsets,
                                batch.encoded_bytes, target, recv, codebooks=books,
                                directory=torch.from_numpy(directory).cuda())
    torch.cuda.synchronize()
    assert got == batch.total_raw_bytes
    back = u16(target).reshape(2, pool, bw)
    for r, dst_t in enumerate(recv.block_tables):
        if r == 1:
            assert not back[:, dst_t].any()
        else:
            assert np.array_equal(back[:, dst_t].reshape(-1), sources[r])


def test_directory_declines_without_the_tile_layout(sz, codebooks):
    """A directory needs the tile kernels: a KV layer 2 bytes off 16-byte alignment
    (generic kernels) or a directory one word short is declined. Payload sections
    at odd byte offsets do take the tile kernels, directory included."""
    say("directory declines")
    books = codebooks[:32]
    batch = sz.PagedBatch([[0, 1], [2]], 2048, "cuda")
    ws = batch.new_workspace()
    directory = batch.new_directory()
    aligned = batch.new_payload_buffer()
    backing = torch.zeros(2 * 4 * 2048 + 1, dtype=torch.bfloat16, device="cuda")
    kv_off = backing[1:].view(2, 4, 2048)
    assert sz.encode_top16_paged(kv_off, batch, aligned, ws, codebooks=books,
                                 directory=directory) is None
    assert sz.encode_top16_paged(kv_off, batch, aligned, ws, codebooks=books) == \
        batch.total_encoded_bytes
    assert sz.decode_top16_paged(aligned, batch.out_offsets, batch.encoded_bytes, kv_off, batch,
                                 codebooks=books, directory=directory) is None
    words = random_words(np.random.default_rng(8), 2 * 4 * 2048, books, 0.003)
    kv = bf16(words).view(2, 4, 16, 1, 128)
    short = torch.zeros(batch.directory_bytes() - 4, dtype=torch.uint8, device="cuda")
    assert sz.encode_top16_paged(kv, batch, aligned, ws, codebooks=books, directory=short) is None
    out = torch.zeros(batch.out_bytes + 16, dtype=torch.uint8, device="cuda")[3:]
    assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books, directory=directory) == \
        batch.total_encoded_bytes
    target = torch.full_like(kv, 1.0)
    assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, batch,
                                 codebooks=books, directory=directory) == batch.total_raw_bytes
    torch.cuda.synchronize()
    assert torch.equal(target[:, :3].view(torch.int16), kv[:, :3].view(torch.int16))
    assert bool((target[:, 3] == 1.0).all())


def test_unsuitable_workspaces_are_declined(sz, codebooks):
    """A workspace that is not a contiguous uint8 buffer on the layer's device is
    declined by the encoders; the attention and histogram wrappers allocate their
    own in its place."""
    say("unsuitable workspaces")
    books = codebooks[:32]
    batch = sz.PagedBatch([[0, 1], [2]], 2048, "cuda")
    # no escapes: at most 64 distinct high bytes, so fixed6 takes the words too
    words = random_words(np.random.default_rng(9), 2 * 4 * 2048, books, 0.0)
    kv = bf16(words).view(2, 4, 2048)
    out = batch.new_payload_buffer()
    ws = batch.new_workspace()
    for bad in (ws.view(torch.int32), ws[::2], ws.cpu()):
        assert sz.encode_top16_paged(kv, batch, out, bad, codebooks=books) is None
    six = batch.new_palette_buffer(6)
    pws = batch.new_palette_workspace()
    assert sz.encode_bf16_paged(kv, batch, six, pws.cpu(), bits=6) is None
    assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books) == batch.total_encoded_bytes
    assert sz.encode_bf16_paged(kv, batch, six, pws, bits=6) is not None
    counts = sz.exponent_histogram_paged(kv, batch, workspace=torch.zeros(8, dtype=torch.int32,
                                                                          device="cuda"))
    torch.cuda.synchronize()
    assert counts is not None and int(counts.sum()) == 2 * 3 * 2048
