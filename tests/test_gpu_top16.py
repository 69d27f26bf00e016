"""GPU parity of the HIP Top-16 codec against the CPU oracle.

Encode output must be byte-identical to the oracle's canonical payload
(escapes ascending, unused slots zeroed); decode + scatter must reproduce the
source bf16 words exactly, for payloads from the oracle (canonical) and for
payloads with shuffled escapes and garbage padding (the byte streams the
reference's atomic-ordered encoder produces).
"""

import ctypes
import random

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sz():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda

    assert splitzip_cuda.available(), splitzip_cuda.load_error()
    return splitzip_cuda


def u16(t) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def bf16(words: np.ndarray, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(words).view(np.int16).copy()).to(device).view(
        torch.bfloat16)


def random_words(rng, n, books, escape_rate):
    half = n // 2
    k_book = np.frombuffer(books[:16], dtype=np.uint8)
    v_book = np.frombuffer(books[16:], dtype=np.uint8)
    outside = np.array(sorted(set(range(256)) - set(books)), dtype=np.uint16)
    exps = np.empty(n, dtype=np.uint16)
    exps[:half] = k_book[rng.integers(0, 16, half)]
    exps[half:] = v_book[rng.integers(0, 16, n - half)]
    esc = rng.random(n) < escape_rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    low = rng.integers(0, 128, n).astype(np.uint16)
    sign = rng.integers(0, 2, n).astype(np.uint16) << 15
    return (sign | (exps << 7) | low).astype(np.uint16)


def say(*parts):
    print("[case]", *parts, flush=True)


# ---------------------------------------------------------------------------
# known answers

def test_kat256_encode_and_decode(sz, golden_dir, codebooks):
    import json

    kat = json.loads((golden_dir / "kat_top16_256.json").read_text())
    payload = bytes.fromhex(kat["payload_hex"])
    words = np.frombuffer(bytes.fromhex(kat["raw_hex"]), "<u2").copy()
    say("kat256 encode")
    source = bf16(words)
    out = torch.empty(512, dtype=torch.uint8, device="cuda")
    size = sz.encode_top16(source, out, 0)
    torch.cuda.synchronize()
    assert size == len(payload)
    assert bytes(out[:size].cpu().numpy()) == payload
    say("kat256 decode")
    comp = torch.tensor(list(payload), dtype=torch.uint8, device="cuda")
    target = torch.zeros((2, 16, 8), dtype=torch.bfloat16, device="cuda")
    copied = sz.decode_top16(comp, target, list(range(16)), 512, 0)
    torch.cuda.synchronize()
    assert copied == 512
    assert np.array_equal(u16(target), words)


@pytest.mark.parametrize("block_count,target_blocks,block_ids", [
    (1, 4, [3]), (128, 256, list(range(0, 256, 2)))])
def test_reference_roundtrip_inputs(sz, codebooks, block_count, target_blocks, block_ids):
    """tests/test_splitzip_cuda.py:137-185 of the reference, plus byte parity."""
    say("reference roundtrip", block_count)
    count = 2 * block_count * 2048
    index = torch.arange(count, dtype=torch.int32, device="cuda")
    books = torch.tensor(list(codebooks[:32]), device="cuda").reshape(2, 16)
    plane = torch.div(index, count // 2, rounding_mode="floor")
    exponent = books[plane.long(), torch.remainder(index, 16).long()]
    exponent[::400] = 100
    words = torch.bitwise_or(
        torch.bitwise_left_shift(torch.remainder(index, 2), 15),
        torch.bitwise_or(torch.bitwise_left_shift(exponent.to(torch.int32), 7),
                         torch.remainder(index, 128))).to(torch.int16)
    source = words.view(torch.bfloat16).reshape(2, block_count, 2048)
    raw_bytes = source.numel() * source.element_size()
    encoded = torch.empty(raw_bytes, dtype=torch.uint8, device="cuda")
    size = sz.encode_top16(source, encoded, 0)
    target = torch.zeros((2, target_blocks, 2048), dtype=torch.bfloat16, device="cuda")
    copied = sz.decode_top16(encoded[:size], target, block_ids, raw_bytes, 0)
    torch.cuda.synchronize()
    assert raw_bytes / size >= 1.30
    assert int(encoded[0].item()) == 5
    assert copied == raw_bytes
    assert torch.equal(target[:, block_ids].view(torch.int16), source.view(torch.int16))
    ref = oracle.top16_encode(u16(source), oracle.top16_tables(codebooks[:32]))
    assert bytes(encoded[:size].cpu().numpy()) == bytes(ref)


# ---------------------------------------------------------------------------
# drop-in entry points: sizes, misalignment, capacity modes

@pytest.mark.parametrize("n", [22, 23, 255, 256, 1000, 4096, 8192, 8202, 65536, 200_000])
@pytest.mark.parametrize("shift", [0, 3, 11])
@pytest.mark.parametrize("roomy", [True, False])
def test_dropin_encode_matches_oracle(sz, codebooks, n, shift, roomy):
    say("dropin encode", n, shift, roomy)
    rng = np.random.default_rng(n + 17 * shift)
    books = codebooks[7 * 32:8 * 32]
    words = random_words(rng, n, books, 0.003)
    ref = oracle.top16_encode(words, oracle.top16_tables(books))
    size = codec_format.top16_encoded_size(n)
    capacity = 2 * n if roomy else ((size + 3) & ~3) + 8
    if ref is None or capacity < ((size + 3) & ~3) + 8:
        pytest.skip("the reference declines this size")
    backing = torch.full((capacity + shift + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    out = backing[shift:shift + capacity]
    source = bf16(words)
    got = sz.encode_top16(source, out, 7)
    torch.cuda.synchronize()
    assert got == size
    assert bytes(out[:size].cpu().numpy()) == bytes(ref)
    # nothing before the payload was touched
    assert bytes(backing[:shift].cpu().numpy()) == b"\xa5" * shift


def test_dropin_encode_more_tiles_than_one_finalize_pass(sz, codebooks):
    """A payload of 4100 tiles: the finalize scans the tile counts in two passes
    (4096 tiles per pass when a payload has 16 finalize workgroups), and the
    escape slots carry over from one pass to the next."""
    n = 4100 * 4096
    say("dropin encode, two finalize passes", n)
    rng = np.random.default_rng(41)
    books = codebooks[3 * 32:4 * 32]
    words = random_words(rng, n, books, 0.004)
    ref = oracle.top16_encode(words, oracle.top16_tables(books))
    size = codec_format.top16_encoded_size(n)
    out = torch.empty((size + 64,), dtype=torch.uint8, device="cuda")
    got = sz.encode_top16(bf16(words), out, 3)
    torch.cuda.synchronize()
    assert got == size
    assert bytes(out[:size].cpu().numpy()) == bytes(ref)


@pytest.mark.parametrize("label,n,src_shift,out_shift", [
    ("llama3-8b 64 blocks", 2 * 64 * 16384, 0, 0),
    ("70b 5 blocks, short last tiles", 2 * 5 * 2048, 0, 3),
    ("unaligned source: generic kernels", 2 * 9 * 2048, 1, 0),
])
@pytest.mark.parametrize("rate", [0.001, 0.006])
def test_dropin_encode_at_minimum_capacity_is_parallel(sz, codebooks, label, n, src_shift,
                                                       out_shift, rate):
    """Capacity align4(E) + 8, the reference ABI's minimum: the tiles stage their
    escapes in their own body bytes (escape-dense tiles re-scanned, and at 0.6 %
    the payload overflows), byte-identical to the oracle; bytes past the scratch
    tail untouched."""
    say("dropin min capacity", label, rate)
    rng = np.random.default_rng(n + src_shift + int(rate * 1e4))
    books = codebooks[6 * 32:7 * 32]
    words = random_words(rng, n + src_shift, books, rate)
    if rate < 0.005:
        # three dense tiles: 300 escapes in one (re-scanned), 100 in another
        outside = sorted(set(range(256)) - set(books))
        for lo, count in ((4096 + 10, 300), (n // 2 + 50, 100), (n - 70, 60)):
            for i in range(lo, lo + count):
                words[src_shift + i] = (words[src_shift + i] & 0x807F) | (
                    outside[i % len(outside)] << 7)
    ref = oracle.top16_encode(words[src_shift:], oracle.top16_tables(books))
    size = codec_format.top16_encoded_size(n)
    capacity = ((size + 3) & ~3) + 8
    backing = torch.full((capacity + out_shift + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    out = backing[out_shift:out_shift + capacity]
    source = bf16(words)[src_shift:]
    got = sz.encode_top16(source, out, 6)
    torch.cuda.synchronize()
    assert got == size
    assert bytes(out[:size].cpu().numpy()) == bytes(ref)
    assert bytes(backing[out_shift + capacity:].cpu().numpy()) == b"\xa5" * 64


def test_dropin_encode_unaligned_source(sz, codebooks):
    say("dropin encode unaligned source")
    rng = np.random.default_rng(5)
    n = 9000
    books = codebooks[:32]
    words = random_words(rng, n + 1, books, 0.002)
    backing = bf16(words)
    source = backing[1:]  # 2-byte offset: not 16-byte aligned
    out = torch.empty(2 * n, dtype=torch.uint8, device="cuda")
    got = sz.encode_top16(source, out, 0)
    torch.cuda.synchronize()
    ref = oracle.top16_encode(words[1:], oracle.top16_tables(books))
    assert bytes(out[:got].cpu().numpy()) == bytes(ref)


@pytest.mark.parametrize("rate", [0.0, 0.004, 0.02])
@pytest.mark.parametrize("bw,blocks,pool", [(2048, 8, 40), (16384, 3, 12), (48, 50, 120), (40, 30, 90)])
def test_dropin_decode_scatter_matches_oracle(sz, codebooks, rate, bw, blocks, pool):
    say("dropin decode", rate, bw, blocks)
    rng = np.random.default_rng(bw + blocks)
    books = codebooks[11 * 32:12 * 32]
    n = 2 * blocks * bw
    words = random_words(rng, n, books, rate)
    tables = oracle.top16_tables(books)
    payload = oracle.top16_encode(words, tables)
    ids = sorted(rng.choice(pool, blocks, replace=False).tolist(), key=lambda _: rng.random())
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    marker = torch.full_like(target, 1.5)
    target.copy_(marker)
    comp = torch.from_numpy(payload.copy()).cuda()
    copied = sz.decode_top16(comp, target, ids, 2 * n, -1, codebooks=books)
    torch.cuda.synchronize()
    assert copied == 2 * n
    expected = np.full((2, pool, bw), u16(marker)[0], np.uint16)
    if payload[0] == 5:
        oracle.scatter(oracle.top16_decode(payload, n, tables), expected.reshape(-1), blocks, bw,
                       pool * bw, bw, ids=ids)
    assert np.array_equal(u16(target), expected.reshape(-1))


@pytest.mark.parametrize("blocks", [256, 257])
def test_dropin_decode_host_table_limit(sz, codebooks, blocks):
    """A shuffled table of 256 ids rides in the kernel arguments; 257 ids go through
    the device copy of the table. Both restore every block exactly."""
    say("dropin decode host table", blocks)
    rng = np.random.default_rng(blocks)
    books = codebooks[2 * 32:3 * 32]
    bw, pool = 1024, 700
    n = 2 * blocks * bw
    words = random_words(rng, n, books, 0.004)
    payload = oracle.top16_encode(words, oracle.top16_tables(books))
    ids = rng.permutation(pool)[:blocks].tolist()
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    comp = torch.from_numpy(payload.copy()).cuda()
    assert sz.decode_top16(comp, target, ids, 2 * n, -1, codebooks=books) == 2 * n
    got = u16(target).reshape(2, pool, bw)
    assert np.array_equal(got[:, ids].reshape(-1), words)
    rest = np.setdiff1d(np.arange(pool), ids)
    assert not got[:, rest].any()


def test_decode_accepts_shuffled_escapes_and_garbage_padding(sz, codebooks):
    say("decode shuffled escapes")
    rng = np.random.default_rng(21)
    bw, blocks, pool = 1024, 16, 40
    n = 2 * blocks * bw
    books = codebooks[2 * 32:3 * 32]
    tables = oracle.top16_tables(books)
    words = random_words(rng, n, books, 0.004)
    payload = bytearray(oracle.top16_encode(words, tables))
    count = int.from_bytes(payload[1:5], "little")
    lo, hi = codec_format.top16_sections(n)["escapes"]
    slots = [bytes(payload[lo + 5 * s: lo + 5 * s + 5]) for s in range(count)]
    random.Random(3).shuffle(slots)
    payload[lo:lo + 5 * count] = b"".join(slots)
    payload[lo + 5 * count:hi] = bytes(rng.integers(0, 256, hi - lo - 5 * count, dtype=np.uint8))
    ids = rng.permutation(pool)[:blocks].tolist()
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    comp = torch.tensor(list(payload), dtype=torch.uint8, device="cuda")
    assert sz.decode_top16(comp, target, ids, 2 * n, -1, codebooks=books) == 2 * n
    torch.cuda.synchronize()
    got = u16(target).reshape(2, pool, bw)[:, ids].reshape(-1)
    assert np.array_equal(got, words)


def test_decode_of_reference_cpu_decoder_fixtures(sz):
    """Payloads with shuffled escape lists and random unused slots, decoded by the
    reference's CPU decoder into the fixture words (tests/golden/
    make_top16_cpu_golden.py): the GPU decode + scatter writes the same words, at
    tile geometry (1024-word blocks) and at block sizes the tile kernels do not
    take. Repeated positions are left out: the GPU patches escapes in parallel, and
    the reference's CUDA decode has no order among them either."""
    import json
    from pathlib import Path

    golden = Path(__file__).resolve().parent / "golden"
    index = json.loads((golden / "top16_cpu_cases.json").read_text())
    blocks_for = {256: 2, 1000: 4, 4096: 2, 16384: 8, 10004: 82}
    rng = np.random.default_rng(5)
    done = 0
    with np.load(golden / "top16_cpu_payloads.npz") as data:
        for case in index["cases"]:
            if not (case["decoded"] and case["distinct"]):
                continue
            key, n = case["key"], case["raw_bytes"] // 2
            blocks = blocks_for[n]
            bw = n // (2 * blocks)
            say("reference cpu decoder fixture", case["name"], "blocks", blocks, "bw", bw)
            pool = blocks + 5
            ids = rng.permutation(pool)[:blocks].tolist()
            target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
            comp = torch.from_numpy(data[key + "_payload"].copy()).cuda()
            books = data[key + "_books"].tobytes()
            assert sz.decode_top16(comp, target, ids, 2 * n, -1, codebooks=books) == 2 * n
            torch.cuda.synchronize()
            got = u16(target).reshape(2, pool, bw)[:, ids].reshape(-1)
            assert np.array_equal(got, data[key + "_words"]), case["name"]
            done += 1
    assert done == 15


def test_decode_leaves_overflowed_payload_unapplied(sz, codebooks):
    say("decode mode 255")
    n = 2 * 4 * 512
    payload = torch.zeros(codec_format.top16_encoded_size(n), dtype=torch.uint8, device="cuda")
    payload[0] = 255
    target = torch.full((2, 8, 512), 2.0, dtype=torch.bfloat16, device="cuda")
    assert sz.decode_top16(payload, target, [1, 5, 2, 7], 2 * n, 0) == 2 * n
    torch.cuda.synchronize()
    assert torch.all(target == 2.0)


# ---------------------------------------------------------------------------
# escape-heavy tiles (finalize re-scan path) and overflow

def test_tile_with_many_escapes_and_overflow(sz, codebooks):
    books = codebooks[4 * 32:5 * 32]
    tables = oracle.top16_tables(books)
    rng = np.random.default_rng(8)
    n = 2 * 8 * 4096  # 16 tiles, cap 328
    words = random_words(rng, n, books, 0.0)
    outside = sorted(set(range(256)) - set(books))
    # 200 escapes packed into tile 3 (more than the 128 staged per tile), 50 elsewhere
    for pos in list(range(3 * 4096 + 100, 3 * 4096 + 300)) + rng.choice(n, 50, replace=False).tolist():
        words[pos] = (words[pos] & 0x807F) | (outside[pos % len(outside)] << 7)
    for label, w in (("dense tile", words), ("overflow", random_words(rng, n, books, 0.01))):
        say("escape-heavy", label)
        ref = oracle.top16_encode(w, tables)
        out = torch.empty(2 * n, dtype=torch.uint8, device="cuda")
        size = sz.encode_top16(bf16(w), out, -1, codebooks=books)
        torch.cuda.synchronize()
        assert bytes(out[:size].cpu().numpy()) == bytes(ref)
    assert ref[0] == 255


# ---------------------------------------------------------------------------
# batched paged entry points

@pytest.mark.parametrize("bw,pool,requests,rate,offset", [
    (16384, 64, [8, 16, 3], 0.0005, 0),     # Llama-3-8B block (8 heads x 128 x 16)
    (2048, 300, [8, 40, 17, 64], 0.001, 0),  # 70B TP8 share (1 head)
    (8192, 80, [64], 0.002, 0),             # Llama-3.2-1B block
    (48, 400, [50, 7, 99], 0.003, 0),       # small block, several blocks per tile
    (40, 300, [60, 5], 0.003, 0),           # block words not a multiple of 16: generic path
    (2048, 100, [10, 20], 0.001, 1),        # KV view at a 2-byte offset: generic path
    (2048, 400, [3] * 70 + [5], 0.002, 0),  # 71 payloads: two launches of 64 and 7
    (48, 600, [8] * 66, 0.001, 0),          # 66 payloads on the generic kernels
])
def test_paged_encode_decode_matches_oracle(sz, codebooks, bw, pool, requests, rate, offset):
    say("paged", bw, pool, requests, rate, offset)
    rng = np.random.default_rng(bw * 3 + pool)
    books = codebooks[9 * 32:10 * 32]
    tables = oracle.top16_tables(books)
    words = random_words(rng, 2 * pool * bw + offset, books, rate)
    backing = bf16(words)
    kv = backing[offset:].view(2, pool, bw)
    kv_host = words[offset:].reshape(2, pool, bw)
    perm = rng.permutation(pool).tolist()
    block_tables, at = [], 0
    for r in requests:
        block_tables.append(perm[at:at + r])
        at += r
    batch = sz.PagedBatch(block_tables, bw, "cuda")
    out = batch.new_payload_buffer()
    out.fill_(0x5A)
    ws = batch.new_workspace()
    # with offset=1 the layer starts 2 bytes past a 16-byte boundary and the
    # library takes its generic (any alignment) kernels
    total = sz.encode_top16_paged(kv, batch, out, ws, codebooks=books)
    torch.cuda.synchronize()
    assert total == batch.total_encoded_bytes
    host = out.cpu().numpy()
    for r, t in enumerate(block_tables):
        ref = oracle.top16_encode(kv_host[:, t].reshape(-1), tables)
        got = host[batch.out_offsets[r]:batch.out_offsets[r] + batch.encoded_bytes[r]]
        assert bytes(got) == bytes(ref), f"payload {r}"
    # receiver with an independent block table
    rperm = rng.permutation(pool).tolist()
    recv_tables, at = [], 0
    for r in requests:
        recv_tables.append(rperm[at:at + r])
        at += r
    recv_batch = sz.PagedBatch(recv_tables, bw, "cuda")
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    copied = sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target,
                                   recv_batch, codebooks=books)
    torch.cuda.synchronize()
    assert copied == batch.total_raw_bytes
    got = u16(target).reshape(2, pool, bw)
    for src_t, dst_t in zip(block_tables, recv_tables):
        assert np.array_equal(got[:, dst_t], kv_host[:, src_t])
    used = {b for t in recv_tables for b in t}
    free = [b for b in range(pool) if b not in used]
    assert not got[:, free].any()


@pytest.mark.parametrize("shift", [1, 6, 11])
def test_paged_payloads_at_unaligned_offsets(sz, codebooks, shift):
    """Payloads packed back to back at offsets of odd residues (bodies and code
    sections at any byte address) take the tile kernels: encode with the escape
    directory, byte-identical to the oracle, the gaps between payloads untouched;
    then the one-kernel decode through that directory restores every block."""
    say("paged unaligned offsets", shift)
    bw, pool = 2048, 96
    books = codebooks[5 * 32:6 * 32]
    tables = oracle.top16_tables(books)
    rng = np.random.default_rng(70 + shift)
    words = random_words(rng, 2 * pool * bw, books, 0.003)
    kv_host = words.reshape(2, pool, bw)
    kv = bf16(words).view(2, pool, bw)
    perm = rng.permutation(pool).tolist()
    block_tables = [perm[0:9], perm[9:10], perm[10:40], perm[40:43]]
    batch = sz.PagedBatch(block_tables, bw, "cuda")
    offsets, at = [], 0
    for e in batch.encoded_bytes:
        at += shift
        offsets.append(at)
        at += e
    assert any((o + 5) % 16 for o in offsets)
    batch.out_offsets = offsets  # the batch's own offsets would be aligned
    batch._out_offsets = (ctypes.c_ulonglong * len(offsets))(*offsets)
    out = torch.full((at + 64,), 0xA5, dtype=torch.uint8, device="cuda")
    directory = batch.new_directory()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), codebooks=books,
                                 directory=directory) == batch.total_encoded_bytes
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    prev = 0
    for r, t in enumerate(block_tables):
        o, e = offsets[r], batch.encoded_bytes[r]
        assert bytes(host[o:o + e]) == bytes(oracle.top16_encode(kv_host[:, t].reshape(-1),
                                                                 tables)), f"payload {r}"
        assert not (host[prev:o] != 0xA5).any(), f"gap before payload {r}"
        prev = o + e
    assert not (host[prev:] != 0xA5).any()
    recv_tables = [[(b + 7) % pool for b in t] for t in block_tables]
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    target = torch.zeros_like(kv)
    assert sz.decode_top16_paged(out, offsets, batch.encoded_bytes, target, recv,
                                 codebooks=books, directory=directory) == batch.total_raw_bytes
    got = u16(target).reshape(2, pool, bw)
    for src_t, dst_t in zip(block_tables, recv_tables):
        assert np.array_equal(got[:, dst_t], kv_host[:, src_t])


@pytest.mark.parametrize("label", ["dense tile", "overflow"])
def test_paged_escape_heavy_tiles(sz, codebooks, label):
    """Tiles with more escapes than the tile kernel stages (re-scan in the finalize
    kernel), and a payload whose escapes overflow the capacity (header 255)."""
    say("paged escape-heavy", label)
    bw, pool = 2048, 64
    books = codebooks[3 * 32:4 * 32]
    tables = oracle.top16_tables(books)
    rng = np.random.default_rng(31)
    words = random_words(rng, 2 * pool * bw, books, 0.0 if label == "dense tile" else 0.01)
    kv_host = words.reshape(2, pool, bw)
    block_tables = [[5, 9, 1, 30, 50, 51, 52, 53, 54, 55, 56, 57, 58, 59, 60, 61, 62, 3, 4, 6],
                    [44, 2], [7, 8, 63, 12, 40, 41, 42, 43]]
    if label == "dense tile":
        outside = sorted(set(range(256)) - set(books))
        # 300 escapes inside one tile of payload 0's V plane (cap 410: re-scanned)
        # and 100 in one tile of payload 2's K plane (cap 164: all staged)
        for blk, lo, count in ((1, 2048 + 100, 300), (12, 0, 100)):
            for w in range(lo % bw, lo % bw + count):
                plane = 1 if blk == 1 else 0
                kv_host[plane, blk, w] = (kv_host[plane, blk, w] & 0x807F) | (
                    outside[w % len(outside)] << 7)
    kv = bf16(kv_host.reshape(-1)).view(2, pool, bw)
    batch = sz.PagedBatch(block_tables, bw, "cuda")
    out = batch.new_payload_buffer()
    out.fill_(0x77)
    ws = batch.new_workspace()
    assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books) == batch.total_encoded_bytes
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    for r, t in enumerate(block_tables):
        ref = oracle.top16_encode(kv_host[:, t].reshape(-1), tables)
        got = host[batch.out_offsets[r]:batch.out_offsets[r] + batch.encoded_bytes[r]]
        assert bytes(got) == bytes(ref), f"payload {r}"
        if label == "overflow":
            assert got[0] == 255
    # decode: 300 escapes in one tile are all patched; overflowed payloads stay
    # untouched (the reference decoder skips a payload whose byte 0 is not 5)
    target = torch.zeros_like(kv)
    sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, batch,
                          codebooks=books)
    got = u16(target).reshape(2, pool, bw)
    for r, t in enumerate(block_tables):
        if label == "overflow":
            assert not got[:, t].any(), r
        else:
            assert np.array_equal(got[:, t], kv_host[:, t]), r


def test_paged_full_size_llama3_8b_layer(sz):
    """One full layer of the Llama-3-8B paged encode workload (8 requests x 4096
    tokens from a 4096-block pool): byte parity of every payload with the oracle
    and an exact round trip into an independent receiver table."""
    from unchainkv_amd import workloads

    shape = workloads.LLAMA3_8B
    say("full-size llama3-8b layer")
    kv = workloads.make_kv_layer(torch, shape, 4096, seed=1, layer=5, device="cuda")
    tables = workloads.random_block_tables(torch, 4096, [256] * 8, seed=1)
    books = workloads.fit_codebook(torch, kv, tables)
    batch = sz.PagedBatch(tables, shape.block_words, "cuda")
    out = batch.new_payload_buffer()
    ws = batch.new_workspace()
    assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books) == batch.total_encoded_bytes
    recv_tables = workloads.random_block_tables(torch, 4096, [256] * 8, seed=2)
    recv_batch = sz.PagedBatch(recv_tables, shape.block_words, "cuda")
    target = torch.zeros_like(kv)
    assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, recv_batch,
                                 codebooks=books) == batch.total_raw_bytes
    torch.cuda.synchronize()
    src_ids = torch.tensor([b for t in tables for b in t], device="cuda")
    dst_ids = torch.tensor([b for t in recv_tables for b in t], device="cuda")
    assert torch.equal(kv.view(torch.int16)[:, src_ids], target.view(torch.int16)[:, dst_ids])
    host = out.cpu().numpy()
    kv_host = u16(kv).reshape(2, 4096, -1)
    ref = oracle.encode_paged_batch(kv_host, 4096 * shape.block_words, shape.block_words,
                                    shape.block_words, tables, batch.out_offsets, batch.out_bytes,
                                    oracle.top16_tables(books), threads=oracle.default_threads())
    for r in range(8):
        a, b = batch.out_offsets[r], batch.out_offsets[r] + batch.encoded_bytes[r]
        assert host[a] == 5
        assert bytes(host[a:b]) == bytes(ref[a:b]), f"payload {r}"
