"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against what the reference itself fixes:
golden vectors rebuilt from the reference's tests, closed forms, inverse
properties, brute force on tiny inputs and an independent pure-Python
restatement. The mutant tests plant plausible mistakes in a copy of the
restated decoder and show that the golden vectors catch them.
"""

import hashlib
import json
import random

import numpy as np
import pytest

import oracle
from unchainkv_amd import codec_format

SHA_ALL = "00ed4ba48c4c9f85f3e0a960e1be8edaf5d9bf7e16a9d454b85eb361d1144342"
SHA_EXT = "71658a97e33340a808bfbe010d7c570386ef319111d2b22e3e64678da712e0ef"


def _kat(golden_dir):
    data = json.loads((golden_dir / "kat_top16_256.json").read_text())
    payload = bytes.fromhex(data["payload_hex"])
    raw = bytes.fromhex(data["raw_hex"])
    words = np.frombuffer(raw, dtype="<u2").copy()
    return data, payload, raw, words


def _random_words(rng, n, books, escape_rate):
    """bf16 words whose exponents come from the layer codebooks, with a fraction
    replaced by exponents outside them."""
    half = n // 2
    k_book = np.frombuffer(books[:16], dtype=np.uint8)
    v_book = np.frombuffer(books[16:], dtype=np.uint8)
    outside = np.array(sorted(set(range(256)) - set(books[:16]) - set(books[16:])), dtype=np.uint16)
    exps = np.empty(n, dtype=np.uint16)
    exps[:half] = k_book[rng.integers(0, 16, half)]
    exps[half:] = v_book[rng.integers(0, 16, n - half)]
    esc = rng.random(n) < escape_rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    low = rng.integers(0, 128, n).astype(np.uint16)
    sign = rng.integers(0, 2, n).astype(np.uint16) << 15
    return (sign | (exps << 7) | low).astype(np.uint16)


# ---------------------------------------------------------------------------
# a1: codebook bytes

def test_codebook_fixture_matches_reference_literal(codebooks):
    assert len(codebooks) == 1024
    assert hashlib.sha256(codebooks).hexdigest() == SHA_ALL
    assert hashlib.sha256(codebooks[896:]).hexdigest() == SHA_EXT


def test_embedded_codebooks_have_no_duplicates_and_ship_with_the_package(codebooks):
    from unchainkv_amd import splitzip_cuda

    assert splitzip_cuda._TOP16_CODEBOOKS == codebooks
    for layer in range(32):
        for plane in range(2):
            book = codebooks[layer * 32 + plane * 16: layer * 32 + plane * 16 + 16]
            assert len(set(book)) == 16
    # layers 28-31 carry exponent 0 (zero/denormal words), per the extension block
    assert all(0 in codebooks[l * 32:(l + 1) * 32] for l in range(28, 32))


# ---------------------------------------------------------------------------
# a2: lookup table

def test_tables_closed_form_all_layers(codebooks):
    for layer in range(32):
        books = codebooks[layer * 32:(layer + 1) * 32]
        c_table = bytes(oracle.top16_tables(books))
        py_table = oracle.top16_tables_py(books)
        assert c_table == py_table == codec_format.top16_tables(books)
        assert len(c_table) == 544
        for plane in range(2):
            for code in range(16):
                assert c_table[plane * 256 + books[plane * 16 + code]] == code
            hits = sum(1 for e in range(256) if c_table[plane * 256 + e] != 255)
            assert hits == 16
        assert c_table[512:] == books


def test_tables_later_code_wins_for_repeated_exponent():
    books = bytes([7] * 16 + list(range(100, 116)))
    table = bytes(oracle.top16_tables(books))
    assert table[7] == 15  # code 15 written last
    assert table == oracle.top16_tables_py(books) == codec_format.top16_tables(books)


# ---------------------------------------------------------------------------
# a4/a6: sizes and header

def test_size_known_answer(golden_dir):
    kat = json.loads((golden_dir / "kat_sizes.json").read_text())
    n = 2 * kat["tokens"] * kat["kv_heads"] * kat["head_dim"]
    assert 2 * n == kat["raw_bytes"] == 65_536_000
    assert oracle.top16_encoded_size(n) == kat["top16_bytes"] == 49_971_205
    assert oracle.load().sz_top16_encoded_size(n) == kat["top16_bytes"]
    assert codec_format.top16_encoded_size(n) == kat["top16_bytes"]


@pytest.mark.parametrize("n", [22, 23, 200, 201, 256, 1_048_576, 8_388_608, 16_777_216])
def test_size_closed_forms(n):
    lib = oracle.load()
    cap = -(-n // 200)
    assert lib.sz_top16_escape_capacity(n) == cap == codec_format.top16_escape_capacity(n)
    assert lib.sz_top16_encoded_size(n) == 5 + n + -(-n // 2) + 5 * cap
    assert lib.sz_fixed6_encoded_size(n) == 65 + n + 3 * -(-n // 4) == codec_format.fixed6_encoded_size(n)


def test_compression_ratio_limits():
    assert codec_format.top16_ratio(8_388_608) == pytest.approx(1.31147, abs=1e-5)
    assert codec_format.top16_encoded_size(8_388_608) == 12_792_637
    assert codec_format.top16_encoded_size(1_048_576) == 1_599_084
    assert codec_format.top16_encoded_size(16_777_216) == 25_585_264
    assert 2 * 8_388_608 / codec_format.fixed6_encoded_size(8_388_608) == pytest.approx(1.14285, abs=1e-5)


def test_encoder_declines_where_reference_does():
    tables = oracle.top16_tables(bytes(range(32)))
    # E(n) >= 2n for n < 22: the reference returns 0 (kvq_splitzip_cuda.cu:393)
    assert oracle.top16_encode(np.zeros(21, np.uint16), tables) is None
    assert oracle.top16_encode(np.zeros(22, np.uint16), tables) is not None
    assert oracle.encode_top16_py([0] * 21, bytes(tables)) is None


# ---------------------------------------------------------------------------
# a5/a10/a11/a12: the 256-word known answer (tests/test_vllm_connector.py:333-372)

def test_kat256_encode_is_byte_exact(golden_dir, codebooks):
    data, payload, raw, words = _kat(golden_dir)
    tables = oracle.top16_tables(codebooks[:32])
    assert bytes(oracle.top16_encode(words, tables)) == payload
    assert oracle.encode_top16_py(list(map(int, words)), bytes(tables)) == payload


def test_kat256_decode_is_byte_exact(golden_dir, codebooks):
    data, payload, raw, words = _kat(golden_dir)
    tables = oracle.top16_tables(codebooks[:32])
    decoded = oracle.top16_decode(np.frombuffer(payload, np.uint8), data["count_words"], tables)
    assert decoded.tobytes() == raw
    assert oracle.decode_top16_payload_py(payload, data["raw_bytes"], codebooks[:32]) == raw


def test_kat256_shape(golden_dir):
    data, payload, raw, words = _kat(golden_dir)
    assert payload[0] == 5 and int.from_bytes(payload[1:5], "little") == 1
    assert len(payload) == codec_format.top16_encoded_size(256) == 399
    # the one escape: position 3, exponent 100
    assert codec_format.top16_escapes(payload, 256) == [(3, 100)]


def _mutant_decoder(kind):
    def decode(data, raw_bytes, codebooks):
        view = memoryview(data)
        count = raw_bytes // 2
        code_bytes = (count + 1) // 2
        raw = bytearray(raw_bytes)
        half = count // 2 + (1 if kind == "plane_split" else 0)
        for i in range(count):
            shift = ((i + 1) % 2) * 4 if kind == "nibble_order" else (i % 2) * 4
            code = (view[5 + count + i // 2] >> shift) & 0x0F
            exponent = codebooks[(i >= half) * 16 + code]
            value = view[5 + i]
            sign = 0 if kind == "sign" else (value & 0x80) << 8
            word = (value & 0x7F) | sign | (exponent << 7)
            raw[2 * i:2 * i + 2] = word.to_bytes(2, "little")
        at = 5 + count + code_bytes
        esc = int.from_bytes(view[1:5], "little")
        for slot in range(esc):
            e = at + 5 * slot
            order = "big" if kind == "position_endian" else "little"
            pos = int.from_bytes(view[e:e + 4], order)
            if pos >= count:
                continue
            word = int.from_bytes(raw[2 * pos:2 * pos + 2], "little")
            word = (word & 0x807F) | (view[e + 4] << 7)
            raw[2 * pos:2 * pos + 2] = word.to_bytes(2, "little")
        return bytes(raw)

    return decode


@pytest.mark.parametrize("kind", ["nibble_order", "sign", "plane_split", "position_endian"])
def test_kat256_catches_planted_mistakes(golden_dir, codebooks, kind):
    data, payload, raw, words = _kat(golden_dir)
    assert _mutant_decoder("none")(payload, data["raw_bytes"], codebooks[:32]) == raw
    assert _mutant_decoder(kind)(payload, data["raw_bytes"], codebooks[:32]) != raw


# ---------------------------------------------------------------------------
# a16: codebook fit (tests/test_extract_llama_top16_codebooks.py:15-38)

def test_fit_known_answer(golden_dir):
    kat = json.loads((golden_dir / "kat_fit.json").read_text())
    assert bytes(oracle.fit_top16_py(kat["histogram"])).hex() == kat["first_codebook_hex"]
    # ties break on the smaller exponent; fewer than 16 observed -> no codebook
    hist = [0] * 256
    for e in range(40, 60):
        hist[e] = 5
    assert oracle.fit_top16_py(hist) == list(range(40, 56))
    hist = [0] * 256
    hist[3] = 1
    assert oracle.fit_top16_py(hist) is None


def test_histogram_matches_bincount():
    rng = np.random.default_rng(3)
    words = rng.integers(0, 1 << 16, 5001, dtype=np.uint16)
    counts = oracle.exponent_histogram(words)
    half = words.size // 2
    exps = (words.astype(np.int64) >> 7) & 0xFF
    assert np.array_equal(counts[0], np.bincount(exps[:half], minlength=256))
    assert np.array_equal(counts[1], np.bincount(exps[half:], minlength=256))


# ---------------------------------------------------------------------------
# encoder/decoder on random data: inverse property and brute force

@pytest.mark.parametrize("n,rate", [(22, 0.0), (23, 0.05), (1000, 0.003), (4097, 0.001),
                                    (20000, 0.004), (20000, 0.02)])
def test_random_roundtrip_and_bruteforce(codebooks, n, rate):
    rng = np.random.default_rng(n * 7 + int(rate * 1000))
    books = codebooks[5 * 32:6 * 32]
    tables = oracle.top16_tables(books)
    words = _random_words(rng, n, books, rate)
    payload = oracle.top16_encode(words, tables)
    assert payload is not None
    if n <= 5000:
        assert oracle.encode_top16_py(list(map(int, words)), bytes(tables)) == bytes(payload)
    escapes = int(((np.frombuffer(bytes(tables), np.uint8)[
        np.where(np.arange(n) >= n // 2, 256, 0) + ((words.astype(np.int64) >> 7) & 0xFF)]) == 255).sum())
    cap = codec_format.top16_escape_capacity(n)
    assert payload[0] == (255 if escapes > cap else 5)
    assert int.from_bytes(bytes(payload[1:5]), "little") == min(escapes, cap)
    if escapes <= cap:
        decoded = oracle.top16_decode(payload, n, tables)
        assert np.array_equal(decoded, words)
        if n % 2 == 0 and n <= 5000:
            assert oracle.decode_top16_payload_py(bytes(payload), 2 * n, books) == words.tobytes()
        # entries ascending, padding zero
        entries = codec_format.top16_escapes(payload, n)
        assert [p for p, _ in entries] == sorted(p for p, _ in entries)
        lo, hi = codec_format.top16_sections(n)["escapes"]
        assert not any(bytes(payload[lo + 5 * escapes:hi]))


def test_decoder_accepts_any_escape_order_and_padding(codebooks):
    rng = np.random.default_rng(11)
    n = 4000
    books = codebooks[:32]
    tables = oracle.top16_tables(books)
    words = _random_words(rng, n, books, 0.004)
    payload = bytearray(oracle.top16_encode(words, tables))
    assert payload[0] == 5
    count = int.from_bytes(payload[1:5], "little")
    assert count > 3
    lo, hi = codec_format.top16_sections(n)["escapes"]
    slots = [bytes(payload[lo + 5 * s: lo + 5 * s + 5]) for s in range(count)]
    random.Random(5).shuffle(slots)
    payload[lo:lo + 5 * count] = b"".join(slots)
    payload[lo + 5 * count:hi] = bytes(rng.integers(0, 256, hi - lo - 5 * count, dtype=np.uint8))
    shuffled = np.frombuffer(bytes(payload), np.uint8)
    assert np.array_equal(oracle.top16_decode(shuffled, n, tables), words)
    assert oracle.decode_top16_payload_py(bytes(payload), 2 * n, books) == words.tobytes()
    assert codec_format.top16_equivalent(bytes(payload), bytes(oracle.top16_encode(words, tables)), n)


def test_decode_skips_payload_without_mode5(codebooks):
    tables = oracle.top16_tables(codebooks[:32])
    payload = np.zeros(codec_format.top16_encoded_size(64), np.uint8)
    payload[0] = 255
    initial = np.arange(64, dtype=np.uint16)
    assert np.array_equal(oracle.top16_decode(payload, 64, tables, initial=initial), initial)


# ---------------------------------------------------------------------------
# a7 gather and a10 scatter: brute force against numpy indexing

def test_gather_and_scatter_match_fancy_indexing():
    rng = np.random.default_rng(2)
    blocks, bw = 9, 24
    kv = rng.integers(0, 1 << 16, (2, blocks, bw), dtype=np.uint16)
    ids = [7, 2, 5, 0]
    got = oracle.gather(kv, blocks * bw, bw, bw, ids)
    assert np.array_equal(got, kv[:, ids].reshape(-1))
    target = np.zeros_like(kv)
    flat = target.reshape(-1)
    oracle.scatter(got, flat, len(ids), bw, blocks * bw, bw, ids=ids)
    assert np.array_equal(target[:, ids], kv[:, ids])
    untouched = [b for b in range(blocks) if b not in ids]
    assert not target[:, untouched].any()
    target2 = np.zeros_like(kv)
    oracle.scatter(kv[:, 3:6].reshape(-1), target2.reshape(-1), 3, bw, blocks * bw, bw,
                   block_start=3)
    assert np.array_equal(target2[:, 3:6], kv[:, 3:6])


def test_paged_batch_equals_gather_then_encode(codebooks):
    rng = np.random.default_rng(9)
    pool, bw = 64, 256
    books = codebooks[3 * 32:4 * 32]
    tables = oracle.top16_tables(books)
    kv = np.empty((2, pool, bw), np.uint16)
    kv[:] = _random_words(rng, kv.size, books, 0.002).reshape(kv.shape)
    perm = rng.permutation(pool)
    tables_r = [perm[0:5], perm[5:17], perm[17:18]]
    sizes = [codec_format.top16_encoded_size(2 * len(t) * bw) for t in tables_r]
    offsets = np.cumsum([0] + sizes[:-1]) + 3
    out = oracle.encode_paged_batch(kv, pool * bw, bw, bw, tables_r, offsets, int(sum(sizes)) + 3,
                                    tables, chunk=512, threads=4)
    for t, off, size in zip(tables_r, offsets, sizes):
        ref = oracle.top16_encode(oracle.gather(kv, pool * bw, bw, bw, t), tables)
        assert bytes(out[off:off + size]) == bytes(ref)
    # decode batch into an independent receiver table == scatter(decode)
    recv = np.zeros((2, pool, bw), np.uint16)
    rperm = rng.permutation(pool)
    recv_tables = [rperm[0:5], rperm[5:17], rperm[17:18]]
    oracle.decode_paged_batch(out, offsets, recv.reshape(-1), pool * bw, bw, bw, recv_tables,
                              tables, chunk=777, threads=3)
    for src_t, dst_t in zip(tables_r, recv_tables):
        assert np.array_equal(recv[:, dst_t], kv[:, src_t])


# ---------------------------------------------------------------------------
# the reference's own GPU round-trip inputs (tests/test_splitzip_cuda.py:137-185),
# here on the CPU oracle

@pytest.mark.parametrize("block_count,target_blocks,block_ids", [
    (1, 4, [3]), (128, 256, list(range(0, 256, 2)))])
def test_reference_formula_roundtrip(codebooks, block_count, target_blocks, block_ids):
    count = 2 * block_count * 2048
    index = np.arange(count)
    books = np.frombuffer(codebooks[:32], np.uint8).reshape(2, 16)
    plane = index // (count // 2)
    exponent = books[plane, index % 16].astype(np.int64)
    exponent[::400] = 100
    words = (((index % 2) << 15) | (exponent << 7) | (index % 128)).astype(np.uint16)
    tables = oracle.top16_tables(codebooks[:32])
    payload = oracle.top16_encode(words, tables)
    assert payload[0] == 5
    assert 2 * count / payload.size >= 1.30
    target = np.zeros((2, target_blocks, 2048), np.uint16)
    decoded = oracle.top16_decode(payload, count, tables)
    oracle.scatter(decoded, target.reshape(-1), block_count, 2048, target_blocks * 2048, 2048,
                   ids=block_ids)
    assert np.array_equal(target[:, block_ids].reshape(-1), words)


# ---------------------------------------------------------------------------
# fixed6 (mode 3), the Top-16 overflow fallback

def test_fixed6_matches_bit_unpacking_restatement():
    rng = np.random.default_rng(4)
    n = 1003
    highs = np.array([0x3F, 0x40, 0xBF, 0xC0, 0x41, 0x3E], np.uint16)
    words = ((highs[rng.integers(0, highs.size, n)] << 8) | rng.integers(0, 256, n)).astype(np.uint16)
    payload = oracle.fixed6_encode(words)
    assert payload[0] == 3
    palette = bytes(payload[1:65])
    assert list(palette[:6]) == sorted(int(h) for h in highs) and not any(palette[6:])
    low = bytes(payload[65:65 + n])
    codes = oracle.unpack_bits_py(bytes(payload[65 + n:]), n, 6)
    rebuilt = np.array([(palette[c] << 8) | low[i] for i, c in enumerate(codes)], np.uint16)
    assert np.array_equal(rebuilt, words)
    assert np.array_equal(oracle.fixed6_decode(payload, n), words)
    # a permuted palette (the reference's first-come order) decodes the same
    perm = [2, 0, 5, 1, 4, 3]
    remap = {old: new for new, old in enumerate(perm)}
    pal2 = bytes(palette[i] for i in perm) + bytes(58)
    codes2 = [remap[c] for c in codes]
    value = sum(c << (6 * i) for i, c in enumerate(codes2))
    packed2 = value.to_bytes(len(payload) - 65 - n, "little")
    payload2 = np.frombuffer(bytes([3]) + pal2 + bytes(low) + packed2, np.uint8)
    assert np.array_equal(oracle.fixed6_decode(payload2, n), words)


def test_fixed6_overflow_marks_255():
    words = (np.arange(65, dtype=np.uint16) << 8) | 1
    words = np.tile(words, 8)
    payload = oracle.fixed6_encode(words)
    assert payload[0] == 255
    ok = oracle.fixed6_encode(np.tile(words[:64], 8))
    assert ok is not None and ok[0] == 3


def test_fixed5_matches_bit_unpacking_restatement():
    """fixed5 (mode 4): 32-entry ascending palette, 8 x 5-bit codes per 5 bytes,
    LSB first, as the connector's mode-4 torch decoder reads them
    (src/unchain_kv/vllm_connector.py:5266-5275 with _unpack_splitzip_bits)."""
    rng = np.random.default_rng(12)
    n = 1001
    highs = np.array(sorted(rng.choice(256, 29, replace=False)), np.uint16)
    words = ((highs[rng.integers(0, highs.size, n)] << 8) | rng.integers(0, 256, n)).astype(np.uint16)
    payload = oracle.palette_encode(words, 5)
    assert payload.size == 33 + n + ((n + 7) // 8) * 5 and payload[0] == 4
    palette = bytes(payload[1:33])
    assert list(palette[:29]) == [int(h) for h in highs] and not any(palette[29:])
    low = bytes(payload[33:33 + n])
    codes = oracle.unpack_bits_py(bytes(payload[33 + n:]), n, 5)
    rebuilt = np.array([(palette[c] << 8) | low[i] for i, c in enumerate(codes)], np.uint16)
    assert np.array_equal(rebuilt, words)
    assert np.array_equal(oracle.palette_decode(payload, n, 5), words)
    # a fixed5 payload is not a fixed6 payload: the fixed6 decoder leaves it alone
    assert not oracle.palette_decode(payload, n, 6).any()


def test_fixed5_overflow_marks_255_and_fixed6_agrees_with_generic_form():
    words = np.tile((np.arange(33, dtype=np.uint16) << 8) | 7, 4)
    assert oracle.palette_encode(words, 5)[0] == 255
    assert oracle.palette_encode(np.tile((np.arange(32, dtype=np.uint16) << 8) | 7, 4), 5)[0] == 4
    rng = np.random.default_rng(2)
    w6 = ((rng.integers(0, 40, 777) << 8) | rng.integers(0, 256, 777)).astype(np.uint16)
    assert np.array_equal(oracle.palette_encode(w6, 6), oracle.fixed6_encode(w6))
