"""The torch-CPU restatement of the Top-16 codec (oracle/torch_codec.py, the
``ref-cpu-torch`` CPU baseline) gives the C oracle's bytes: canonical payloads on
random words with and without escapes and overflow, the reference's 256-word
known answer, and paged gather/scatter round trips."""

import json

import numpy as np
import pytest

import oracle
from oracle import torch_codec

torch = pytest.importorskip("torch")


def _words(rng, n, books, rate):
    half = n // 2
    outside = np.array(sorted(set(range(256)) - set(books)), dtype=np.uint16)
    exps = np.empty(n, dtype=np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:], np.uint8)[rng.integers(0, 16, n - half)]
    esc = rng.random(n) < rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    low = rng.integers(0, 256, n).astype(np.uint16)
    return ((exps << 7) | (low & 0x7F) | ((low & 0x80) << 8)).astype(np.uint16)


@pytest.mark.parametrize("n,rate", [(22, 0.0), (23, 0.1), (1001, 0.004), (65536, 0.001),
                                    (20000, 0.02)])
def test_torch_encode_decode_match_the_c_oracle(codebooks, n, rate):
    rng = np.random.default_rng(n)
    books = codebooks[4 * 32:5 * 32]
    tables = oracle.top16_tables(books)
    words = _words(rng, n, books, rate)
    ref = oracle.top16_encode(words, tables)
    tab_t = torch.from_numpy(tables.copy())
    got = torch_codec.encode_top16(torch.from_numpy(words.view(np.int16).copy()), tab_t, torch)
    assert bytes(got.numpy()) == bytes(ref)
    decoded = torch_codec.decode_top16(got, n, tab_t, torch)
    if ref[0] == 5:
        assert np.array_equal(decoded.numpy().astype(np.uint16), words)
    else:
        assert decoded is None


def test_torch_decoder_known_answer(golden_dir, codebooks):
    kat = json.loads((golden_dir / "kat_top16_256.json").read_text())
    payload = torch.tensor(list(bytes.fromhex(kat["payload_hex"])), dtype=torch.uint8)
    words = np.frombuffer(bytes.fromhex(kat["raw_hex"]), "<u2")
    tables = torch.from_numpy(oracle.top16_tables(codebooks[:32]).copy())
    got = torch_codec.decode_top16(payload, 256, tables, torch)
    assert np.array_equal(got.numpy().astype(np.uint16), words)


def test_torch_paged_roundtrip(codebooks):
    rng = np.random.default_rng(8)
    books = codebooks[:32]
    tables = torch.from_numpy(oracle.top16_tables(books).copy())
    pool, bw = 12, 2048
    kv = torch.from_numpy(_words(rng, 2 * pool * bw, books, 0.002).view(np.int16)).reshape(
        2, pool, 16, 1, 128)
    send = [[3, 7, 1], [10, 0]]
    recv = [[2, 4, 5], [11, 9]]
    payloads = torch_codec.encode_paged(kv, send, tables, torch)
    for ids, p in zip(send, payloads):
        ref = oracle.top16_encode(kv.index_select(1, torch.tensor(ids)).reshape(-1).numpy()
                                  .view(np.uint16), tables.numpy())
        assert bytes(p.numpy()) == bytes(ref)
    target = torch.zeros_like(kv)
    torch_codec.decode_paged(payloads, target, recv, tables, torch)
    for s, r in zip(send, recv):
        assert torch.equal(target[:, r], kv[:, s])
