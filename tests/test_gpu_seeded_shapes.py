"""Seeded sweep of shapes through the drop-in and batched Top-16 entry points:
block sizes of 1 to 16 KiB words, one to five requests of 1 to 12 blocks, payload
buffers at every byte offset mod 16, escape rates from none to overflow. Every
payload is compared byte for byte with the oracle's, every decode with the source
words (through the host block table, the device table and the escape directory).
UNCHAIN_KV_TEST_SEEDS sets the number of seeds (16 by default).
"""

import ctypes
import os

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


def say(*parts):
    print("[case]", *parts, flush=True)


def u16(t) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def words_for(rng, n, books, rate):
    half = n // 2
    outside = np.array(sorted(set(range(256)) - set(books)), np.uint16)
    exps = np.empty(n, np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:], np.uint8)[rng.integers(0, 16, n - half)]
    esc = rng.random(n) < rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    return ((rng.integers(0, 2, n).astype(np.uint16) << 15) | (exps << 7) |
            rng.integers(0, 128, n).astype(np.uint16)).astype(np.uint16)


# more seeds for a wider sweep: UNCHAIN_KV_TEST_SEEDS=<count>
SEEDS = int(os.environ.get("UNCHAIN_KV_TEST_SEEDS", "16"))


@pytest.mark.parametrize("seed", range(SEEDS))
def test_seeded_shapes(sz, codebooks, seed):
    rng = np.random.default_rng(1000 + seed)
    bw = int(rng.choice([1024, 2048, 3072, 8192, 16384]))
    counts = rng.integers(1, 13, int(rng.integers(1, 6))).tolist()
    rate = float(rng.choice([0.0, 0.0005, 0.003, 0.012]))
    shift = int(rng.integers(0, 16))
    layer = int(rng.integers(0, 32))
    say("seeded", seed, bw, counts, rate, shift, layer)
    books = codebooks[32 * layer:32 * layer + 32]
    tables = oracle.top16_tables(books)
    pool = sum(counts) + 5
    words = words_for(rng, 2 * pool * bw, books, rate)
    host = words.reshape(2, pool, bw)
    kv = torch.from_numpy(words.view(np.int16).copy()).cuda().view(torch.bfloat16).view(2, pool, bw)
    perm = rng.permutation(pool).tolist()
    block_tables, at = [], 0
    for c in counts:
        block_tables.append(perm[at:at + c])
        at += c
    refs = [oracle.top16_encode(host[:, t].reshape(-1), tables) for t in block_tables]
    recv_perm = rng.permutation(pool).tolist()
    recv_tables, at = [], 0
    for c in counts:
        recv_tables.append(recv_perm[at:at + c])
        at += c

    # drop-in, per request: gathered source, payload `shift` bytes into its buffer
    target = torch.zeros_like(kv)
    for t, rt, ref in zip(block_tables, recv_tables, refs):
        n = 2 * len(t) * bw
        source = kv[:, t].contiguous()
        backing = torch.full((2 * n + shift + 64,), 0xA5, dtype=torch.uint8, device="cuda")
        out = backing[shift:shift + 2 * n]
        size = sz.encode_top16(source, out, layer)
        assert size == codec_format.top16_encoded_size(n)
        got = out[:size].cpu().numpy()
        assert bytes(got) == bytes(ref)
        if ref[0] == 5:
            assert sz.decode_top16(out[:size], target, rt, 2 * n, layer) == 2 * n
    torch.cuda.synchronize()
    dst = u16(target).reshape(2, pool, bw)
    for t, rt, ref in zip(block_tables, recv_tables, refs):
        if ref[0] == 5:
            assert np.array_equal(dst[:, rt], host[:, t])

    # batched: payloads packed at odd offsets, with the escape directory
    batch = sz.PagedBatch(block_tables, bw, "cuda")
    offsets, at = [], 0
    for e in batch.encoded_bytes:
        at += shift + 1
        offsets.append(at)
        at += e
    batch.out_offsets = offsets
    batch._out_offsets = (ctypes.c_ulonglong * len(offsets))(*offsets)
    out = torch.zeros(at + 64, dtype=torch.uint8, device="cuda")
    directory = batch.new_directory()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), layer,
                                 directory=directory) == batch.total_encoded_bytes
    got = out.cpu().numpy()
    for o, ref in zip(offsets, refs):
        assert bytes(got[o:o + len(ref)]) == bytes(ref)
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    target2 = torch.zeros_like(kv)
    assert sz.decode_top16_paged(out, offsets, batch.encoded_bytes, target2, recv, layer,
                                 directory=directory) == batch.total_raw_bytes
    torch.cuda.synchronize()
    dst2 = u16(target2).reshape(2, pool, bw)
    for t, rt, ref in zip(block_tables, recv_tables, refs):
        if ref[0] == 5:
            assert np.array_equal(dst2[:, rt], host[:, t])
        else:
            assert not dst2[:, rt].any()
