"""Seeded sweep of the batched palette codecs (fixed6 mode 3, fixed5 mode 4): block
sizes from 48 to 16 Ki words, one to five requests of 1 to 12 blocks from a shuffled
pool, palettes from one high byte to one past the mode's limit (overflow), and the
KV view at an even or a 2-byte offset. Each payload is compared byte for byte with
the oracle's canonical encode (an overflowed one: byte 0 = 255, nothing else
written), and the decode + scatter of every batch without overflow with the source
words. UNCHAIN_KV_TEST_SEEDS sets the number of seeds (16 by default)."""

import os

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SEEDS = int(os.environ.get("UNCHAIN_KV_TEST_SEEDS", "16"))


@pytest.fixture(scope="module")
def sz():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda

    assert splitzip_cuda.available(), splitzip_cuda.load_error()
    return splitzip_cuda


def u16(t) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


@pytest.mark.parametrize("seed", range(SEEDS))
def test_seeded_palette_shapes(sz, seed):
    rng = np.random.default_rng(5000 + seed)
    bits = int(rng.choice([6, 5]))
    limit = 64 if bits == 6 else 32
    bw = int(rng.choice([48, 1024, 2048, 3072, 8192, 16384]))
    counts = rng.integers(1, 13, int(rng.integers(1, 6))).tolist()
    offset = int(rng.choice([0, 0, 1]))
    pool = sum(counts) + int(rng.integers(0, 5))
    print("[case] seeded palette", seed, bits, bw, counts, offset, flush=True)
    # each request draws its high bytes from its own palette; some go one past the limit
    perm = rng.permutation(pool).tolist()
    tables, at = [], 0
    for c in counts:
        tables.append(perm[at:at + c])
        at += c
    kv_host = rng.integers(0, 1 << 16, (2, pool, bw), dtype=np.uint16)
    sizes_wanted = []
    for t in tables:
        distinct = int(rng.choice([1, 2, limit // 2, limit - 1, limit, limit + 1]))
        highs = rng.choice(256, distinct, replace=False).astype(np.uint16)
        picks = highs[rng.integers(0, distinct, (2, len(t), bw))]
        if distinct <= limit:
            kv_host[:, t] = (picks << 8) | (kv_host[:, t] & 0xFF)
        else:
            # every high byte present at least once
            flat = picks.reshape(-1)
            flat[:distinct] = highs
            kv_host[:, t] = (flat.reshape(picks.shape) << 8) | (kv_host[:, t] & 0xFF)
        sizes_wanted.append(distinct)
    backing = torch.from_numpy(
        np.concatenate([np.zeros(offset, np.uint16), kv_host.reshape(-1)]).view(np.int16).copy()
    ).cuda().view(torch.bfloat16)
    kv = backing[offset:].view(2, pool, bw)
    batch = sz.PagedBatch(tables, bw, "cuda")
    offsets, sizes, _ = batch.palette_layout(bits)
    out = batch.new_palette_buffer(bits)
    out.fill_(0x5A)
    ws = batch.new_palette_workspace()
    if any(size >= raw for size, raw in zip(sizes, batch.raw_bytes)):
        # a payload that would not be smaller than its raw words: the whole call
        # declines, as the reference's encode does per request
        assert sz.encode_bf16_paged(kv, batch, out, ws, bits=bits) is None
        return
    assert sz.encode_bf16_paged(kv, batch, out, ws, bits=bits) == sum(sizes)
    torch.cuda.synchronize()
    host = out.cpu().numpy()
    overflowed = False
    for r, t in enumerate(tables):
        got = host[offsets[r]:offsets[r] + sizes[r]]
        if sizes_wanted[r] > limit:
            overflowed = True
            assert got[0] == 255 and not (got[1:] != 0x5A).any(), f"payload {r}"
        else:
            ref = oracle.palette_encode(kv_host[:, t].reshape(-1), bits)
            assert bytes(got) == bytes(ref), f"payload {r}"
    if overflowed:
        return
    rperm = rng.permutation(pool).tolist()
    recv_tables, at = [], 0
    for c in counts:
        recv_tables.append(rperm[at:at + c])
        at += c
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    target = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    assert sz.decode_bf16_paged(out, offsets, sizes, target, recv, bits=bits) == \
        batch.total_raw_bytes
    torch.cuda.synchronize()
    got = u16(target).reshape(2, pool, bw)
    for src_t, dst_t in zip(tables, recv_tables):
        assert np.array_equal(got[:, dst_t], kv_host[:, src_t])
