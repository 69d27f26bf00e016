"""Parity at the benchmark workloads' full sizes.

* Llama-3-8B paged (8 x 4096 tokens, 4096-block pool): every one of the 32 layers
  is encoded with its escape directory (the benchmark's path), matches the oracle
  byte for byte, and round-trips exactly into an independent receiver table.
* The same shapes with 1% outliers: every Top-16 payload overflows (byte 0 = 255,
  capacity-clamped count, the first ``cap`` escapes in ascending order), matches
  the oracle byte for byte, and the fixed6 re-encode of the batch matches the
  oracle and decodes + scatters exactly.
* One GPU's share of Llama-3-70B under TP=8 (64 requests of log-uniform
  128 .. 32768 tokens): byte parity of all 64 payloads of a layer with the oracle,
  exact round trip.
* Llama-3.2-1B, one 1024-token request on contiguous blocks: the per-request
  drop-in calls and the batched call give the oracle's payload and round-trip.
"""

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda, workloads

    assert splitzip_cuda.available(), splitzip_cuda.load_error()
    return splitzip_cuda, workloads


def say(*parts):
    print("[case]", *parts, flush=True)


def host_words(kv):
    return kv.view(torch.int16).cpu().numpy().view(np.uint16).reshape(2, kv.shape[1], -1)


def test_llama3_8b_all_layers_round_trip(env):
    sz, wl = env
    shape = wl.LLAMA3_8B
    tables = wl.random_block_tables(torch, 4096, [256] * 8, seed=1)
    recv_tables = wl.random_block_tables(torch, 4096, [256] * 8, seed=7920)
    batch = sz.PagedBatch(tables, shape.block_words, "cuda")
    recv = sz.PagedBatch(recv_tables, shape.block_words, "cuda")
    out, ws = batch.new_payload_buffer(), batch.new_workspace()
    directory = batch.new_directory()
    src = torch.tensor([b for t in tables for b in t], device="cuda")
    dst = torch.tensor([b for t in recv_tables for b in t], device="cuda")
    target = None
    for layer in range(shape.layers):
        say("llama3-8b layer", layer)
        kv = wl.make_kv_layer(torch, shape, 4096, seed=1, layer=layer, device="cuda")
        books = wl.fit_codebook(torch, kv, tables)
        if target is None:
            target = torch.zeros_like(kv)
        assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books, directory=directory) \
            == batch.total_encoded_bytes
        assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, recv,
                                     codebooks=books, directory=directory) == batch.total_raw_bytes
        assert torch.equal(kv.view(torch.int16)[:, src], target.view(torch.int16)[:, dst])
        host = out.cpu().numpy()
        ref = oracle.encode_paged_batch(host_words(kv), 4096 * shape.block_words,
                                        shape.block_words, shape.block_words, tables,
                                        batch.out_offsets, batch.out_bytes,
                                        oracle.top16_tables(books),
                                        threads=oracle.default_threads())
        for r, (a, e) in enumerate(zip(batch.out_offsets, batch.encoded_bytes)):
            assert host[a] == 5 and bytes(host[a:a + e]) == bytes(ref[a:a + e]), (layer, r)


def test_llama3_8b_outliers_overflow_then_fixed6(env):
    sz, wl = env
    shape = wl.LLAMA3_8B
    say("llama3-8b outliers")
    kv = wl.make_kv_layer(torch, shape, 4096, seed=1, layer=3, device="cuda", outlier_rate=0.01)
    tables = wl.random_block_tables(torch, 4096, [256] * 8, seed=1)
    recv_tables = wl.random_block_tables(torch, 4096, [256] * 8, seed=7920)
    books = wl.fit_codebook(torch, kv, tables)
    batch = sz.PagedBatch(tables, shape.block_words, "cuda")
    out = batch.new_payload_buffer()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), codebooks=books) == \
        batch.total_encoded_bytes
    kv_host = host_words(kv)
    bw = shape.block_words
    ref = oracle.encode_paged_batch(kv_host, 4096 * bw, bw, bw, tables, batch.out_offsets,
                                    batch.out_bytes, oracle.top16_tables(books),
                                    threads=oracle.default_threads())
    got = out.cpu().numpy()
    for r in range(8):
        a, b = batch.out_offsets[r], batch.out_offsets[r] + batch.encoded_bytes[r]
        assert got[a] == 255  # escapes beyond the 0.5% capacity
        assert int.from_bytes(bytes(got[a + 1:a + 5]), "little") == (batch.count_words[r] + 199) // 200
        assert bytes(got[a:b]) == bytes(ref[a:b]), f"payload {r}"
    offsets, sizes, _ = batch.palette_layout(6)
    six = batch.new_palette_buffer(6)
    assert sz.encode_bf16_paged(kv, batch, six, batch.new_palette_workspace(), bits=6) == sum(sizes)
    host6 = six.cpu().numpy()
    for r, t in enumerate(tables):
        expect = oracle.palette_encode(kv_host[:, t].reshape(-1), 6)
        assert expect[0] == 3
        assert bytes(host6[offsets[r]:offsets[r] + sizes[r]]) == bytes(expect), f"fixed6 {r}"
    recv = sz.PagedBatch(recv_tables, shape.block_words, "cuda")
    target = torch.zeros_like(kv)
    assert sz.decode_bf16_paged(six, offsets, sizes, target, recv, bits=6) == batch.total_raw_bytes
    src = torch.tensor([b for t in tables for b in t], device="cuda")
    dst = torch.tensor([b for t in recv_tables for b in t], device="cuda")
    assert torch.equal(kv.view(torch.int16)[:, src], target.view(torch.int16)[:, dst])


@pytest.mark.parametrize("layer", [0, 79])
def test_llama3_70b_tp8_mixed_batch(env, layer):
    sz, wl = env
    shape = wl.LLAMA3_70B_TP8
    say("70b tp8 mixed layer", layer)
    tokens = wl.mixed_context_lengths(torch, 64, 128, 32768, shape.block_size, seed=1)
    blocks = [t // shape.block_size for t in tokens]
    pool = sum(blocks) + 64
    tables = wl.random_block_tables(torch, pool, blocks, seed=1)
    recv_tables = wl.random_block_tables(torch, pool, blocks, seed=7920)
    kv = wl.make_kv_layer(torch, shape, pool, seed=1, layer=layer, device="cuda")
    books = wl.fit_codebook(torch, kv, tables)
    batch = sz.PagedBatch(tables, shape.block_words, "cuda")
    out = batch.new_payload_buffer()
    assert sz.encode_top16_paged(kv, batch, out, batch.new_workspace(), codebooks=books) == \
        batch.total_encoded_bytes
    bw = shape.block_words
    ref = oracle.encode_paged_batch(host_words(kv), pool * bw, bw, bw, tables, batch.out_offsets,
                                    batch.out_bytes, oracle.top16_tables(books),
                                    threads=oracle.default_threads())
    got = out.cpu().numpy()
    for r in range(len(tables)):
        a, b = batch.out_offsets[r], batch.out_offsets[r] + batch.encoded_bytes[r]
        assert bytes(got[a:b]) == bytes(ref[a:b]), f"payload {r}"
    recv = sz.PagedBatch(recv_tables, shape.block_words, "cuda")
    target = torch.zeros_like(kv)
    assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, recv,
                                 codebooks=books) == batch.total_raw_bytes
    src = torch.tensor([b for t in tables for b in t], device="cuda")
    dst = torch.tensor([b for t in recv_tables for b in t], device="cuda")
    assert torch.equal(kv.view(torch.int16)[:, src], target.view(torch.int16)[:, dst])


def test_llama32_1b_contiguous_request(env):
    sz, wl = env
    shape = wl.LLAMA32_1B
    say("llama3.2-1b contiguous")
    for layer in (0, 15):
        kv = wl.make_kv_layer(torch, shape, 64, seed=1, layer=layer, device="cuda")
        ids = list(range(64))
        books = wl.fit_codebook(torch, kv, [ids])
        ref = oracle.top16_encode(host_words(kv).reshape(-1), oracle.top16_tables(books))
        # per-request drop-in (the reference's call): contiguous source
        source = kv.contiguous()
        out = torch.empty(source.numel() * 2, dtype=torch.uint8, device="cuda")
        size = sz.encode_top16(source, out, layer, codebooks=books)
        target = torch.zeros_like(kv)
        assert sz.decode_top16(out[:size], target, ids, source.numel() * 2, layer,
                               codebooks=books) == source.numel() * 2
        torch.cuda.synchronize()
        assert bytes(out[:size].cpu().numpy()) == bytes(ref)
        assert torch.equal(target.view(torch.int16), kv.view(torch.int16))
        # batched call: same payload
        batch = sz.PagedBatch([ids], shape.block_words, "cuda")
        paged = batch.new_payload_buffer()
        sz.encode_top16_paged(kv, batch, paged, batch.new_workspace(), codebooks=books)
        a = batch.out_offsets[0]
        assert bytes(paged[a:a + batch.encoded_bytes[0]].cpu().numpy()) == bytes(ref)
