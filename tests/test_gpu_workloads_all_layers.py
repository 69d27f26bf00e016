"""Encoder byte parity with the oracle on every layer of the other benchmark
workloads (the Llama-3-8B paged workload's 32 layers are covered in
test_gpu_workloads.py):

* Llama-3.2-1B, one 1024-token request on contiguous blocks: all 16 layers through
  the batched call, payload bytes equal to the oracle's, exact round trip.
* Llama-3-8B with 1% outliers: all 32 layers on the path the benchmark times for
  them, a Top-16 probe encode (presence masks and palette records in its launches,
  no escape placement in an overflowed payload) and the fixed6 re-encode from the
  palette records. Every overflowed payload has the oracle's header, body and
  codes; every fixed6 payload is the oracle's; the fixed6 payloads decode and
  scatter exactly.
* One GPU's share of Llama-3-70B under TP=8 (64 requests of 128 .. 32768 tokens):
  all 80 layers, byte parity of all 64 payloads with the oracle, exact round trip
  (in chunks of layers, one test each, so every test stays short).
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


def round_trip_equal(kv, target, tables, recv_tables):
    src = torch.tensor([b for t in tables for b in t], device="cuda")
    dst = torch.tensor([b for t in recv_tables for b in t], device="cuda")
    return torch.equal(kv.view(torch.int16)[:, src], target.view(torch.int16)[:, dst])


def test_llama32_1b_every_layer(env):
    sz, wl = env
    shape = wl.LLAMA32_1B
    ids = list(range(64))
    batch = sz.PagedBatch([ids], shape.block_words, "cuda")
    out, ws = batch.new_payload_buffer(), batch.new_workspace()
    for layer in range(shape.layers):
        say("llama3.2-1b layer", layer)
        kv = wl.make_kv_layer(torch, shape, 64, seed=1, layer=layer, device="cuda")
        books = wl.fit_codebook(torch, kv, [ids])
        ref = oracle.top16_encode(host_words(kv).reshape(-1), oracle.top16_tables(books))
        assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books) == \
            batch.total_encoded_bytes
        a = batch.out_offsets[0]
        assert bytes(out[a:a + batch.encoded_bytes[0]].cpu().numpy()) == bytes(ref), layer
        target = torch.zeros_like(kv)
        assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, batch,
                                     codebooks=books) == batch.total_raw_bytes
        assert torch.equal(target.view(torch.int16), kv.view(torch.int16)), layer


def test_llama3_8b_outliers_every_layer_probe_then_fixed6(env):
    sz, wl = env
    shape = wl.LLAMA3_8B
    bw = shape.block_words
    tables = wl.random_block_tables(torch, 4096, [256] * 8, seed=1)
    recv_tables = wl.random_block_tables(torch, 4096, [256] * 8, seed=7920)
    batch = sz.PagedBatch(tables, bw, "cuda")
    out, ws = batch.new_payload_buffer(), batch.new_workspace()
    presence, info = batch.new_presence(), batch.new_palette_info()
    for layer in range(shape.layers):
        say("llama3-8b outliers layer", layer)
        kv = wl.make_kv_layer(torch, shape, 4096, seed=1, layer=layer, device="cuda",
                              outlier_rate=0.01)
        books = wl.fit_codebook(torch, kv, tables)
        tab = oracle.top16_tables(books)
        assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books, presence=presence,
                                     palette_info=info) == batch.total_encoded_bytes
        kv_host = host_words(kv)
        got = out.cpu().numpy()
        ref = oracle.encode_paged_batch(kv_host, 4096 * bw, bw, bw, tables, batch.out_offsets,
                                        batch.out_bytes, tab, threads=oracle.default_threads())
        over = []
        for r, n in enumerate(batch.count_words):
            a, e = batch.out_offsets[r], batch.encoded_bytes[r]
            if ref[a] == 255:
                over.append(r)
                body_end = 5 + n + (n + 1) // 2
                assert bytes(got[a:a + body_end]) == bytes(ref[a:a + body_end]), (layer, r)
            else:
                assert bytes(got[a:a + e]) == bytes(ref[a:a + e]), (layer, r)
        assert over, layer  # 1 % outliers exceed the 0.5 % escape capacity
        sub = sz.PagedBatch([tables[r] for r in over], bw, "cuda")
        offsets, sizes, _ = sub.palette_layout(6)
        six = sub.new_palette_buffer(6)
        assert sz.encode_bf16_paged(kv, sub, six, None, bits=6, palette_info=info,
                                    info_first=over) == sum(sizes)
        host6 = six.cpu().numpy()
        for k, r in enumerate(over):
            expect = oracle.palette_encode(kv_host[:, tables[r]].reshape(-1), 6)
            assert bytes(host6[offsets[k]:offsets[k] + sizes[k]]) == bytes(expect), (layer, r)
        sub_recv = sz.PagedBatch([recv_tables[r] for r in over], bw, "cuda")
        target = torch.zeros_like(kv)
        assert sz.decode_bf16_paged(six, offsets, sizes, target, sub_recv, bits=6) == \
            sub.total_raw_bytes
        assert round_trip_equal(kv, target, [tables[r] for r in over],
                                [recv_tables[r] for r in over]), layer


@pytest.mark.parametrize("first", list(range(0, 80, 10)))
def test_llama3_70b_tp8_every_layer(env, first):
    sz, wl = env
    shape = wl.LLAMA3_70B_TP8
    bw = shape.block_words
    tokens = wl.mixed_context_lengths(torch, 64, 128, 32768, shape.block_size, seed=1)
    blocks = [t // shape.block_size for t in tokens]
    pool = sum(blocks) + 64
    tables = wl.random_block_tables(torch, pool, blocks, seed=1)
    recv_tables = wl.random_block_tables(torch, pool, blocks, seed=7920)
    batch = sz.PagedBatch(tables, bw, "cuda")
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    out, ws = batch.new_payload_buffer(), batch.new_workspace()
    directory = batch.new_directory()
    for layer in range(first, min(first + 10, shape.layers)):
        say("70b tp8 layer", layer)
        kv = wl.make_kv_layer(torch, shape, pool, seed=1, layer=layer, device="cuda")
        books = wl.fit_codebook(torch, kv, tables)
        assert sz.encode_top16_paged(kv, batch, out, ws, codebooks=books, directory=directory) \
            == batch.total_encoded_bytes
        ref = oracle.encode_paged_batch(host_words(kv), pool * bw, bw, bw, tables,
                                        batch.out_offsets, batch.out_bytes,
                                        oracle.top16_tables(books),
                                        threads=oracle.default_threads())
        got = out.cpu().numpy()
        for r in range(len(tables)):
            a, b = batch.out_offsets[r], batch.out_offsets[r] + batch.encoded_bytes[r]
            assert bytes(got[a:b]) == bytes(ref[a:b]), (layer, r)
        target = torch.zeros_like(kv)
        assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, recv,
                                     codebooks=books, directory=directory) == \
            batch.total_raw_bytes
        assert round_trip_equal(kv, target, tables, recv_tables), layer
