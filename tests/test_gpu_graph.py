"""The batched codec calls under HIP graph capture.

The library's entry points only launch kernels with by-value arguments on the
caller's stream (no allocation, no memset, no host synchronisation), so a layer's
encode and decode can be captured once and replayed. Each replay here follows
eager work that changes the KV layer, and is checked byte for byte against the
oracle's payloads for the new contents and against the exact round trip.
"""

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


def layer_words(rng, books, n, escape_rate):
    half = n // 2
    exps = np.empty(n, np.uint16)
    exps[:half] = np.frombuffer(books[:16], np.uint8)[rng.integers(0, 16, half)]
    exps[half:] = np.frombuffer(books[16:], np.uint8)[rng.integers(0, 16, n - half)]
    outside = np.array(sorted(set(range(256)) - set(books)), np.uint16)
    esc = rng.random(n) < escape_rate
    exps[esc] = outside[rng.integers(0, outside.size, int(esc.sum()))]
    return ((rng.integers(0, 2, n).astype(np.uint16) << 15) | (exps << 7)
            | rng.integers(0, 128, n).astype(np.uint16))


def test_paged_encode_decode_replay(sz, codebooks):
    books = codebooks[6 * 32:7 * 32]
    tab = oracle.top16_tables(books)
    bw, pool = 2048, 96
    rng = np.random.default_rng(4)
    perm = rng.permutation(pool).tolist()
    tables = [perm[0:9], perm[9:30], perm[30:34]]
    recv_tables = [perm[40:49], perm[49:70], perm[70:74]]
    batch = sz.PagedBatch(tables, bw, "cuda")
    recv = sz.PagedBatch(recv_tables, bw, "cuda")
    device_tables = sz.top16_tables_for(books, torch.device("cuda"), torch)
    kv = torch.zeros((2, pool, bw), dtype=torch.bfloat16, device="cuda")
    out = batch.new_payload_buffer()
    ws = batch.new_workspace()
    target = torch.zeros_like(kv)

    def step():
        assert sz.encode_top16_paged(kv, batch, out, ws, tables=device_tables)
        assert sz.decode_top16_paged(out, batch.out_offsets, batch.encoded_bytes, target, recv,
                                     tables=device_tables)

    step()  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for replay in range(3):
        say("graph replay", replay)
        words = layer_words(rng, books, 2 * pool * bw, 0.002 * replay)
        # eager work between replays: new layer contents, receiver cleared
        kv.copy_(torch.from_numpy(words.view(np.int16)).cuda().view(torch.bfloat16).view(2, pool, bw))
        target.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        host = out.cpu().numpy()
        kv_host = words.reshape(2, pool, bw)
        got = target.view(torch.int16).cpu().numpy().view(np.uint16).reshape(2, pool, bw)
        for r, t in enumerate(tables):
            ref = oracle.top16_encode(kv_host[:, t].reshape(-1), tab)
            a = batch.out_offsets[r]
            assert bytes(host[a:a + batch.encoded_bytes[r]]) == bytes(ref), (replay, r)
            assert np.array_equal(got[:, recv_tables[r]], kv_host[:, t]), (replay, r)
