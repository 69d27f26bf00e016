"""The batched Top-16 encode that allocates nothing
(kvq_splitzip_bf16_encode_top16_paged_noalloc), called through the C ABI, against
the workspace entry point kvq_splitzip_bf16_encode_top16_paged: byte-identical
payload buffers on two calls in a row, the second with a smaller batch, and the
oracle's payloads for both. The scratch-size refusal needs no GPU."""

import ctypes

import numpy as np
import pytest

import oracle
from unchainkv_amd import splitzip_cuda as sz
from unchainkv_amd import workloads

torch = pytest.importorskip("torch")

U64 = ctypes.c_ulonglong


def _lib():
    lib = sz._load()
    if lib is None:
        pytest.skip(f"HIP library not built: {sz.load_error()}")
    return lib


def _u64s(values):
    values = [int(v) for v in values]
    return (U64 * len(values))(*values)


def test_noalloc_refuses_batches_beyond_its_scratch():
    """No GPU work: the size check comes before anything is launched."""
    lib = _lib()
    cap = int(lib.kvq_splitzip_top16_noalloc_scratch_bytes())
    assert cap == 16 << 20
    block_words = 16384
    # 40 payloads of 256 blocks: 20,480 tiles per 16 payloads ... well above the cap
    offsets = _u64s(range(0, 257 * 256, 256))
    need = int(lib.kvq_splitzip_top16_paged_workspace_bytes(block_words, offsets, 256))
    assert need > cap
    # every device pointer 0: were the size check not first, the call would decline
    # with 0 before any launch
    rc = lib.kvq_splitzip_bf16_encode_top16_paged_noalloc(
        0, 1 << 30, 1 << 14, block_words, 0, offsets, 256, 0, _u64s([0] * 256), 1 << 40, 0, 0, 0)
    assert rc == -1
    message = lib.kvq_splitzip_last_error().decode()
    assert "scratch" in message and str(need) in message and str(cap) in message


def test_noalloc_declines_decreasing_offsets_before_the_size_check():
    """Decreasing block offsets decline with 0, as the workspace entry point does,
    instead of a scratch-size error computed from a wrapped difference."""
    lib = _lib()
    offsets = _u64s([0, 256, 128, 384])
    assert int(lib.kvq_splitzip_top16_paged_workspace_bytes(16384, offsets, 3)) == 0
    rc = lib.kvq_splitzip_bf16_encode_top16_paged_noalloc(
        0, 1 << 30, 1 << 14, 16384, 0, offsets, 3, 0, _u64s([0] * 3), 1 << 40, 0, 0, 0)
    assert rc == 0


def _encode_both(lib, kv, batch, tables):
    """Payload buffers from the workspace entry point and from the no-allocation one."""
    ref = torch.zeros(batch.out_bytes, dtype=torch.uint8, device=kv.device)
    got = torch.zeros(batch.out_bytes, dtype=torch.uint8, device=kv.device)
    ws = batch.new_workspace()
    stream = int(torch.cuda.current_stream(kv.device).cuda_stream)
    common = (int(kv.data_ptr()), int(kv.stride(0)), int(kv.stride(1)), batch.block_words,
              int(batch.ids.data_ptr()), batch._block_offsets, batch.payload_count)
    a = lib.kvq_splitzip_bf16_encode_top16_paged(
        *common, int(ref.data_ptr()), batch._out_offsets, int(ref.numel()),
        int(tables.data_ptr()), int(ws.data_ptr()), int(ws.numel()), 0, stream)
    b = lib.kvq_splitzip_bf16_encode_top16_paged_noalloc(
        *common, int(got.data_ptr()), batch._out_offsets, int(got.numel()),
        int(tables.data_ptr()), 0, stream)
    torch.cuda.synchronize(kv.device)
    return a, b, ref.cpu().numpy(), got.cpu().numpy()


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point_twice():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    lib = _lib()
    device = torch.device("cuda", 0)
    shape = workloads.LLAMA3_8B
    pool = 512
    kv = workloads.make_kv_layer(torch, shape, pool, seed=7, layer=3, device=device,
                                 outlier_rate=0.002)
    kv_host = kv.view(torch.int16).cpu().numpy().view(np.uint16).reshape(2, pool, -1)
    # first call: 6 requests (one escape-heavy block range through the outliers);
    # second call: 2 smaller requests over other blocks
    for case, blocks in (("six requests", [64, 32, 48, 16, 80, 8]), ("two requests", [12, 4])):
        print("[case] noalloc", case, blocks, flush=True)
        tables = workloads.random_block_tables(torch, pool, blocks, seed=len(blocks))
        books = workloads.fit_codebook(torch, kv, tables)
        batch = sz.PagedBatch(tables, shape.block_words, device)
        tab = sz.top16_tables_for(books, device, torch)
        a, b, ref, got = _encode_both(lib, kv, batch, tab)
        assert a == b == batch.total_encoded_bytes
        assert np.array_equal(ref, got)
        tables_host = oracle.top16_tables(books)
        for r, t in enumerate(batch.block_tables):
            o = batch.out_offsets[r]
            expect = oracle.top16_encode(kv_host[:, t].reshape(-1), tables_host)
            assert bytes(got[o:o + batch.encoded_bytes[r]]) == bytes(expect), (case, r)
