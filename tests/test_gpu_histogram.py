"""GPU exponent histograms (the codebook-fit statistics) against numpy bincount.

The reference bins (word >> 7) & 0xFF per K/V plane of a gathered request with
torch.bincount (src/unchain_kv/vllm_connector.py:2871-2904); the checks here are
exact counts of the gathered words (numpy), the fitted codebook against the fit
rule applied to those counts, and, at the Llama-3-8B layer size, torch.bincount on
the GPU.
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


def bincount_planes(kv_host, tables):
    ids = [b for t in tables for b in t]
    out = []
    for plane in range(2):
        words = kv_host[plane, ids].reshape(-1)
        out.append(np.bincount((words >> 7) & 0xFF, minlength=256))
    return np.stack(out)


@pytest.mark.parametrize("bw,pool,tables,offset", [
    (2048, 40, [[3, 1, 7, 30], [0, 39], [12]], 0),          # chunk kernel
    (16384, 12, [[11, 2, 5, 0, 9]], 0),                      # chunk kernel, Llama-3-8B blocks
    (48, 200, [list(range(0, 200, 3)), [199, 1]], 0),        # generic kernel
    (2048, 24, [[5, 6, 5], [23]], 1),                        # misaligned layer, repeated block
    (1024, 64, [list(range(1, 64, 2)) + [0], [9, 4, 60]], 0),  # odd chunk count (36 blocks)
    (16384, 520, [list(range(519, 6, -1))], 0),              # many batches per wave (513 blocks)
])
def test_histogram_matches_bincount(sz, bw, pool, tables, offset):
    say("histogram", bw, pool, offset)
    rng = np.random.default_rng(bw + pool)
    # exponents from a wide, skewed distribution (many lanes share a bin)
    exps = np.clip(rng.normal(120, 6, 2 * pool * bw + offset), 0, 255).astype(np.uint16)
    words = (rng.integers(0, 2, exps.size).astype(np.uint16) << 15) | (exps << 7) | \
        rng.integers(0, 128, exps.size).astype(np.uint16)
    backing = torch.from_numpy(words.view(np.int16).copy()).cuda().view(torch.bfloat16)
    kv = backing[offset:].view(2, pool, bw)
    kv_host = words[offset:].reshape(2, pool, bw)
    batch = sz.PagedBatch(tables, bw, "cuda")
    if offset:
        # a misaligned layer is not contiguous-aligned for the chunk kernel; it is
        # still a contiguous tensor, so the call is accepted and takes the generic path
        assert kv.data_ptr() % 16 != 0
    counts = sz.exponent_histogram_paged(kv, batch)
    torch.cuda.synchronize()
    assert counts is not None
    assert np.array_equal(counts.cpu().numpy(), bincount_planes(kv_host, tables))


def test_fit_on_gpu_histogram_follows_the_rule(sz):
    from unchainkv_amd import workloads

    say("fit llama3-8b layer")
    shape = workloads.LLAMA3_8B
    kv = workloads.make_kv_layer(torch, shape, 4096, seed=1, layer=2, device="cuda")
    tables = workloads.random_block_tables(torch, 4096, [256] * 8, seed=1)
    batch = sz.PagedBatch(tables, shape.block_words, "cuda")
    counts = sz.exponent_histogram_paged(kv, batch)
    # torch.bincount per plane over the gathered blocks, as the reference's trace does
    ids = torch.tensor([b for t in tables for b in t], device="cuda")
    for plane in range(2):
        words = kv[plane].index_select(0, ids).reshape(-1).view(torch.int16).to(torch.int32)
        ref = torch.bincount(torch.bitwise_and(torch.bitwise_right_shift(words, 7), 0xFF),
                             minlength=256)
        assert torch.equal(counts[plane], ref)
    book = sz.fit_top16_codebook_paged(kv, batch)
    k, v = counts.cpu().tolist()
    assert book == bytes(oracle.fit_top16_py(k) + oracle.fit_top16_py(v))
    assert book == workloads.fit_codebook(torch, kv, tables)


def test_fit_declines_with_fewer_than_16_exponents(sz):
    say("fit declines")
    bw, pool = 2048, 8
    words = np.full(2 * pool * bw, 0x3F80, dtype=np.uint16)  # one exponent only
    kv = torch.from_numpy(words.view(np.int16)).cuda().view(torch.bfloat16).view(2, pool, bw)
    batch = sz.PagedBatch([[0, 1, 2]], bw, "cuda")
    counts = sz.exponent_histogram_paged(kv, batch)
    assert int(counts[0, 0x7F]) == 3 * bw and int(counts.sum()) == 6 * bw
    assert sz.fit_top16_codebook_paged(kv, batch) is None
